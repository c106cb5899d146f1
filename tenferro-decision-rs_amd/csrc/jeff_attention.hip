// Jeff (Qwen3.5) full attention on gfx950 matrix cores.
//
// Arithmetic follows cpu-kernels jeff_full_attention_into
// (crates/cpu-kernels/src/lib.rs:609-763): per head, centered RMSNorm of q and
// k with x * (scale * (1 + w)) (676-691), partial RoPE on channel pairs
// (i, i + rot/2) with angle t * theta^(-2i/rot) (692-709, table built on the
// host with the same f32 libm calls), keys with key > query or mask == 0 are
// dropped (716), s = (q.k)/sqrt(hd), softmax, o = sum p*v skipping p == 0 and
// o = 0 when nothing is kept (731-754), out = o * 1/(1 + exp(-gate)) (755-758).
//
// Layout: every (L, W) tensor is token-contiguous (element t + L*f), so a
// wavefront's 32 queries or a tile's 32 keys are one 128-byte run per
// feature.
//
// One workgroup = 4 wavefronts sharing one kv head. With G = heads/kv_heads
// query heads per kv head, a workgroup holds hg = gcd(G, 4) heads x (4/hg)
// query sub-tiles of 16, so each K/V tile staged in LDS is used by every
// query head of the group (native GQA). K is RMS-normalized and rotated while
// it is staged; Q is normalized and rotated once per wave into registers.
// Key tiles outside [first active key, last query] are never visited.
//
// Each wavefront owns 16 queries and walks 32-key tiles on the 16x16x4 f32
// MFMA: S^T = K Q^T as two 16-key blocks, then O^T += V^T P^T. At hd = 256
// this keeps Q (hd/4 registers) and O^T (hd/4) within one wave's registers.
#include <type_traits>

#include "jeff_common.hpp"
#include "tfd_device.hpp"
#include "tfd_internal.hpp"

namespace tfd {

// Scans one row's key mask: first and last active key (mask != 0).
__device__ __forceinline__ void scan_active(const float *maskr, int L, int tid, int lane,
                                            int *s_span) {
  int lo = 0x7fffffff, hi = -1;
  for (int k0 = 0; k0 < L; k0 += 256 * 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {  // 8 loads in flight per thread
      const int k = k0 + tid + 256 * u;
      const float x = maskr[min(k, L - 1)];
      v[u] = k < L ? x : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int k = k0 + tid + 256 * u;
      if (v[u] != 0.0f) {
        lo = min(lo, k);
        hi = max(hi, k);
      }
    }
  }
  lo = wave_min(lo);
  hi = wave_max(hi);
  if (lane == 0) {
    atomicMin(&s_span[0], lo);
    atomicMax(&s_span[1], hi);
  }
}

// First active key of a row (rows with no active key: 0), for TFD_TRIM_LEADING.
__device__ __forceinline__ int row_start(const JeffArgs &a, const float *maskr, int tid, int lane,
                                         int *s_span) {
  if (!a.trim) return 0;
  if (tid == 0) {
    s_span[0] = 0x7fffffff;
    s_span[1] = -1;
  }
  __syncthreads();
  scan_active(maskr, a.L, tid, lane, s_span);
  __syncthreads();
  return s_span[1] >= 0 ? s_span[0] : 0;
}

// ---------------------------------------------------------------- K prep

// First active key of a row (mask != 0; 0 for a row with none), computed by
// one wave on its own.
__device__ __forceinline__ int wave_first_active(const float *maskr, int L, int lane) {
  int lo = 0x7fffffff;
  for (int k0 = 0; k0 < L; k0 += 64 * 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = maskr[min(k0 + lane + 64 * u, L - 1)];
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (k0 + lane + 64 * u < L && v[u] != 0.0f) lo = min(lo, k0 + lane + 64 * u);
  }
  lo = wave_min(lo);
  return __builtin_amdgcn_readfirstlane(lo == 0x7fffffff ? 0 : lo);
}

// Row span of the mask, computed by one wave on its own (no barrier): first
// and last active key (mask != 0), or (0, -1) for a row with none.
__device__ __forceinline__ void wave_active_span(const float *maskr, int L, int lane, int &first,
                                                 int &last) {
  int lo = 0x7fffffff, hi = -1;
  for (int k0 = 0; k0 < L; k0 += 64 * 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = maskr[min(k0 + lane + 64 * u, L - 1)];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int k = k0 + lane + 64 * u;
      if (k < L && v[u] != 0.0f) {
        lo = min(lo, k);
        hi = max(hi, k);
      }
    }
  }
  lo = wave_min(lo);
  hi = wave_max(hi);
  first = __builtin_amdgcn_readfirstlane(hi >= 0 ? lo : 0);
  last = __builtin_amdgcn_readfirstlane(hi);
}

// Split layout (f32, HDP = 256, for the split-head kernel): each (row, kv
// head) holds Lp = L rounded up to 16 keys, as blocks of 16 keys x 64
// features (tile kt, wave slice w) of 4 KB, each four 1 KB runs c: run c,
// 16-byte chunk 16g + col is key 16kt + col, features 64w + 16c + 4g .. + 3.
// A wave's load of run c is then one contiguous 1 KB read. Keys L .. Lp - 1
// hold zeros.
__device__ __forceinline__ size_t split_kp_offset(int key, int d) {
  const int kt = key >> 4, col = key & 15;
  const int w = d >> 6, c = (d >> 4) & 3, g = (d >> 2) & 3, e = d & 3;
  return ((size_t)(kt * 4 + w) * 4 + c) * 256 + (g * 16 + col) * 4 + e;
}

// One wavefront: the row's active keys (mask != 0) as one bit per key (zero
// past L, 32 keys per word) and its (first, last) span, (0, -1) for a row
// with none, for the attention kernels' scalar loads.
__device__ void write_row_bits_span(const float *__restrict__ maskr, int L, int lane, int row,
                                    int *__restrict__ spans, uint32_t *__restrict__ kbits) {
  uint32_t *bits = kbits + (size_t)row * ((L + 31) / 32);
  int lo = 0x7fffffff, hi = -1;
  for (int b0 = 0; b0 < L; b0 += 64 * 8) {
    float mv[8];
#pragma unroll
    for (int v = 0; v < 8; ++v) mv[v] = maskr[min(b0 + 64 * v + lane, L - 1)];
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      const int kb = b0 + 64 * v;
      const uint64_t bm = __ballot(kb + lane < L && mv[v] != 0.0f);
      if (lane == 0 && kb < L) {
        bits[kb / 32] = (uint32_t)bm;
        if (kb + 32 < L) bits[kb / 32 + 1] = (uint32_t)(bm >> 32);
      }
      if (bm != 0) {
        lo = min(lo, kb + (int)__builtin_ctzll(bm));
        hi = max(hi, kb + 63 - (int)__builtin_clzll(bm));
      }
    }
  }
  if (lane == 0) {
    spans[2 * row] = hi >= 0 ? lo : 0;
    spans[2 * row + 1] = hi;
  }
}

// RMSNorm (lib.rs:676-691) and partial RoPE (692-709) of every key of one
// (row, kv head) once per call, so attention workgroups stage finished keys.
// One workgroup = 32 keys; output kp[row][kvh][key][HDP] (zero-padded past
// hd), written in whole 16-byte chunks. Out: f32, or for the bf16 attention
// kernels fp16 (RNE) of the key times 2^-e, e = norm_weight_exp(k_norm): the
// Q.K^T product of those kernels takes fp16 operands. Every global load
// (keys, norm weights, RoPE table)
// is issued before the first is used. With kbits set, the workgroups of kv
// head 0 also write their 32 keys' active bits (mask != 0), one word each.

template <int HDP, typename OutT>
__global__ __launch_bounds__(256) void jeff_k_prep_kernel(const JeffArgs a, OutT *__restrict__ kp,
                                                          uint32_t *__restrict__ kbits) {
  constexpr int DP = HDP / 8;  // dims per thread: 8 threads per key
  // LDS rows of the tile: feature d of key k at kx(k, d), one pad word after
  // every 32 features, so that the output loop's lanes (8 consecutive
  // features each, 32 lanes along one key) hit 32 different banks (with
  // rows of HDP + 1 they shared 4 of them).
  constexpr int KS = HDP + HDP / 32 + 1;
  auto kx = [](int k, int d) { return k * KS + d + (d >> 5); };
  constexpr int RT = (HDP / 2 + 7) / 8;  // RoPE pairs per thread, at most
  __shared__ float Kt[kKeyTile * KS];
  __shared__ float s_red[8 * kKeyTile];
  const int tid = threadIdx.x, lane = tid & 63;
  const int row = blockIdx.z, kvh = blockIdx.y;
  const int L = a.L, hd = a.hd, rh = a.rot_half;
  // Key blocks 2m and 2m + 1 go to workgroups i and i + 8 of each 16, which
  // the dispatcher sends to one XCD: in bf16 the two blocks are the two
  // halves of every 128-byte run of a feature's keys, so the second half's
  // loads find the run in that XCD's L2 (C5 prep 16.1 -> 15.1 us).
  int kb = (int)blockIdx.x;
  if ((gridDim.x & 15) == 0) {
    const int g = kb >> 4, r = kb & 15;
    kb = 16 * g + 2 * (r & 7) + (r >> 3);
  }
  const int k0 = kb * kKeyTile;
  const bool bf = sizeof(OutT) == 2;
  const size_t kv_off = row * a.kv_row + (size_t)kvh * a.kv_head;
  const int kk = tid & 31, part = tid >> 5;
  const int key = k0 + kk;
  const bool kin = key < L;
  const bool rope = a.cos_t != nullptr && rh > 0;
  const int start = a.trim ? wave_first_active(a.mask + (size_t)row * L, L, lane) : 0;
  if (kbits != nullptr && kvh == 0 && tid < 64) {
    const float mv = a.mask[(size_t)row * L + min(k0 + lane, L - 1)];
    const uint64_t bm = __ballot(lane < kKeyTile && k0 + lane < L && mv != 0.0f);
    if (lane == 0) kbits[(size_t)row * ((L + 31) / 32) + kb] = (uint32_t)bm;
  }
  float xs[DP], wn[DP], c[RT], sn[RT];
#pragma unroll
  for (int i = 0; i < DP; ++i) {
    const int d = part * DP + i;
    const int dc = d < hd ? d : hd - 1;
    const size_t at = kv_off + (kin ? key : 0) + (size_t)L * dc;
    xs[i] = bf ? __uint_as_float((uint32_t)static_cast<const uint16_t *>(a.k)[at] << 16)
               : static_cast<const float *>(a.k)[at];
  }
  // Norm weights: 16 bytes per load when the thread's run is whole and aligned.
  if (DP % 4 == 0 && part * DP + DP <= hd && (reinterpret_cast<uintptr_t>(a.k_norm) & 15) == 0) {
#pragma unroll
    for (int i = 0; i < DP; i += 4) {
      const f32x4 w4 = *reinterpret_cast<const f32x4 *>(a.k_norm + part * DP + i);
#pragma unroll
      for (int t = 0; t < 4; ++t) wn[i + t] = w4[t];
    }
  } else {
#pragma unroll
    for (int i = 0; i < DP; ++i) wn[i] = a.k_norm[min(part * DP + i, hd - 1)];
  }
  // Thread (kk, part) rotates pairs i = part, part + 8, ... of key k0 + kk.
  const size_t pos = (size_t)min(max(key - start, 0), L - 1) * rh;
  if (rope) {
#pragma unroll
    for (int u = 0; u < RT; ++u) {
      // Only the pairs below rot/2 are rotated (8u < rh: uniform).
      if (8 * u < rh) {
        const int i = min(part + 8 * u, rh - 1);
        c[u] = a.cos_t[pos + i];
        sn[u] = a.sin_t[pos + i];
      }
    }
  }
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < DP; ++i) {
    const int d = part * DP + i;
    xs[i] = (kin && d < hd) ? xs[i] : 0.0f;
    ss += xs[i] * xs[i];
  }
  s_red[part * kKeyTile + kk] = ss;
  __syncthreads();
  {
    float tot = 0.0f;
#pragma unroll
    for (int p = 0; p < 8; ++p) tot += s_red[p * kKeyTile + kk];
    const float scale = rms_scale(tot, hd, a.eps);
#pragma unroll
    for (int i = 0; i < DP; ++i) {
      const int d = part * DP + i;
      Kt[kx(kk, d)] = (kin && d < hd) ? rms_apply(xs[i], scale, wn[i]) : 0.0f;
    }
  }
  if (rope) {
    __syncthreads();
#pragma unroll
    for (int u = 0; u < RT; ++u) {
      const int i = part + 8 * u;
      if (i < rh && kin) {
        const float x = Kt[kx(kk, i)], y = Kt[kx(kk, i + rh)];
        Kt[kx(kk, i)] = rope_lo(x, y, c[u], sn[u]);
        Kt[kx(kk, i + rh)] = rope_hi(x, y, c[u], sn[u]);
      }
    }
  }
  __syncthreads();
  OutT *dst = kp + (((size_t)row * a.kv_heads + kvh) * L + k0) * HDP;
  const int nkeys = min(kKeyTile, L - k0);
  const float ksig = bf ? ldexpf(1.0f, -norm_weight_exp(a.k_norm, hd, lane)) : 1.0f;
  constexpr int CH = 16 / (int)sizeof(OutT);  // elements per 16-byte chunk
  for (int e = tid; e < nkeys * (HDP / CH); e += 256) {
    const int k2 = e / (HDP / CH), d0 = (e % (HDP / CH)) * CH;
    const float *src = &Kt[kx(k2, d0)];  // d0 .. d0 + CH - 1 share one 32-feature run
    if constexpr (sizeof(OutT) == 2) {
      u16x8 o;
#pragma unroll
      for (int t = 0; t < 8; ++t) o[t] = f32_to_f16_bits(src[t] * ksig);
      *reinterpret_cast<u16x8 *>(dst + (size_t)k2 * HDP + d0) = o;
    } else {
      const f32x4 o = {src[0], src[1], src[2], src[3]};
      *reinterpret_cast<f32x4 *>(dst + (size_t)k2 * HDP + d0) = o;
    }
  }
}

// K prep for the split-head kernel (f32, HDP = 256): one workgroup = 32 keys
// (two 16-key tiles) of one (row, kv head), written in the split layout
// above. K arrives along keys as whole 128-byte rows (feature d, keys
// k0 .. k0 + 31: eight 16-byte loads per feature, eight per thread) and is
// transposed through LDS; thread (key tid & 31, part tid >> 5) then owns
// features 32 part .. + 31 of its key: RMSNorm (lib.rs:676-691) with the
// sum of squares reduced over the eight parts (lane swap, then LDS),
// partial RoPE (692-709) in registers when the partner feature i + rot/2
// sits in the same wave (rot/2 = 32: part p pairs with part p + 1, lane
// + 32), else through LDS. Workgroups with blockIdx.x == 0 and kv head 0
// also write the row's active-key bits and key span.
__global__ __launch_bounds__(256) void jeff_k_prep_split_kernel(const JeffArgs a,
                                                                float *__restrict__ kp,
                                                                int *__restrict__ spans,
                                                                uint32_t *__restrict__ kbits) {
  constexpr int HDP = 256, KB = 32, KS = HDP + 4;
  __shared__ __attribute__((aligned(16))) float Kt[KB * KS];
  __shared__ float s_red[4 * KB];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int row = blockIdx.z, kvh = blockIdx.y;
  const int L = a.L, hd = a.hd, rh = a.rot_half;
  const int k0 = blockIdx.x * KB;
  const float *maskr = a.mask + (size_t)row * L;
  const float *K = static_cast<const float *>(a.k) + row * a.kv_row + (size_t)kvh * a.kv_head;

  // A block with no active key is never read: the attention kernel walks
  // only from the row's first active key on, and inside that range it skips
  // (or masks whole) tiles without active keys. Such blocks leave their
  // workspace untouched, except the one that also writes the row's bits.
  if (!(blockIdx.x == 0 && kvh == 0)) {
    const int kl = min(k0 + (lane & 31), L - 1);
    const bool act = k0 + (lane & 31) < L && maskr[kl] != 0.0f;
    if (__ballot(act) == 0) return;  // the same in every wave
  }

  // Raw block along keys: task (feature d, keys k0 + 4 g8 .. + 3), L % 4 == 0;
  // features past hd and keys past L read as 0 (keys past L of this feature
  // are the next feature's and are zeroed below).
  const __amdgpu_buffer_rsrc_t rk = buffer_rsrc(K, (uint32_t)((size_t)hd * L * 4));
  f32x4 x[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const int e = tid + 256 * t, d = e >> 3, g8 = e & 7;
    x[t] = buffer_load4(rk, (d * L + 4 * g8) * 4, k0 * 4);
  }
  const int kk = tid & 31, part = tid >> 5;  // this thread's key and 32-feature part
  const int key = k0 + kk;
  const bool kin = key < L;
  const __amdgpu_buffer_rsrc_t rn = buffer_rsrc(a.k_norm, (uint32_t)(hd * 4));
  f32x4 wn[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) wn[c] = buffer_load4(rn, (32 * part + 4 * c) * 4, 0);
  const bool rope = a.cos_t != nullptr && rh > 0;
  const int start = a.trim ? wave_first_active(maskr, L, lane) : 0;
  const size_t pos = (size_t)min(max(key - start, 0), L - 1) * rh;
  f32x4 tc[8], ts[8];  // rot/2 == 32, parts 0 and 1 (wave 0): pairs i = 4c + e of its key
  if (rope && rh == 32 && part < 2) {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      tc[c] = *reinterpret_cast<const f32x4 *>(a.cos_t + pos + 4 * c);
      ts[c] = *reinterpret_cast<const f32x4 *>(a.sin_t + pos + 4 * c);
    }
  }

  if (blockIdx.x == 0 && kvh == 0 && wave == 0) write_row_bits_span(maskr, L, lane, row, spans, kbits);

#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const int e = tid + 256 * t, d = e >> 3, g8 = e & 7;
#pragma unroll
    for (int i = 0; i < 4; ++i) Kt[(4 * g8 + i) * KS + d] = x[t][i];
  }
  __syncthreads();
  float kv[32];
  float ss = 0.0f;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const f32x4 y = *reinterpret_cast<const f32x4 *>(&Kt[kk * KS + 32 * part + 4 * c]);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      kv[4 * c + e] = kin ? y[e] : 0.0f;
      ss += kv[4 * c + e] * kv[4 * c + e];
    }
  }
  ss = pair_sum(ss);  // the wave's two parts of this key
  if (lane < 32) s_red[wave * KB + lane] = ss;
  __syncthreads();
  const float tot = s_red[kk] + s_red[KB + kk] + s_red[2 * KB + kk] + s_red[3 * KB + kk];
  const float scale = rms_scale(tot, hd, a.eps);
#pragma unroll
  for (int c = 0; c < 8; ++c)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int d = 32 * part + 4 * c + e;
      kv[4 * c + e] = (kin && d < hd) ? rms_apply(kv[4 * c + e], scale, wn[c][e]) : 0.0f;
    }
  if (rope && rh == 32) {
    // Part 0 (lanes 0..31 of wave 0) holds pairs i = j, part 1 (lanes
    // 32..63 of the same wave) their partners i + 32.
    if (wave == 0) {
#pragma unroll
      for (int j = 0; j < 32; ++j) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(kv[j]),
                                                        __float_as_uint(kv[j]), false, false);
        const float other = __uint_as_float(lane < 32 ? r[1] : r[0]);
        const float xl = part == 0 ? kv[j] : other, yh = part == 0 ? other : kv[j];
        const float cc = tc[j >> 2][j & 3], sn = ts[j >> 2][j & 3];
        if (kin) kv[j] = part == 0 ? rope_lo(xl, yh, cc, sn) : rope_hi(xl, yh, cc, sn);
      }
    }
  } else if (rope) {
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 32; ++j) Kt[kk * KS + 32 * part + j] = kv[j];
    __syncthreads();
    if (kin) {
      for (int i = part; i < rh; i += 8) {
        const float xl = Kt[kk * KS + i], yh = Kt[kk * KS + i + rh];
        const float cc = a.cos_t[pos + i], sn = a.sin_t[pos + i];
        Kt[kk * KS + i] = rope_lo(xl, yh, cc, sn);
        Kt[kk * KS + i + rh] = rope_hi(xl, yh, cc, sn);
      }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 32; ++j) kv[j] = Kt[kk * KS + 32 * part + j];
  }
  const int Lp = (L + 15) & ~15;
  if (key < Lp) {
    float *unit = kp + ((size_t)row * a.kv_heads + kvh) * (size_t)Lp * HDP;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const f32x4 o = {kv[4 * c], kv[4 * c + 1], kv[4 * c + 2], kv[4 * c + 3]};
      *reinterpret_cast<f32x4 *>(unit + split_kp_offset(key, 32 * part + 4 * c)) = o;
    }
  }
}

// ----------------------------------------------------------- f32 attention

// RMSNorm + partial RoPE of one wave's 16 queries of one head into the
// B-operand registers of S^T = K Q^T: lane (col, grp) ends with
// Qn[q0 + col][grp*QS + s]. Goes through the wave's own LDS rows qw
// (16 x (HDP + 4) floats): raw rows (16-byte loads along tokens when VEC),
// normalized in registers, rotated pairs in LDS, read back. Queries that are
// past L or dropped (q < start) get zeros.
template <int HDP, bool VEC>
__device__ __forceinline__ void jeff_q_prep(const JeffArgs &a, const float *Q, int q0, int start,
                                            float *qw, float (&qreg)[HDP / 4]) {
  constexpr int QS = HDP / 4, QP = HDP + 4;
  const int lane = threadIdx.x & 63, col = lane & 15, grp = lane >> 4;
  const int L = a.L, hd = a.hd, rh = a.rot_half;
  const int q = q0 + col;
  const bool q_live = q < L && q >= start;
  // Issued first, so that they share the Q loads' round trip: this lane's
  // norm weights (past hd they read 0 or anything; those dims are zeroed
  // below) and the table entries of its first 8 RoPE pairs i = grp + 4u.
  const __amdgpu_buffer_rsrc_t rn = buffer_rsrc(a.q_norm, (uint32_t)(hd * 4));
  f32x4 wv[QS / 4];
#pragma unroll
  for (int c = 0; c < QS / 4; ++c) wv[c] = buffer_load4(rn, (grp * QS + 4 * c) * 4, 0);
  const bool rope = a.cos_t != nullptr && rh > 0;
  const size_t pos = (size_t)min(max(q - start, 0), L - 1) * rh;
  float c8[8], s8[8];
  if (rope) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = min(grp + 4 * u, rh - 1);
      c8[u] = a.cos_t[pos + i];
      s8[u] = a.sin_t[pos + i];
    }
  }
  if constexpr (VEC) {
    // Task (d, g): queries q0 + 4g .. +3 of feature d, one 16-byte load;
    // features past hd read as 0.
    const __amdgpu_buffer_rsrc_t rq = buffer_rsrc(Q, (uint32_t)((size_t)hd * L * 4));
#pragma unroll
    for (int i0 = 0; i0 < HDP * 4; i0 += 64 * 4) {
      f32x4 x[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {  // HDP * 4 < 256 only at HDP = 32: clamp, skip below
        const int e = min(i0 + lane + 64 * u, HDP * 4 - 1), d = e >> 2, g = e & 3;
        x[u] = buffer_load4(rq, (int)(((size_t)d * L + 4 * g) * 4), q0 * 4);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int e = i0 + lane + 64 * u, d = e >> 2, g = e & 3;
        if (HDP * 4 % 256 == 0 || e < HDP * 4) {
#pragma unroll
          for (int t = 0; t < 4; ++t) qw[(4 * g + t) * QP + d] = x[u][t];
        }
      }
    }
  } else {
    for (int e0 = 0; e0 < 16 * HDP; e0 += 64 * 8) {
      float x[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int e = e0 + lane + 64 * u, d = e >> 4, t = e & 15;
        x[u] = Q[min(q0 + t, L - 1) + (size_t)L * min(d, hd - 1)];
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int e = e0 + lane + 64 * u, d = e >> 4, t = e & 15;
        qw[t * QP + d] = d < hd ? x[u] : 0.0f;
      }
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float *qs = qw + col * QP + grp * QS;
  f32x4 xv[QS / 4];
  float ss = 0.0f;
#pragma unroll
  for (int c = 0; c < QS / 4; ++c) {
    xv[c] = *reinterpret_cast<const f32x4 *>(qs + 4 * c);
    ss += xv[c][0] * xv[c][0] + xv[c][1] * xv[c][1] + xv[c][2] * xv[c][2] + xv[c][3] * xv[c][3];
  }
  ss += __shfl_xor(ss, 16);
  ss += pair_sum(ss) - ss;  // lanes l and l ^ 32 hold the other two groups
  const float scale = rms_scale(ss, hd, a.eps);
#pragma unroll
  for (int c = 0; c < QS / 4; ++c) {
    f32x4 y;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int d = grp * QS + 4 * c + t;
      y[t] = (q_live && d < hd) ? rms_apply(xv[c][t], scale, wv[c][t]) : 0.0f;
    }
    *reinterpret_cast<f32x4 *>(qs + 4 * c) = y;
  }
  if (rope) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // Lane (col, grp) rotates pairs i = grp, grp + 4, ... of query q0 + col;
    // the first 8 with the entries loaded up front.
    if (q_live) {
      float *qr = qw + col * QP;
      for (int i0 = grp; i0 < rh; i0 += 4 * 8) {
        float c[8], sn[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int i = min(i0 + 4 * u, rh - 1);
          c[u] = i0 == grp ? c8[u] : a.cos_t[pos + i];
          sn[u] = i0 == grp ? s8[u] : a.sin_t[pos + i];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int i = i0 + 4 * u;
          if (i < rh) {
            const float x = qr[i], y = qr[i + rh];
            qr[i] = rope_lo(x, y, c[u], sn[u]);
            qr[i + rh] = rope_hi(x, y, c[u], sn[u]);
          }
        }
      }
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
  for (int c = 0; c < QS / 4; ++c) {
    const f32x4 y = *reinterpret_cast<const f32x4 *>(qs + 4 * c);
#pragma unroll
    for (int t = 0; t < 4; ++t) qreg[4 * c + t] = y[t];
  }
}

// o = O^T * inv (0 when nothing was kept), times the sigmoid gate, stored
// feature-major: the wave writes its 16 x HDP block through its LDS rows ow
// (16 x (HDP + 4) floats) so that gate loads and output stores run along
// tokens, 16 bytes at a time, when VEC. Dropped queries (q < start) get 0.
// Only features d_lo <= d < d_hi are stored (a workgroup that owns part of
// the head's features).
template <int HDP, bool VEC>
__device__ __forceinline__ void jeff_store(const JeffArgs &a, const float *Gt, float *OUT, int q0,
                                           int start, float *ow, const f32x4 (&O)[HDP / 16],
                                           float inv, int d_lo = 0, int d_hi = 1 << 30) {
  constexpr int NB = HDP / 16, QP = HDP + 4;
  const int lane = threadIdx.x & 63, col = lane & 15, grp = lane >> 4;
  const int L = a.L, hd = a.hd;
  if constexpr (VEC) {
    // The gate loads go out before O is written to LDS.
    const __amdgpu_buffer_rsrc_t rg = buffer_rsrc(Gt, (uint32_t)((size_t)hd * L * 4));
    const __amdgpu_buffer_rsrc_t ro = buffer_rsrc(OUT, (uint32_t)((size_t)hd * L * 4));
    constexpr int NG = (HDP * 4 + 63) / 64;
    f32x4 g[NG];
#pragma unroll
    for (int u = 0; u < NG; ++u) {  // clamped as in the Q prep
      const int e = min(lane + 64 * u, HDP * 4 - 1), d = e >> 2, gq = e & 3;
      g[u] = buffer_load4(rg, (int)(((size_t)d * L + 4 * gq) * 4), q0 * 4);
    }
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const f32x4 v = O[j] * inv;  // dims 16j + 4grp + 0..3 of query q0 + col
      *reinterpret_cast<f32x4 *>(ow + col * QP + 16 * j + 4 * grp) = v;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    {
      const int i0 = 0;
#pragma unroll
      for (int u = 0; u < NG; ++u) {
        const int e = min(i0 + lane + 64 * u, HDP * 4 - 1), d = e >> 2, gq = e & 3;
        const int qa = q0 + 4 * gq;  // L % 4 == 0: the 4 queries are all in or all out
        f32x4 o;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float x = ow[(4 * gq + t) * QP + d] * fast_sigmoid(g[u][t]);
          o[t] = qa + t < start ? 0.0f : x;
        }
        if (qa < L && d < hd && d >= d_lo && d < d_hi)
          buffer_store4_nt(o, ro, (int)(((size_t)d * L + 4 * gq) * 4), q0 * 4);
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const f32x4 v = O[j] * inv;  // dims 16j + 4grp + 0..3 of query q0 + col
      *reinterpret_cast<f32x4 *>(ow + col * QP + 16 * j + 4 * grp) = v;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    for (int e0 = 0; e0 < 16 * HDP; e0 += 64 * 8) {
      float g[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int e = e0 + lane + 64 * u, d = e >> 4, t = e & 15;
        g[u] = Gt[min(q0 + t, L - 1) + (size_t)L * min(d, hd - 1)];
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int e = e0 + lane + 64 * u, d = e >> 4, t = e & 15;
        const int qq = q0 + t;
        if (qq < L && d < hd && d >= d_lo && d < d_hi)
          __builtin_nontemporal_store(qq < start ? 0.0f : ow[t * QP + d] * fast_sigmoid(g[u]),
                                      &OUT[qq + (size_t)L * d]);
      }
    }
  }
}

// Tile data for one 16-key tile, prefetched into registers: finished K rows
// from the prep workspace and V columns, all 16-byte buffer loads with a
// fixed per-lane offset and a scalar tile offset (VEC), or element loads
// with clamped indices. Keys past L read as 0 (K) or are zeroed at commit
// (V). LDS holds K as [key][d] and V as [d][key], V's layout in memory.
template <int HDP, bool VEC, int NT>
struct JeffStage {
  static constexpr int KT = kJeffKeyTile;
  static constexpr int TASKS = KT * HDP / 4;       // 16-byte chunks of K (and of V)
  static constexpr int KN = (TASKS + NT - 1) / NT;  // chunks per thread (NT threads)
  f32x4 k[KN], v[KN];
  __amdgpu_buffer_rsrc_t rk, rv;
  int ok[KN], ov[KN];

  __device__ __forceinline__ void init(const float *KP, const float *V, int L, int hd, int tid) {
    rk = buffer_rsrc(KP, (uint32_t)((size_t)L * HDP * 4));
    rv = buffer_rsrc(V, (uint32_t)((size_t)hd * L * 4));
#pragma unroll
    for (int i = 0; i < KN; ++i) {
      const int e = min(tid + NT * i, TASKS - 1);
      ok[i] = e * 16;                                  // chunk e of the KT x HDP tile
      const int d = e / (KT / 4), g = e % (KT / 4);    // feature d, keys 4g .. 4g+3
      ov[i] = (int)(((size_t)d * L + 4 * g) * 4);
    }
  }

  __device__ __forceinline__ void fetch(const float *KP, const float *V, int L, int hd, int k0,
                                        int tid) {
    if constexpr (VEC) {
#pragma unroll
      for (int i = 0; i < KN; ++i) {
        k[i] = buffer_load4(rk, ok[i], k0 * HDP * 4);
        v[i] = buffer_load4(rv, ov[i], k0 * 4);
      }
    } else {
#pragma unroll
      for (int i = 0; i < KN; ++i) {
        const int e = min(tid + NT * i, TASKS - 1);
        const int kk = min((4 * e) / HDP, L - 1 - k0);
        k[i] = reinterpret_cast<const f32x4 *>(KP + (size_t)k0 * HDP)[kk * (HDP / 4) + e % (HDP / 4)];
        const int d = min(e / (KT / 4), hd - 1), g = e % (KT / 4);
        const float *src = V + (size_t)L * d;
#pragma unroll
        for (int t = 0; t < 4; ++t) v[i][t] = src[min(k0 + 4 * g + t, L - 1)];
      }
    }
  }

  __device__ __forceinline__ void commit(float *Ks, float *Vs, int tid, int k0, int L, int hd) {
    constexpr int KS = HDP + 4, VS = KT + 4;
    const bool tail = k0 + KT > L;  // uniform: the row's last, partial tile
#pragma unroll
    for (int i = 0; i < KN; ++i) {
      const int e = tid + NT * i;
      if (TASKS % NT == 0 || e < TASKS) {  // blockDim is NT
        const int kk = (4 * e) / HDP, dk = (4 * e) % HDP;
        f32x4 kv = k[i];
        const int d = e / (KT / 4), g = e % (KT / 4);
        f32x4 vv = v[i];
        if (!VEC || tail) {
#pragma unroll
          for (int t = 0; t < 4; ++t) vv[t] = (d < hd && k0 + 4 * g + t < L) ? vv[t] : 0.0f;
          if (k0 + kk >= L) kv = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
        *reinterpret_cast<f32x4 *>(&Ks[kk * KS + dk]) = kv;
        *reinterpret_cast<f32x4 *>(&Vs[d * VS + 4 * g]) = vv;
      }
    }
  }
};

// TAG gives each calling kernel its own copy, compiled to that kernel's
// register budget; TAG 1 (the split-head kernel) reads the split K layout,
// TAG 2 (the fused kernel, no K prep) normalizes and rotates each key tile
// from K itself into LDS.
template <int HDP, bool VEC, int TAG = 0>
__device__ __noinline__ void jeff_redo_wave(const JeffArgs *ap, const float *__restrict__ kp,
                                            int row, int head, int q0, int kt_begin, int kt_end,
                                            int start, float *ws, int d_lo = 0,
                                            int d_hi = 1 << 30);

// The calling kernel's JeffArgs (its first parameter, at offset 0 of the
// kernel argument segment), for the out-of-line redo: passing the struct by
// value would make every wave copy it to scratch on entry.
__device__ __forceinline__ const JeffArgs *kernel_jeff_args() {
  return (const JeffArgs *)__builtin_amdgcn_kernarg_segment_ptr();
}

// One workgroup = 8 wavefronts (one workgroup per CU) sharing one kv head:
// hg = heads_per_group query heads x (8 / hg) query tiles of 16. The query
// tiles come in causal pairs (p, n - 1 - p), n = ceil(L / 16), so every
// workgroup carries about the same number of key tiles; the walk covers the
// group's span and a wave skips the tiles its own queries do not reach.
template <int HDP, bool VEC>
__global__ __launch_bounds__(kJeffF32Waves * 64, 1) void jeff_attention_f32_kernel(
    const JeffArgs a, const float *__restrict__ kp) {
  constexpr int NT = kJeffF32Waves * 64;
  constexpr int KT = kJeffKeyTile;  // 16 keys per tile
  constexpr int QS = HDP / 4;       // Q registers per lane (4 lane groups split hd)
  constexpr int NB = HDP / 16;      // 16-row blocks of O^T
  constexpr int KS = HDP + 4;       // K stored [key][d]
  constexpr int VS = KT + 4;        // V stored [d][key]: conflict-free 16-byte reads
  constexpr int KBUF = KT * KS, VBUF = HDP * VS;
  constexpr int QP = HDP + 4;       // per-wave Q / output rows before and after the walk
  constexpr int WROWS = kJeffF32Waves * kJeffWaveQueries * QP;
  constexpr int SMEM = WROWS > 2 * (KBUF + VBUF) ? WROWS : 2 * (KBUF + VBUF);
  __shared__ __attribute__((aligned(16))) float smem[SMEM];
  auto Ks = [&](int i) { return smem + i * KBUF; };
  auto Vs = [&](int i) { return smem + 2 * KBUF + i * VBUF; };

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform, in a scalar register
  const int col = lane & 15, grp = lane >> 4;
  const int hg = a.heads_per_group, S = kJeffF32Waves / hg;  // query tiles per workgroup
  // XCD-aware order: the dispatcher hands workgroup p to XCD p % 8, each XCD
  // with its own L2. Workgroups sharing one (row, kv head) -- its K/V -- are
  // given ids p = 8*i + c for one c, so they land on one XCD; consecutive
  // groups go to consecutive XCDs.
  int bx = blockIdx.x, by = blockIdx.y, bz = blockIdx.z;
  {
    const int nx = gridDim.x, ngroups = gridDim.y * gridDim.z;
    const int p = blockIdx.x + nx * (blockIdx.y + gridDim.y * blockIdx.z);
    if (ngroups % 8 == 0) {
      const int c = p % 8, i = p / 8;  // i-th workgroup of XCD c
      const int g = 8 * (i / nx) + c;  // (row, kv group) index
      bx = i % nx;
      by = g % gridDim.y;
      bz = g / gridDim.y;
    }
  }
  const int row = bz;
  const int head = by * hg + wave % hg;
  const int kvh = min(head / a.groups, a.kv_heads - 1);
  const int L = a.L, hd = a.hd;
  const int nq = (L + kJeffWaveQueries - 1) / kJeffWaveQueries;
  const int npairs = (nq + 1) / 2;
  const int s_idx = wave / hg, pair = bx * (S / 2) + s_idx / 2;
  const bool hi_member = s_idx & 1;
  const int qtile = hi_member ? nq - 1 - pair : pair;
  // a wave with no query tile (past the pairs, or the middle tile's twin)
  const bool wave_live = pair < npairs && (!hi_member || nq - 1 - pair != pair);
  const int q0 = qtile * kJeffWaveQueries;
  const int q = q0 + col;
  // the group's last query: the upper member of its lowest pair
  const int q_last = min((nq - bx * (S / 2)) * kJeffWaveQueries, L) - 1;
  const float *maskr = a.mask + (size_t)row * L;
  const float *Q = static_cast<const float *>(a.q) + row * a.q_row + (size_t)head * hd * L;
  const float *Gt = static_cast<const float *>(a.gate) + row * a.q_row + (size_t)head * hd * L;
  const float *V = static_cast<const float *>(a.v) + row * a.kv_row + (size_t)kvh * a.kv_head;
  const float *KP = kp + ((size_t)row * a.kv_heads + kvh) * L * HDP;
  float *OUT = a.out + row * a.q_row + (size_t)head * hd * L;
  float *qw = smem + wave * (kJeffWaveQueries * QP);

  // -------- active-key span (each wave on its own); RoPE positions restart
  // at `start` when trimming. Tiles past the group's last query are causal-
  // ly dead.
  int first, last;
  wave_active_span(maskr, L, lane, first, last);
  const int start = (a.trim && last >= 0) ? first : 0;
  int kt_begin = 0, kt_end = 0;
  {
    const int kl = min(last, q_last);
    if (last >= 0 && first <= kl) {
      kt_begin = first / KT;
      kt_end = kl / KT + 1;
    }
  }
  const bool q_live = wave_live && q < L && q >= start;

  // The first tile's loads go out before the Q prep and land during it.
  JeffStage<HDP, VEC, NT> st;
  st.init(KP, V, L, hd, tid);
  float m0 = 0.0f;
  if (kt_begin < kt_end) {
    m0 = maskr[min(kt_begin * KT + col, L - 1)];
    st.fetch(KP, V, L, hd, kt_begin * KT, tid);
  }
  float qreg[QS];
  jeff_q_prep<HDP, VEC>(a, Q, wave_live ? q0 : 0, start, qw, qreg);
  __syncthreads();  // the wave rows become the K/V buffers

  // Keep word for a 16-key tile: active key, key >= start, causal key <= query.
  // The mask value is fetched one tile ahead (mask_of) and turned into the
  // word (keep_word) only after that tile's barrier.
  auto mask_of = [&](int kt) -> float { return maskr[min(kt * KT + col, L - 1)]; };
  auto keep_word = [&](int kt, float mv) -> uint32_t {
    const int k0 = kt * KT;
    const int kc = k0 + col;
    const bool act = kc < L && kc >= start && mv != 0.0f;
    const uint32_t abits = (uint32_t)__ballot(act) & 0xffffu;
    return q_live ? (abits & range_bits(0, q - k0)) : 0u;
  };

  f32x4 O[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) O[j][r] = 0.0f;
  float m = kNoMax, l = 0.0f;
  const float c1 = a.c1;

  // -------- the walk (see the Laya kernel for the scheme): tile kt+1 is
  // fetched before the products of tile kt and committed after them; one
  // barrier per tile; lazily moved exponent reference; a wave whose kept
  // scores sum to NaN or inf stops computing, and it or a wave whose O took
  // a NaN or inf redoes its queries with the reference's exact semantics.
  uint32_t w = 0u;
  float m_next = 0.0f;
  if (kt_begin < kt_end) {
    st.commit(Ks(0), Vs(0), tid, kt_begin * KT, L, hd);
    w = keep_word(kt_begin, m0);
  }
  __syncthreads();
  bool tainted = false;  // wave-uniform
  int cur = 0;
  for (int kt = kt_begin; kt < kt_end; ++kt) {
    const bool more = kt + 1 < kt_end;
    if (more) {
      m_next = mask_of(kt + 1);
      st.fetch(KP, V, L, hd, (kt + 1) * KT, tid);
    }
    if (!tainted && __ballot(w != 0u) != 0) {
      const float *Kc = Ks(cur);
      f32x4 s0, s1;  // two partial sums over alternate chunks of hd
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        s0[r] = 0.0f;
        s1[r] = 0.0f;
      }
      const f32x4 *krow = reinterpret_cast<const f32x4 *>(&Kc[col * KS + grp * QS]);
#pragma unroll
      for (int c = 0; c < QS / 4; ++c) {
        const f32x4 ka = krow[c];
        if (c & 1) {
#pragma unroll
          for (int e = 0; e < 4; ++e) s1 = mfma_16x16x4(ka[e], qreg[4 * c + e], s1);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) s0 = mfma_16x16x4(ka[e], qreg[4 * c + e], s0);
        }
      }
      s0 += s1;
      // lane group g holds keys 4g + r of its query
      if (__ballot(q_live && w != 0xffffu) != 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r) s0[r] = ((w >> (4 * grp + r)) & 1u) ? s0[r] : -INFINITY;
      }
      float mx = fmaxf(fmaxf(s0[0], s0[1]), fmaxf(s0[2], s0[3]));
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = pair_max(mx);
      const float mxs = mx * c1;
      const bool need = mxs > m + kRescaleSlack;
      const float mn = need ? mxs : m;
      float rs = 0.0f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        s0[r] = fast_exp2(__builtin_fmaf(s0[r], c1, -mn));
        rs += s0[r];
      }
      if (__ballot(q_live && !__builtin_isfinite(rs)) != 0) {
        tainted = true;
      } else {
        if (__ballot(need) != 0) {
          const float alpha = fast_exp2(m - mn);  // exactly 1 where the reference stays
#pragma unroll
          for (int j = 0; j < NB; ++j) O[j] *= alpha;
          l *= alpha;
        }
        l += rs;
        m = mn;
        // A operand of block j: V[key 4*grp + r][d = 16*j + col], one 16-byte read.
        const float *v0 = &Vs(cur)[col * VS + 4 * grp];
#pragma unroll
        for (int j = 0; j < NB; ++j) {
          const f32x4 vv = *reinterpret_cast<const f32x4 *>(v0 + j * 16 * VS);
#pragma unroll
          for (int r = 0; r < 4; ++r) O[j] = mfma_16x16x4(vv[r], s0[r], O[j]);
        }
      }
    }
    if (more) st.commit(Ks(cur ^ 1), Vs(cur ^ 1), tid, (kt + 1) * KT, L, hd);
    __syncthreads();
    if (more) w = keep_word(kt + 1, m_next);
    cur ^= 1;
  }

  // -------- careful redo (rare), out of line; every wave's LDS reads of the
  // walk precede its last barrier, so each wave may now use its own rows.
  bool bad = false;
#pragma unroll
  for (int j = 0; j < NB; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) bad |= !__builtin_isfinite(O[j][r]);
  if (!wave_live) return;
  if (tainted || __ballot(q_live && bad) != 0) {
    jeff_redo_wave<HDP, VEC>(kernel_jeff_args(), kp, row, head, q0, kt_begin, kt_end, start, qw);
    return;
  }

  // -------- o / sum (0 when nothing was kept), sigmoid gate, store
  float lt = l + __shfl_xor(l, 16);
  lt = pair_sum(lt);
  const float inv = lt > 0.0f ? fast_rcp(lt) : 0.0f;
  jeff_store<HDP, VEC>(a, Gt, OUT, q0, start, qw, O, inv);
}

// The careful path for one wave's 16 queries of one head (rare: NaN or inf
// among its kept scores or values), from global memory without barriers:
// the reference's masked softmax with an exact running max (non-finite
// scores weigh 0, a +inf score empties the row) and o = sum p*v over
// p != 0 in key order (lib.rs:716-754), then the gate. Kept out of line so
// that its registers never weigh on the walk. ws: the wave's LDS rows.
template <int HDP, bool VEC, int TAG>
__device__ __noinline__ void jeff_redo_wave(const JeffArgs *ap, const float *__restrict__ kp,
                                            int row, int head, int q0, int kt_begin, int kt_end,
                                            int start, float *ws, int d_lo, int d_hi) {
  const JeffArgs &a = *ap;
  constexpr int KT = kJeffKeyTile, QS = HDP / 4, NB = HDP / 16, PS = KT + 1;
  const int lane = threadIdx.x & 63, col = lane & 15, grp = lane >> 4;
  const int L = a.L, hd = a.hd;
  const int kvh = min(head / a.groups, a.kv_heads - 1);
  const int q = q0 + col;
  const bool q_live = q < L && q >= start;
  const float *maskr = a.mask + (size_t)row * L;
  const float *Q = static_cast<const float *>(a.q) + row * a.q_row + (size_t)head * hd * L;
  const float *Gt = static_cast<const float *>(a.gate) + row * a.q_row + (size_t)head * hd * L;
  const float *V = static_cast<const float *>(a.v) + row * a.kv_row + (size_t)kvh * a.kv_head;
  constexpr bool SPLIT = TAG == 1;
  constexpr bool RAW = TAG == 2;  // keys straight from K, normalized per tile into LDS
  const size_t Lu = SPLIT ? (size_t)((L + 15) & ~15) : (size_t)L;
  const float *KP = RAW ? nullptr : kp + ((size_t)row * a.kv_heads + kvh) * Lu * HDP;
  const float *Kraw = static_cast<const float *>(a.k) + row * a.kv_row + (size_t)kvh * a.kv_head;
  constexpr int QP = HDP + 4;
  float *Kw = ws + 512;  // RAW: 16 keys x QP floats, after Pw
  float *OUT = a.out + row * a.q_row + (size_t)head * hd * L;
  float qreg[QS];
  jeff_q_prep<HDP, VEC>(a, Q, q0, start, ws, qreg);
  f32x4 O[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) O[j][r] = 0.0f;
  float m = kNoMax, l = 0.0f;
  float *Pw = ws;  // 16 keys x 17 floats, after the Q rows are consumed
#pragma unroll 1
  for (int kt = kt_begin; kt < kt_end; ++kt) {
    const int k0 = kt * KT;
    const int kc = k0 + col;
    const bool act = kc < L && kc >= start && maskr[min(kc, L - 1)] != 0.0f;
    const uint32_t abits = (uint32_t)__ballot(act) & 0xffffu;
    const uint32_t w = q_live ? (abits & range_bits(0, q - k0)) : 0u;
    if (__ballot(w != 0u) == 0) continue;
    const int kcl = min(kc, L - 1);
    if constexpr (RAW) {
      // The reference's key arithmetic (lib.rs:676-709) for keys k0 .. k0 +
      // 15: lane (col, grp) normalizes features grp*QS .. + QS - 1 of key
      // kcl, then rotates pairs i = grp, grp + 4, ... of it.
      float xk[QS];
      float ss = 0.0f;
#pragma unroll
      for (int x = 0; x < QS; ++x) {
        const int d = grp * QS + x;
        xk[x] = d < hd ? Kraw[kcl + (size_t)L * d] : 0.0f;
        ss += xk[x] * xk[x];
      }
      ss += __shfl_xor(ss, 16);
      ss += __shfl_xor(ss, 32);
      const float scale = rms_scale(ss, hd, a.eps);
#pragma unroll
      for (int x = 0; x < QS; ++x) {
        const int d = grp * QS + x;
        Kw[col * QP + d] = d < hd ? rms_apply(xk[x], scale, a.k_norm[d]) : 0.0f;
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      if (a.cos_t != nullptr && a.rot_half > 0) {
        const int rh = a.rot_half;
        const size_t pos = (size_t)min(max(kcl - start, 0), L - 1) * rh;
        for (int i = grp; i < rh; i += 4) {
          const float x = Kw[col * QP + i], y = Kw[col * QP + i + rh];
          Kw[col * QP + i] = rope_lo(x, y, a.cos_t[pos + i], a.sin_t[pos + i]);
          Kw[col * QP + i + rh] = rope_hi(x, y, a.cos_t[pos + i], a.sin_t[pos + i]);
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    const float *krow = RAW ? Kw + col * QP + grp * QS : KP + (size_t)kcl * HDP + grp * QS;
    f32x4 s;
#pragma unroll
    for (int r = 0; r < 4; ++r) s[r] = 0.0f;
#pragma unroll
    for (int x = 0; x < QS; ++x) {
      const float kx = SPLIT ? KP[split_kp_offset(kcl, grp * QS + x)] : krow[x];  // RAW: LDS
      s = mfma_16x16x4(kc < L ? kx : 0.0f, qreg[x], s);
    }
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float x = ((w >> (4 * grp + r)) & 1u) ? s[r] * a.c1 : -INFINITY;
      s[r] = x;
      mx = fmaxf(mx, x);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = pair_max(mx);
    const float mn = fmaxf(m, mx);
    const float alpha = (m == mn) ? 1.0f : fast_exp2(m - mn);
    float rs = 0.0f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float e = __builtin_isfinite(s[r]) ? fast_exp2(s[r] - mn) : 0.0f;
      s[r] = e;
      rs += e;
    }
    l = l * alpha + rs;
    m = mn;
    // alpha == 0: earlier probabilities are 0 against the new max, so their
    // (possibly infinite) values drop out as in the reference.
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) O[j][r] = alpha == 0.0f ? 0.0f : O[j][r] * alpha;
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int r = 0; r < 4; ++r) Pw[(4 * grp + r) * PS + col] = s[r];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll 1
    for (int kk = 0; kk < KT; ++kk) {
      const float pk = Pw[kk * PS + col];
      if (pk == 0.0f) continue;  // only kept keys inside the row get here
      const float *vcol = V + (k0 + kk);
#pragma unroll
      for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int d = 16 * j + 4 * grp + r;
          if (d < hd) O[j][r] += pk * vcol[(size_t)L * d];
        }
    }
    __builtin_amdgcn_wave_barrier();
  }
  float lt = l + __shfl_xor(l, 16);
  lt = pair_sum(lt);
  const float inv = lt > 0.0f ? fast_rcp(lt) : 0.0f;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  jeff_store<HDP, VEC>(a, Gt, OUT, q0, start, ws, O, inv, d_lo, d_hi);
}

// ------------------------------------------------- f32 attention, split head

// (row, head) of work unit u < rows * heads of the split-head and fused
// kernels, whose grids are (units, query tiles) and dispatch in the linear
// order u + units * y, workgroup id % 8 being the XCD: when the counts allow
// it, the 8 * G consecutive units of one XCD round are the G query heads of
// eight (row, kv head) pairs, so a pair's K/V tiles are read through one L2.
// The divisions go through FastDiv (operands below rows * heads, divisors
// at most heads; the launchers check rows * heads^2 <= 2^32).
__device__ __forceinline__ void jeff_unit_of(const JeffArgs &a, int rows, int u, int &row,
                                             int &head) {
  const int units = rows * a.heads, G = a.groups;
  if (units % 8 == 0 && (rows * a.kv_heads) % 8 == 0) {
    const int x = u % 8, i = u / 8;
    const int ig = (int)a.gdiv.div((uint32_t)i);
    const int kvu = x + 8 * ig;  // (row, kv head) unit of XCD x
    row = (int)a.kvdiv.div((uint32_t)kvu);
    head = (kvu - row * a.kv_heads) * G + (i - ig * G);
  } else {
    row = (int)a.hdiv.div((uint32_t)u);
    head = u - row * a.heads;
  }
}

// One workgroup = 4 wavefronts = one (row, head, 16-query tile). Wave w owns
// features [w*DS, (w+1)*DS) of the head (DS = HDP/4 = 64) in both products:
//   S^T_w (16 keys x 16 queries) = K[keys, slice w] Q[queries, slice w]^T  (16 MFMA 16x16x4)
//   S^T = sum over w of S^T_w, exchanged through LDS, one barrier per tile
//   O^T[slice w] += V[slice w]^T P^T                                       (16 MFMA 16x16x4)
// so a query tile's key walk runs on four SIMDs at once, and the longest
// tiles (the last query tiles of full rows) no longer bound the kernel.
// Every wave holds the same scores and runs the same softmax, so all control
// flow is workgroup-uniform.
//
// Memory: K comes from the prep workspace in the split layout (each wave's
// run of a tile is one contiguous 1 KB read), V columns straight from V;
// the next tile's K and V slices go into the wave's LDS with LDS-DMA loads
// while the current tile is computed, so no second tile of registers is
// held: the kernel fits 128 VGPRs, four workgroups per CU. Q, the gate and
// the output move along tokens
// 16 bytes at a time and are transposed in the wave's own LDS rows, so a
// wave issues four vector memory instructions per tensor. The row's key span
// and active-key bits come from the prep (scalar loads).
//
// Workgroups are numbered from the last query tile down, so the longest
// causal walks start first; within one query tile, the workgroups of one
// (row, kv head) share an id residue mod 8 (one XCD, one L2) when the counts
// allow it (jeff_unit_of).
template <int HDP>
__global__ __launch_bounds__(256, 4) void jeff_split_f32_kernel(const JeffArgs a,
                                                                const float *__restrict__ kp,
                                                                const int *__restrict__ spans,
                                                                const uint32_t *__restrict__ kbits,
                                                                int rows) {
  static_assert(HDP == 256, "split-head kernel: four 64-feature slices");
  constexpr int DS = HDP / 4;    // features per wave
  constexpr int QS = DS / 4;     // Q registers per lane: MFMA steps per tile
  constexpr int NB = DS / 16;    // 16-feature blocks of O^T per wave
  constexpr int KT = kJeffKeyTile;
  constexpr int QW = DS + 4;     // wave rows [query][feature] for Q
  constexpr int OW = 16;         // wave rows [feature][query] for the output (the K slice)
  constexpr int WROWS = DS * OW > 16 * QW ? DS * OW : 16 * QW;
  constexpr int QP = HDP + 4;    // whole-tile Q rows (RoPE widths other than 16, 32)
  constexpr int WAREA = 4 * WROWS > 16 * QP ? 4 * WROWS : 16 * QP;
  constexpr int SX = 2 * 4 * 64 * 4;  // score exchange: 2 buffers x 4 waves x 64 lanes x f32x4
  // Each wave's K and V tile slices (4 KB each), where the next tile lands
  // while the current one is computed; the wave rows and the whole-tile Q
  // rows use the same bytes before the walk and after it. 40 KB in all, so
  // four workgroups share a CU's 160 KB.
  constexpr int KVW = 2 * QS * 64;  // floats per wave: K and V, 16 floats per lane each
  constexpr int KVAREA = 4 * KVW;
  static_assert(WAREA <= KVAREA && WROWS <= KVW && DS * OW <= QS * 64,
                "the wave rows alias the wave's tile slices; the output rows its K slice");
  __shared__ __attribute__((aligned(16))) float smem[KVAREA + SX];
  // RMSNorm partial sums in exchange buffer 1, read before its first use.
  float *const s_ssq = smem + KVAREA + SX / 2;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, grp = lane >> 4;
  const int L = a.L, hd = a.hd;

  // Issue priority (s_setprio, within this kernel's waves on a SIMD): the
  // prologue and the epilogue above the walks of the CU's other workgroups,
  // so that a workgroup reaches its walk, and frees its slot, sooner (f32
  // MFMAs and vector instructions of a SIMD never run at the same time).
  __builtin_amdgcn_s_setprio(2);

  // -------- work item: query tiles from the last one down (blockIdx.y),
  // the (row, head) unit in blockIdx.x.
  const int qt = (int)gridDim.y - 1 - (int)blockIdx.y;
  int row, head;
  jeff_unit_of(a, rows, blockIdx.x, row, head);
  const int kvh = min((int)a.gdiv.div((uint32_t)head), a.kv_heads - 1);
  const int q0 = qt * 16, q = q0 + col;
  const float *Q = static_cast<const float *>(a.q) + row * a.q_row + (size_t)head * hd * L;
  const float *Gt = static_cast<const float *>(a.gate) + row * a.q_row + (size_t)head * hd * L;
  const float *V = static_cast<const float *>(a.v) + row * a.kv_row + (size_t)kvh * a.kv_head;
  const int Lp = (L + 15) & ~15;
  const float *KP = kp + ((size_t)row * a.kv_heads + kvh) * (size_t)Lp * HDP;
  const uint32_t *rbits = kbits + (size_t)row * ((L + 31) / 32);
  float *OUT = a.out + row * a.q_row + (size_t)head * hd * L;
  float *ww = smem + wave * (2 * QS * 64);  // this wave's rows: its K and V slices

  // This lane's features in both products: step (c, e) of the 16x16x4 MFMA
  // chain uses feature d0 + 16c + e (the prep workspace's run order).
  const int d0 = wave * DS + 4 * grp;
  // Along-token tasks of the wave's slice (Q, gate, output): task t is
  // feature wave*DS + (lane >> 2) + 16t, tokens q0 + 4*(lane & 3) .. + 3.
  const int tdl = lane >> 2, tg4 = lane & 3;

  // -------- loads that need nothing: the row's key span, the diagonal key
  // tile (the walk runs from it down to the row's first active key).
  // K: key k0 + col, features d0 + 16c .. + 3 = run c of the tile's block
  // for this wave, chunk lane (zero past hd and past L). V: V[wave*DS + 16j
  // + col][k0 + 4*grp .. + 3].
  const __amdgpu_buffer_rsrc_t rk = buffer_rsrc(KP, (uint32_t)((size_t)Lp * HDP * 4));
  const __amdgpu_buffer_rsrc_t rv = buffer_rsrc(V, (uint32_t)((size_t)hd * L * 4));
  const int okk = wave * 4096 + lane * 16;
  const int ovv = ((wave * DS + col) * L + 4 * grp) * 4;
  f32x4 kc[QS / 4], vc[NB];
  auto fetch = [&](int k0, f32x4 (&kr)[QS / 4], f32x4 (&vr)[NB]) {
    k0 = __builtin_amdgcn_readfirstlane(k0);  // uniform: scalar offsets, no waterfall
#pragma unroll
    for (int c = 0; c < QS / 4; ++c) kr[c] = buffer_load4(rk, okk + 1024 * c, k0 * HDP * 4);
#pragma unroll
    for (int j = 0; j < NB; ++j) vr[j] = buffer_load4(rv, ovv + j * 16 * L * 4, k0 * 4);
  };
  // The Q tile's HBM round trip starts with the item (wasted only for a
  // tile with no key, which never reads it).
  const __amdgpu_buffer_rsrc_t rq = buffer_rsrc(Q, (uint32_t)((size_t)hd * L * 4));
  const int otask = ((wave * DS + tdl) * L + 4 * tg4) * 4;  // byte offset of task 0
  f32x4 qx[NB];
#pragma unroll
  for (int t = 0; t < NB; ++t) qx[t] = buffer_load4(rq, otask + t * 16 * L * 4, q0 * 4);
  const int first = spans[2 * row], last = spans[2 * row + 1];
  fetch(qt * KT, kc, vc);
  const int start = (a.trim && last >= 0) ? first : 0;
  const bool q_live = q < L && q >= start;
  const int q_last = min(q0 + 15, L - 1);
  int kt_begin = 0, kt_end = 0;
  {
    const int kl = min(last, q_last);
    if (last >= 0 && first <= kl && q_last >= start) {
      kt_begin = first / KT;
      kt_end = kl / KT + 1;
    }
  }
  kt_begin = __builtin_amdgcn_readfirstlane(kt_begin);
  kt_end = __builtin_amdgcn_readfirstlane(kt_end);

  const __amdgpu_buffer_rsrc_t rg = buffer_rsrc(Gt, (uint32_t)((size_t)hd * L * 4));
  const __amdgpu_buffer_rsrc_t ro = buffer_rsrc(OUT, (uint32_t)((size_t)hd * L * 4));
  f32x4 gv[NB];
  auto load_gate = [&]() {
#pragma unroll
    for (int t = 0; t < NB; ++t) gv[t] = buffer_load4(rg, otask + t * 16 * L * 4, q0 * 4);
  };
  // o * sigmoid(gate) (lib.rs:755-758) for task t, o = O^T * inv; 0 for a
  // dropped query (q < start). L % 4 == 0: a task's 4 tokens are all in or
  // all out.
  auto store_task = [&](int t, f32x4 o) {
    const int qa = q0 + 4 * tg4, d = wave * DS + tdl + 16 * t;
    f32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = qa + i < start ? 0.0f : o[i] * fast_sigmoid(gv[t][i]);
    if (qa < L && d < hd) buffer_store4_nt(r, ro, otask + t * 16 * L * 4, q0 * 4);
  };
  if (kt_begin >= kt_end) {
    // No key at or before these queries: o = 0 (lib.rs:739-743), and
    // 0 * sigmoid(gate) is 0 for every gate but NaN (sigmoid is in [0, 1],
    // also at +-inf), which it propagates: no exponential needed.
    load_gate();
#pragma unroll
    for (int t = 0; t < NB; ++t) {
      const int qa = q0 + 4 * tg4, d = wave * DS + tdl + 16 * t;
      f32x4 r;
#pragma unroll
      for (int i = 0; i < 4; ++i) r[i] = (qa + i >= start && gv[t][i] != gv[t][i]) ? gv[t][i] : 0.0f;
      if (qa < L && d < hd) buffer_store4_nt(r, ro, otask + t * 16 * L * 4, q0 * 4);
    }
    return;
  }

  // -------- Q: the wave's slice along tokens, transposed through its LDS
  // rows into this lane's B operands (feature d0 + 16c + e of query q0 +
  // col; features past hd read as 0); its norm weights and, where the RoPE
  // partners sit in the same lane (rot/2 = 16 or 32: partner of step (c, e)
  // is (c + rot/32, e)), its table entries.
  const int rh = a.rot_half;
  const bool rope = a.cos_t != nullptr && rh > 0;
  const bool lane_rope = rh == 16 || rh == 32;
  const __amdgpu_buffer_rsrc_t rn = buffer_rsrc(a.q_norm, (uint32_t)(hd * 4));
  f32x4 wv[QS / 4];
#pragma unroll
  for (int c = 0; c < QS / 4; ++c) wv[c] = buffer_load4(rn, (d0 + 16 * c) * 4, 0);
  f32x4 tc[2], ts[2];  // wave 0, lane_rope: table entries of pairs i = 4*grp + 16c + e, c < rh/16
  if (rope && lane_rope && wave == 0) {
    const size_t pos = (size_t)min(max(q - start, 0), L - 1) * rh;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int i = min(4 * grp + 16 * c, rh - 4);
      tc[c] = *reinterpret_cast<const f32x4 *>(a.cos_t + pos + i);
      ts[c] = *reinterpret_cast<const f32x4 *>(a.sin_t + pos + i);
    }
  }
#pragma unroll
  for (int t = 0; t < NB; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) ww[(4 * tg4 + i) * QW + tdl + 16 * t] = qx[t][i];
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float qv[QS];
#pragma unroll
  for (int c = 0; c < QS / 4; ++c) {
    const f32x4 y = *reinterpret_cast<const f32x4 *>(ww + col * QW + 4 * grp + 16 * c);
#pragma unroll
    for (int e = 0; e < 4; ++e) qv[4 * c + e] = y[e];
  }

  // -------- RMSNorm (lib.rs:676-691): the sum of squares over the four
  // waves' slices through LDS, then partial RoPE (692-709).
  float ss = 0.0f;
#pragma unroll
  for (int c = 0; c < QS / 4; ++c)
    ss += qv[4 * c] * qv[4 * c] + qv[4 * c + 1] * qv[4 * c + 1] + qv[4 * c + 2] * qv[4 * c + 2] +
          qv[4 * c + 3] * qv[4 * c + 3];
  ss = pair_sum(pair16_sum(ss));
  if (grp == 0) s_ssq[wave * 16 + col] = ss;
  __syncthreads();
  const float tot = s_ssq[col] + s_ssq[16 + col] + s_ssq[32 + col] + s_ssq[48 + col];
  const float scale = rms_scale(tot, hd, a.eps);
  float qreg[QS];
#pragma unroll
  for (int c = 0; c < QS / 4; ++c)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int d = d0 + 16 * c + e;
      qreg[4 * c + e] = (q_live && d < hd) ? rms_apply(qv[4 * c + e], scale, wv[c][e]) : 0.0f;
    }
  if (rope && lane_rope) {
    if (wave == 0 && q_live) {
      // pc: register-block offset of the partner, a constant in each branch
      // (a run-time one indexes the register array indirectly).
      auto rotate = [&](auto pcv) {
        constexpr int pc = decltype(pcv)::value;
#pragma unroll
        for (int c = 0; c < pc; ++c)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float x = qreg[4 * c + e], y = qreg[4 * (c + pc) + e];
            qreg[4 * c + e] = rope_lo(x, y, tc[c][e], ts[c][e]);
            qreg[4 * (c + pc) + e] = rope_hi(x, y, tc[c][e], ts[c][e]);
          }
      };
      if (rh == 16)
        rotate(std::integral_constant<int, 1>{});
      else
        rotate(std::integral_constant<int, 2>{});
    }
  } else if (rope) {
    // Any other rotary width: rotate the normalized rows of the whole tile
    // in LDS (the wave rows are free again).
    float *Qs = smem;
    __syncthreads();
#pragma unroll
    for (int c = 0; c < QS / 4; ++c)
#pragma unroll
      for (int e = 0; e < 4; ++e) Qs[col * QP + d0 + 16 * c + e] = qreg[4 * c + e];
    __syncthreads();
    const int qi = tid & 15, qa = q0 + qi;
    if (qa < L && qa >= start) {
      const size_t pq = (size_t)(qa - start) * rh;
      float *qr = Qs + qi * QP;
      for (int i = tid >> 4; i < rh; i += 16) {
        const float x = qr[i], y = qr[i + rh];
        const float c = a.cos_t[pq + i], sn = a.sin_t[pq + i];
        qr[i] = rope_lo(x, y, c, sn);
        qr[i + rh] = rope_hi(x, y, c, sn);
      }
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < QS / 4; ++c)
#pragma unroll
      for (int e = 0; e < 4; ++e) qreg[4 * c + e] = Qs[col * QP + d0 + 16 * c + e];
    __syncthreads();  // the tile rows become wave rows again
  }
  f32x4 *sx = reinterpret_cast<f32x4 *>(smem + KVAREA);

  // The next key tile's K and V go into this wave's LDS slices with LDS-DMA
  // loads (no registers held; the wave reads back exactly the bytes it
  // loaded, so it only waits for its own loads). Issued once the previous
  // contents are in registers, one tile ahead of their use.
  unsigned char *const kv_lds = reinterpret_cast<unsigned char *>(smem) + wave * KVW * 4;
  const u32x4r rkw = rsrc_words(KP, (uint32_t)((size_t)Lp * HDP * 4));
  const u32x4r rvw = rsrc_words(V, (uint32_t)((size_t)hd * L * 4));
  auto prefetch = [&](int k0) {
    k0 = __builtin_amdgcn_readfirstlane(k0);
    // One offset register per lane (okk, ovv); the per-load steps go in the
    // scalar offset.
#pragma unroll
    for (int c = 0; c < QS / 4; ++c)
      load_lds16(rkw, (uint32_t)okk, (uint32_t)(k0 * HDP * 4 + 1024 * c), kv_lds + 1024 * c);
#pragma unroll
    for (int j = 0; j < NB; ++j)
      load_lds16(rvw, (uint32_t)ovv, (uint32_t)(k0 * 4 + j * 16 * L * 4),
                 kv_lds + QS * 256 + 1024 * j);
  };
  auto take = [&]() {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int c = 0; c < QS / 4; ++c)
      kc[c] = *reinterpret_cast<const f32x4 *>(kv_lds + 1024 * c + 16 * lane);
#pragma unroll
    for (int j = 0; j < NB; ++j)
      vc[j] = *reinterpret_cast<const f32x4 *>(kv_lds + QS * 256 + 1024 * j + 16 * lane);
  };
  // The gate tasks of the wave's slice go into its V slice during the last
  // step (read back after the walk).
  const u32x4r rgw = rsrc_words(Gt, (uint32_t)((size_t)hd * L * 4));
  auto gate_to_lds = [&]() {
#pragma unroll
    for (int t = 0; t < NB; ++t)
      load_lds16(rgw, (uint32_t)otask, (uint32_t)(q0 * 4 + t * 16 * L * 4),
                 kv_lds + QS * 256 + 1024 * t);
  };

  // Keep word of a 16-key tile for query col: active key (the prep's bits:
  // mask != 0, zero past L), key <= query (lib.rs:716). Keys before `start`
  // are inactive by definition of start. The bits word is loaded one tile
  // ahead (bits_of) and turned into the word after that tile's products.
  auto bits_of = [&](int kt) -> uint32_t { return rbits[kt >> 1]; };
  auto keep_word = [&](int kt, uint32_t word) -> uint32_t {
    const uint32_t abits = (word >> (16 * (kt & 1))) & 0xffffu;
    return q_live ? (abits & range_bits(0, q - kt * KT)) : 0u;
  };

  f32x4 O[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) O[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float m = kNoMax, l = 0.0f;  // l: this lane's share of the row sum
  const float c1 = a.c1;

  // -------- the walk, from the last key tile down (exponents against a
  // lazily moved reference, as in the Laya kernel; the order of the keys
  // only moves rounding). A workgroup whose kept scores sum to NaN or inf
  // stops computing; it, or one whose O took a NaN or inf, redoes the tile
  // with the reference's exact semantics afterwards. The gate loads go out
  // with the last tile. The first tile is in registers (loaded with the
  // item); every later one comes through LDS, prefetched a step ahead (the
  // prologue's last use of the wave rows was before its barrier).
  const int kt_hi = kt_end - 1;
  if (kt_hi != qt) fetch(kt_hi * KT, kc, vc);  // the span ends before the diagonal
  if (kt_hi > kt_begin) prefetch((kt_hi - 1) * KT);
  uint32_t w = keep_word(kt_hi, bits_of(kt_hi));
  bool tainted = false;  // workgroup-uniform
  int xb = 0;            // exchange buffer
  // One step per key tile. The first is peeled off (FIRST): its K and V come
  // from registers, every later one from the slices. So no vector-memory
  // load that the compiler tracks is in flight inside the loop, and the
  // waits it inserts there never hold up the next tile's LDS-DMA loads.
  auto step = [&](int kt, auto first) {
    constexpr bool FIRST = decltype(first)::value;
    const bool more = kt > kt_begin;
    uint32_t bnext = 0u;
    if constexpr (!FIRST) {
      take();
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the slices are in registers
    }
    if (more) {
      if constexpr (!FIRST) prefetch((kt - 1) * KT);
      bnext = bits_of(kt - 1);
    } else {
      gate_to_lds();
    }
    if (kt * KT + KT > L) {  // the row's last, partial tile: V past L is another feature's
#pragma unroll
      for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int t = 0; t < 4; ++t) vc[j][t] = kt * KT + 4 * grp + t < L ? vc[j][t] : 0.0f;
    }
    if (!tainted && __ballot(w != 0u) != 0) {  // workgroup-uniform: every wave has the same w
      f32x4 s0 = {0.0f, 0.0f, 0.0f, 0.0f}, s1 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int c = 0; c < QS / 4; ++c) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (c & 1)
            s1 = mfma_16x16x4(kc[c][e], qreg[4 * c + e], s1);
          else
            s0 = mfma_16x16x4(kc[c][e], qreg[4 * c + e], s0);
        }
      }
      sx[(xb * 4 + wave) * 64 + lane] = s0 + s1;
      __syncthreads();
      f32x4 s = sx[(xb * 4 + 0) * 64 + lane];
#pragma unroll
      for (int v = 1; v < 4; ++v) s += sx[(xb * 4 + v) * 64 + lane];
      xb ^= 1;
      // lane group g holds keys 4g + r of its query
      if (__ballot(q_live && w != 0xffffu) != 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r) s[r] = ((w >> (4 * grp + r)) & 1u) ? s[r] : -INFINITY;
      }
      f32x4 ex;
      float rs = 0.0f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        ex[r] = fast_exp2(__builtin_fmaf(s[r], c1, -m));
        rs += ex[r];
      }
      bool ok = true;
      if (__ballot(q_live && !(rs <= kLazyLimit)) != 0) {
        const float mx = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
        const float mxs = pair_max(pair16_max(mx)) * c1;
        const bool need = mxs > m + kRescaleSlack;
        const float mn = need ? mxs : m;
        rs = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          ex[r] = fast_exp2(__builtin_fmaf(s[r], c1, -mn));
          rs += ex[r];
        }
        if (__ballot(q_live && !__builtin_isfinite(rs)) != 0) {
          tainted = true;
          ok = false;
        } else {
          const float alpha = fast_exp2(m - mn);  // exactly 1 where the reference stays
#pragma unroll
          for (int j = 0; j < NB; ++j) O[j] *= alpha;
          l *= alpha;
          m = mn;
        }
      }
      if (ok) {
        l += rs;
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int j = 0; j < NB; ++j) O[j] = mfma_16x16x4(vc[j][r], ex[r], O[j]);
      }
    }
    if (more) w = keep_word(kt - 1, bnext);
  };
  __builtin_amdgcn_s_setprio(0);
  step(kt_hi, std::true_type{});
  for (int kt = kt_hi - 1; kt >= kt_begin; --kt) step(kt, std::false_type{});
  __builtin_amdgcn_s_setprio(3);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the gate slice, and no LDS-DMA left in flight

  // -------- careful redo (rare): the scores (shared) or this wave's O went
  // non-finite; one wave redoes the whole tile from global memory.
  bool bad = false;
#pragma unroll
  for (int j = 0; j < NB; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) bad |= !__builtin_isfinite(O[j][r]);
  // Flags and the row sums' inverses go into the exchange buffer that the
  // last exchange did not use: every wave finished reading it before that
  // exchange's barrier.
  float *const xs = smem + KVAREA + xb * (SX / 2);
  int *const s_flag = reinterpret_cast<int *>(xs);
  const bool wbad = __ballot(q_live && bad) != 0;
  if (lane == 0) s_flag[wave] = wbad ? 1 : 0;
  __syncthreads();
  if (tainted || (s_flag[0] | s_flag[1] | s_flag[2] | s_flag[3]) != 0) {
    if (wave == 0) jeff_redo_wave<HDP, true, 1>(kernel_jeff_args(), kp, row, head, q0, kt_begin, kt_end, start, smem);
    return;
  }

  // -------- o / sum (0 when nothing was kept), sigmoid gate, store: O^T
  // through the wave's rows [feature][query] so that each task stores 4
  // tokens of one feature.
  float *const s_inv = xs + 64;
  const float lt = pair_sum(pair16_sum(l));
  if (grp == 0) s_inv[wave * 16 + col] = lt > 0.0f ? fast_rcp(lt) : 0.0f;
#pragma unroll
  for (int j = 0; j < NB; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) ww[(16 * j + 4 * grp + r) * OW + col] = O[j][r];
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const f32x4 inv4 = *reinterpret_cast<const f32x4 *>(s_inv + wave * 16 + 4 * tg4);
#pragma unroll
  for (int t = 0; t < NB; ++t)
    gv[t] = *reinterpret_cast<const f32x4 *>(kv_lds + QS * 256 + 1024 * t + 16 * lane);
#pragma unroll
  for (int t = 0; t < NB; ++t) {
    const f32x4 o = *reinterpret_cast<const f32x4 *>(ww + (tdl + 16 * t) * OW + 4 * tg4);
    store_task(t, o * inv4);
  }
}

// ------------------------------------------- f32 attention, fused, hd 256

constexpr int kJeffFusedWaves = 8;  // waves per fused workgroup (the key range's parts)
constexpr int kJeffHalfMaxL = 4096;  // longest row of the two-workgroup fused kernel

// One kernel for the whole op at hd 256 (no K prep): one workgroup = NW
// wavefronts = one (row, head, 16-query tile). The RMSNorm scales are
// folded into the scores: with q' = R_q(x_q (1 + w_q)) and, per key,
// k' = R_k(x_k (1 + w_k)) on the rotated features and x_k elsewhere,
//   s(q, k) = scale_q scale_k (q'' . k') / sqrt(hd),
// where q'' is q' times (1 + w_k) on the features past rot_dim (the same
// product as the reference's q^.k^ of lib.rs:676-716, up to rounding). So
// wave w prepares Q's features 64 w .. 64 w + 63 elementwise (its RoPE pairs
// stay inside slice 0) into LDS, where every wave reads its B operands, and
// scale_q waits in the exponent's factor; a key tile needs only its sum of
// squares, (1 + w_k) and RoPE on its first rot_dim features, all in the
// lanes that feed them to the matrix cores.
//
// Layout (lane = 16 grp + col): B operand Q^T and A operand K carry feature
// f = 64 s + 16 c + 4 grp + e at step (s, c, e) of the S^T chain, for query
// (K: key) col; S^T holds keys 4 grp + r of query col; O^T block J holds
// features 16 J + 4 grp + r. RoPE partners (i, i + rot/2) sit in one lane,
// rot/32 blocks of 16 apart (rot/2 = 16 or 32).
//
// The tile's key range (first active key .. last query) is cut into NW
// contiguous parts walked by the NW waves with no barrier; the partial
// states merge once through LDS. K arrives with 4-byte loads (a lane needs
// one key's features), V with 16-byte loads along tokens; both stream
// through a ring of four 16-register pieces, three ahead: K slices 1, 2, 3,
// then slice 0 (the rotated features, whose table entries load a tile
// ahead), then V groups 0 .. 3. (Eight slots, each piece a whole tile ahead,
// measured slower: 21.7 against 19.3 us per C4 row.)
template <int NW, int RB>  // RB: rotated blocks of 16 in the lower half (rot_dim / 32: 0, 1, 2)
__global__ __launch_bounds__(NW * 64, 8 / NW) void jeff_fused_f32_kernel(const JeffArgs a,
                                                                         int rows) {
  static_assert(RB >= 0 && RB <= 2, "rot_dim 0, 32 or 64");
  constexpr int HDP = 256, NB = 16, KT = 16;
  constexpr int BPW = NB / NW;  // O^T blocks each wave finishes
  static_assert(NW == 4 || NW == 8, "four Q-prep slices; 16 O^T blocks over the waves");
  constexpr int OMF = NW * NB * 64 * 4;  // partial O^T of every wave (the redo's rows too)
  // Q operands [slice][run c][lane] as f32x4 (feature 64 s + 16 c + 4 grp + e
  // of query col), 16 KB at the front of smem until the merge.
  __shared__ __attribute__((aligned(16))) float smem[OMF];
  __shared__ __attribute__((aligned(16))) float s_wkr[4 * 4 * 4];  // (1 + w_k), rotated blocks
  __shared__ float s_ssq[4 * 16];
  __shared__ float s_m[NW * 16], s_l[NW * 16];
  __shared__ int s_bad;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, grp = lane >> 4;
  const int L = a.L;
  const int L4 = 4 * L;

  // -------- work item: query tiles from the last one down; the heads of a
  // (row, kv head) on one XCD.
  const int qt = (int)gridDim.y - 1 - (int)blockIdx.y;
  int row, head;
  jeff_unit_of(a, rows, blockIdx.x, row, head);
  const int kvh = min((int)a.gdiv.div((uint32_t)head), a.kv_heads - 1);
  const int q0 = qt * 16, q = q0 + col;
  const uint32_t bytes = (uint32_t)((size_t)HDP * L * 4);
  const __amdgpu_buffer_rsrc_t rq = buffer_rsrc(
      static_cast<const float *>(a.q) + row * a.q_row + (size_t)head * HDP * L, bytes);
  const __amdgpu_buffer_rsrc_t rg = buffer_rsrc(
      static_cast<const float *>(a.gate) + row * a.q_row + (size_t)head * HDP * L, bytes);
  const __amdgpu_buffer_rsrc_t ro =
      buffer_rsrc(a.out + row * a.q_row + (size_t)head * HDP * L, bytes);
  const float *Kb = static_cast<const float *>(a.k) + row * a.kv_row + (size_t)kvh * a.kv_head;
  const __amdgpu_buffer_rsrc_t rk = buffer_rsrc(Kb, bytes);
  const __amdgpu_buffer_rsrc_t rv = buffer_rsrc(
      static_cast<const float *>(a.v) + row * a.kv_row + (size_t)kvh * a.kv_head, bytes);
  const __amdgpu_buffer_rsrc_t rm = buffer_rsrc(a.mask + (size_t)row * L, (uint32_t)L4);
  // Per-lane byte offsets: feature 4 grp (+ the step's 64s + 16c + e, a
  // scalar offset) of token col (+ the tile's first token, scalar). A lane
  // with nothing to load takes an offset past the buffer's end, which the
  // hardware range check reads as 0 (whether or not it adds the scalar part).
  const int ofs_t = (4 * grp * L + col) * 4;
  const int koob = (int)bytes;
  const int ofs_q = q < L ? ofs_t : koob;

  // -------- loads that need nothing: Q slice `wave` (waves 0 .. 3) in
  // B-operand order (feature 64 wave + 16 c + 4 grp + e), its norm weights.
  const bool prep = wave < 4;
  const int sw = wave & 3;
  float xq[16];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int e = 0; e < 4; ++e)
      xq[4 * c + e] = prep ? buffer_load1(rq, ofs_q, q0 * 4 + (64 * sw + 16 * c + e) * L4) : 0.0f;
  const __amdgpu_buffer_rsrc_t rwq = buffer_rsrc(a.q_norm, HDP * 4);
  const __amdgpu_buffer_rsrc_t rwk = buffer_rsrc(a.k_norm, HDP * 4);
  f32x4 wq[4], wk[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    wq[c] = buffer_load4(rwq, (64 * sw + 16 * c + 4 * grp) * 4, 0);
    wk[c] = buffer_load4(rwk, (64 * sw + 16 * c + 4 * grp) * 4, 0);
  }

  // -------- the row's active span (mask != 0), every wave on its own.
  int first, last;
  {
    int lo = 0x7fffffff, hi = -1;
    for (int k0 = 0; k0 < L; k0 += 256) {
      const f32x4 mv = buffer_load4(rm, (k0 + 4 * lane) * 4, 0);  // past L: 0
#pragma unroll
      for (int t = 0; t < 4; ++t)
        if (mv[t] != 0.0f) {
          lo = min(lo, k0 + 4 * lane + t);
          hi = max(hi, k0 + 4 * lane + t);
        }
    }
    lo = wave_min(lo);
    hi = wave_max(hi);
    first = __builtin_amdgcn_readfirstlane(hi >= 0 ? lo : 0);
    last = __builtin_amdgcn_readfirstlane(hi);
  }
  const int start = (a.trim && last >= 0) ? first : 0;
  const bool q_live = q < L && q >= start;
  const int q_last = min(q0 + 15, L - 1);
  int kt_begin = 0, kt_end = 0;
  {
    const int kl = min(last, q_last);
    if (last >= 0 && first <= kl && q_last >= start) {
      kt_begin = first / KT;
      kt_end = kl / KT + 1;
    }
  }
  // o * sigmoid(gate) (lib.rs:755-758) for the wave's features 16 (BPW wave
  // + j) + 4 grp + r of query col; 0 for a dropped query (q < start).
  auto finish = [&](const f32x4 (&o)[BPW]) {
    float g[4 * BPW];
#pragma unroll
    for (int j = 0; j < BPW; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        g[4 * j + r] = buffer_load1(rg, ofs_q, q0 * 4 + (16 * (BPW * wave + j) + r) * L4);
    if (q < L) {
#pragma unroll
      for (int j = 0; j < BPW; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float x = q < start ? 0.0f : o[j][r] * fast_sigmoid(g[4 * j + r]);
          buffer_store1_nt(x, ro, ofs_t, q0 * 4 + (16 * (BPW * wave + j) + r) * L4);
        }
    }
  };
  if (kt_begin >= kt_end) {  // no key at or before these queries: o = 0 (lib.rs:739-743)
    const f32x4 z[BPW] = {};
    finish(z);
    return;
  }

  // -------- Q: x (1 + w_q), RoPE, (1 + w_k) past rot_dim, into LDS; the sum
  // of squares over the four slices gives scale_q.
  constexpr int rb = RB, rh = 16 * RB;
  float ssq = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) ssq += xq[i] * xq[i];
  ssq += __shfl_xor(ssq, 16);
  ssq += __shfl_xor(ssq, 32);
  if (prep && grp == 0) s_ssq[sw * 16 + col] = ssq;
  float qs[16];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int e = 0; e < 4; ++e) qs[4 * c + e] = xq[4 * c + e] * (1.0f + wq[c][e]);
  if (rb > 0 && wave == 0) {  // slice 0 holds the rotated features
    const int pos = min(max(q - start, 0), L - 1);
#pragma unroll
    for (int b = 0; b < rb; ++b) {
      const f32x4 cs = *reinterpret_cast<const f32x4 *>(a.cos_t + (size_t)pos * rh + 16 * b + 4 * grp);
      const f32x4 sn = *reinterpret_cast<const f32x4 *>(a.sin_t + (size_t)pos * rh + 16 * b + 4 * grp);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x = qs[4 * b + e], y = qs[4 * (b + rb) + e];
        qs[4 * b + e] = rope_lo(x, y, cs[e], sn[e]);
        qs[4 * (b + rb) + e] = rope_hi(x, y, cs[e], sn[e]);
      }
    }
  }
  f32x4 *QL = reinterpret_cast<f32x4 *>(smem);
  if (prep) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const bool rotated = wave == 0 && c < 2 * rb;
      f32x4 y;
#pragma unroll
      for (int e = 0; e < 4; ++e) y[e] = q_live ? qs[4 * c + e] * (rotated ? 1.0f : 1.0f + wk[c][e]) : 0.0f;
      QL[(sw * 4 + c) * 64 + lane] = y;
    }
  }
  if (wave == 0 && col == 0) {
#pragma unroll
    for (int c = 0; c < 4; ++c) *reinterpret_cast<f32x4 *>(s_wkr + (c * 4 + grp) * 4) = wk[c] + 1.0f;
  }
  __syncthreads();
  const float c1q =
      a.c1 * rms_scale(s_ssq[col] + s_ssq[16 + col] + s_ssq[32 + col] + s_ssq[48 + col], HDP, a.eps);

  // -------- this wave's part of the key range.
  const int T = kt_end - kt_begin;
  const int w_begin = kt_begin + (T * wave) / NW, w_end = kt_begin + (T * (wave + 1)) / NW;
  // Ring slot i % 4: piece i of a tile, i = 0, 1, 2: K slice i + 1; 3: K
  // slice 0; 4 .. 7: V group i - 4 (O^T blocks 4 (i - 4) .. + 3). Loads are
  // unconditional (at the last tile the "next" K pieces re-read the current
  // tile), so no ring slot ever holds one of two values.
  f32x4 ring[4][4];
  f32x4 tcs[2], tsn[2];  // the tile's table entries (rotated pairs of key col)
  auto k_off = [&](int kt) -> int { return kt * KT + col < L ? ofs_t : koob; };
  auto load_k = [&](int slot, int sl, int kt) {
    const int vo = k_off(kt);
    kt = __builtin_amdgcn_readfirstlane(kt);
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        ring[slot][c][e] = buffer_load1(rk, vo, kt * KT * 4 + (64 * sl + 16 * c + e) * L4);
  };
  auto load_tab = [&](int kt) {
    if (rb > 0) {
      const int pos = min(max(kt * KT + col - start, 0), L - 1);
#pragma unroll
      for (int b = 0; b < rb; ++b) {
        tcs[b] = *reinterpret_cast<const f32x4 *>(a.cos_t + (size_t)pos * rh + 16 * b + 4 * grp);
        tsn[b] = *reinterpret_cast<const f32x4 *>(a.sin_t + (size_t)pos * rh + 16 * b + 4 * grp);
      }
    }
  };
  // V: features 16 J + col, keys k0 + 4 grp .. + 3 (L % 4 == 0: all in or out).
  const int ofs_v = (col * L + 4 * grp) * 4;
  auto load_v = [&](int slot, int g, int kt) {
    const int k = kt * KT + 4 * grp;
    const int vo = k < L ? ofs_v + kt * KT * 4 : koob;
#pragma unroll
    for (int j = 0; j < 4; ++j) ring[slot][j] = buffer_load4(rv, vo, (4 * g + j) * 16 * L4);
  };

  f32x4 O[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) O[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float m = kNoMax, l = 0.0f;  // l: this lane's share of the row sum
  bool tainted = false;        // wave-uniform

  if (w_begin < w_end) {
    load_tab(w_begin);
    load_k(0, 1, w_begin);
    load_k(1, 2, w_begin);
    load_k(2, 3, w_begin);
  }
  for (int kt = w_begin; kt < w_end; ++kt) {
    const int kn = kt + 1 < w_end ? kt + 1 : kt;
    const int k0 = kt * KT;
    const float mv = buffer_load1(rm, (k0 + col) * 4, 0);  // past L: 0
    f32x4 s0 = {0.0f, 0.0f, 0.0f, 0.0f}, s1 = {0.0f, 0.0f, 0.0f, 0.0f};
    float ssk = 0.0f;
    // S^T over K slices 1, 2, 3 (features past the rotated ones)
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      if (i == 0)
        load_k(3, 0, kt);
      else
        load_v(i - 1, i - 1, kt);  // V groups 0, 1
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float x = ring[i][c][e];
          ssk += x * x;
          const float y = QL[((i + 1) * 4 + c) * 64 + lane][e];
          if (c & 1)
            s1 = mfma_16x16x4(x, y, s1);
          else
            s0 = mfma_16x16x4(x, y, s0);
        }
    }
    // slice 0: sum of squares of the raw key, then x (1 + w_k) and RoPE on
    // the rotated blocks (0 .. 2 rb - 1)
    load_v(2, 2, kt);  // V group 2
    {
      f32x4(&k)[4] = ring[3];
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int e = 0; e < 4; ++e) ssk += k[c][e] * k[c][e];
#pragma unroll
      for (int c = 0; c < 4; ++c)
        if (c < 2 * rb) k[c] *= *reinterpret_cast<const f32x4 *>(s_wkr + (c * 4 + grp) * 4);
#pragma unroll
      for (int b = 0; b < rb; ++b) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float x = k[b][e], y = k[b + rb][e];
          k[b][e] = rope_lo(x, y, tcs[b][e], tsn[b][e]);
          k[b + rb][e] = rope_hi(x, y, tcs[b][e], tsn[b][e]);
        }
      }
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float y = QL[c * 64 + lane][e];
          if (c & 1)
            s1 = mfma_16x16x4(k[c][e], y, s1);
          else
            s0 = mfma_16x16x4(k[c][e], y, s0);
        }
    }
    // the key's scale (lanes col hold key col), to the S^T rows 4 grp + r
    ssk += __shfl_xor(ssk, 16);
    ssk += __shfl_xor(ssk, 32);
    const float sck = rms_scale(ssk, HDP, a.eps);
    const uint32_t abits = (uint32_t)__ballot(mv != 0.0f && k0 + col >= start) & 0xffffu;
    const uint32_t w = q_live ? (abits & range_bits(0, q - k0)) : 0u;
    f32x4 s = s0 + s1;
#pragma unroll
    for (int r = 0; r < 4; ++r) s[r] *= c1q * __shfl(sck, 4 * grp + r);
    if (__ballot(q_live && w != 0xffffu) != 0) {
#pragma unroll
      for (int r = 0; r < 4; ++r) s[r] = ((w >> (4 * grp + r)) & 1u) ? s[r] : -INFINITY;
    }
    load_tab(kn);  // the next tile's table entries
    f32x4 ex;
    float rs = 0.0f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      ex[r] = fast_exp2(s[r] - m);
      rs += ex[r];
    }
    if (__builtin_expect(__ballot(q_live && !(rs <= kLazyLimit)) != 0, 0)) {
      const float mx = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
      const float mxs = pair_max(pair16_max(mx));
      const float mn = mxs > m + kRescaleSlack ? mxs : m;
      rs = 0.0f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        ex[r] = fast_exp2(s[r] - mn);
        rs += ex[r];
      }
      if (__ballot(q_live && !__builtin_isfinite(rs)) != 0) {
        tainted = true;
      } else {
        const float alpha = fast_exp2(m - mn);  // exactly 1 where the reference stays
#pragma unroll
        for (int j = 0; j < NB; ++j) O[j] *= alpha;
        l *= alpha;
        m = mn;
      }
    }
    l += rs;
    // P.V: V groups 0 .. 3 in slots 0, 1, 2 and (loaded now) 3; the next
    // tile's K slices 1 .. 3 into slots 0 .. 2 as they free up.
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      if (g == 0)
        load_v(3, 3, kt);
      else
        load_k(g - 1, g, kn);
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          O[4 * g + j] = mfma_16x16x4(ring[g][j][r], ex[r], O[4 * g + j]);
    }
    if (tainted) break;  // wave-uniform; the whole tile is redone below
  }

  // -------- careful redo (rare): some wave's scores or O went non-finite;
  // one wave redoes the whole tile with the reference's exact semantics.
  if (tid == 0) s_bad = 0;
  __syncthreads();
  bool bad = tainted;
#pragma unroll
  for (int j = 0; j < NB; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) bad |= q_live && !__builtin_isfinite(O[j][r]);
  if (__ballot(bad) != 0 && lane == 0) s_bad = 1;
  __syncthreads();
  if (s_bad != 0) {
    if (wave == 0)
      jeff_redo_wave<HDP, true, 2>(kernel_jeff_args(), nullptr, row, head, q0, kt_begin, kt_end,
                                   start, smem);
    return;
  }

  // -------- merge: O = sum_w 2^(m_w - M) O_w / sum_w 2^(m_w - M) l_w; wave w
  // finishes O^T blocks BPW w .. BPW w + BPW - 1. Every
  // wave is past its walk (the barrier above), so OM may cover the Q rows.
  f32x4 *OM = reinterpret_cast<f32x4 *>(smem);
#pragma unroll
  for (int j = 0; j < NB; ++j) OM[(wave * NB + j) * 64 + lane] = O[j];
  const float lt = pair_sum(pair16_sum(l));
  if (grp == 0) {
    s_m[wave * 16 + col] = m;
    s_l[wave * 16 + col] = lt;
  }
  __syncthreads();
  float M = s_m[col];
#pragma unroll
  for (int v = 1; v < NW; ++v) M = fmaxf(M, s_m[v * 16 + col]);
  float fac[NW], lsum = 0.0f;
#pragma unroll
  for (int v = 0; v < NW; ++v) {
    fac[v] = fast_exp2(s_m[v * 16 + col] - M);  // 0 for a wave without keys (m = kNoMax)
    lsum += fac[v] * s_l[v * 16 + col];
  }
  const float inv = lsum > 0.0f ? fast_rcp(lsum) : 0.0f;
  f32x4 Of[BPW];
#pragma unroll
  for (int j = 0; j < BPW; ++j) {
    Of[j] = OM[(BPW * wave + j) * 64 + lane] * fac[0];
#pragma unroll
    for (int v = 1; v < NW; ++v) Of[j] += OM[(v * NB + BPW * wave + j) * 64 + lane] * fac[v];
    Of[j] *= inv;
  }
  finish(Of);
}

// ------------------------------------ f32 attention, fused, hd 256, halves

// Grids that fill at most half the CUs (a per-row call is 128 work items):
// each (row, head, 16-query tile) item runs as two workgroups, blockIdx.z =
// h, that each compute the item's whole S^T (all 256 features) and its
// softmax, and P.V and the output for features 128 h .. 128 h + 127 only.
// The scores are computed twice, but the grid fills twice as many CUs, an
// item's longest walk on one CU carries 96 instead of 128 MFMAs per key
// tile, and the two workgroups exchange nothing: each writes its own
// features, and decides on its own whether its half needs the careful redo.
// The ring holds one whole tile (six 16-register pieces: K slices 1, 2, 3,
// 0 and V groups 2h, 2h + 1), and every piece is reloaded with the next
// tile's as soon as its MFMAs have read it, so each load has a whole tile
// of the wave's work to land. The eight waves take the key tiles in turn
// from the diagonal down (wave w: the w-th, (w + 8)-th, ... below it), so a
// wave's first tile is known from the query tile alone in rows without
// right padding, and its loads go out with Q's. Layouts, the folded RMSNorm
// scales, the walk's softmax and the merge are those of
// jeff_fused_f32_kernel.
template <int RB, bool TRIM>  // RB: rotated blocks of 16 in the lower half (rot_dim / 32: 0, 1, 2);
                               // TRIM: a.trim (positions count from the row's first active key)
__global__ __launch_bounds__(512, 1) void jeff_fused_half_f32_kernel(const JeffArgs a, int rows) {
  static_assert(RB >= 0 && RB <= 2, "rot_dim 0, 32 or 64");
  constexpr int NW = 8, HDP = 256, NBH = 8, KT = 16;  // NBH: O^T blocks of the half, one per wave
  constexpr int OMF = NW * NBH * 64 * 4;  // partial O^T of every wave (the redo's rows too)
  static_assert(OMF >= 16 * 64 * 4, "the Q operands fit in front of the merge rows");
  __shared__ __attribute__((aligned(16))) float smem[OMF];
  __shared__ __attribute__((aligned(16))) float s_wkr[4 * 4 * 4];  // (1 + w_k), rotated blocks
  __shared__ float s_ssq[4 * 16];
  __shared__ float s_m[NW * 16], s_l[NW * 16];
  __shared__ int s_bad;
  __shared__ uint8_t s_act[kJeffHalfMaxL];  // mask != 0 per key of the row (launcher: L <= this)

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, grp = lane >> 4;
  const int L = a.L;
  const int L4 = 4 * L;
  const int h = (int)blockIdx.z;  // feature half

  const int qt = (int)gridDim.y - 1 - (int)blockIdx.y;
  int row, head;
  jeff_unit_of(a, rows, blockIdx.x, row, head);
  const int kvh = min((int)a.gdiv.div((uint32_t)head), a.kv_heads - 1);
  const int q0 = qt * 16, q = q0 + col;
  const uint32_t bytes = (uint32_t)((size_t)HDP * L * 4);
  const __amdgpu_buffer_rsrc_t rq = buffer_rsrc(
      static_cast<const float *>(a.q) + row * a.q_row + (size_t)head * HDP * L, bytes);
  const __amdgpu_buffer_rsrc_t rg = buffer_rsrc(
      static_cast<const float *>(a.gate) + row * a.q_row + (size_t)head * HDP * L, bytes);
  const __amdgpu_buffer_rsrc_t ro =
      buffer_rsrc(a.out + row * a.q_row + (size_t)head * HDP * L, bytes);
  const float *Kb = static_cast<const float *>(a.k) + row * a.kv_row + (size_t)kvh * a.kv_head;
  const __amdgpu_buffer_rsrc_t rk = buffer_rsrc(Kb, bytes);
  const __amdgpu_buffer_rsrc_t rv = buffer_rsrc(
      static_cast<const float *>(a.v) + row * a.kv_row + (size_t)kvh * a.kv_head, bytes);
  const __amdgpu_buffer_rsrc_t rm = buffer_rsrc(a.mask + (size_t)row * L, (uint32_t)L4);
  // Per-lane byte offsets: feature 4 grp (+ the step's 64s + 16c + e, a
  // scalar offset) of token col (+ the tile's first token, scalar); past the
  // buffer's end (read as 0) for a lane with nothing to load.
  const int ofs_t = (4 * grp * L + col) * 4;
  const int koob = (int)bytes;
  const int ofs_q = q < L ? ofs_t : koob;

  // -------- Q slice `wave` (waves 0 .. 3) and its norm weights.
  const bool prep = wave < 4;
  const int sw = wave & 3;
  float xq[16];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int e = 0; e < 4; ++e)
      xq[4 * c + e] = buffer_load1(rq, ofs_q, q0 * 4 + (64 * sw + 16 * c + e) * L4);  // waves 4-7: unused
  const __amdgpu_buffer_rsrc_t rwq = buffer_rsrc(a.q_norm, HDP * 4);
  const __amdgpu_buffer_rsrc_t rwk = buffer_rsrc(a.k_norm, HDP * 4);
  f32x4 wq[4], wk[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    wq[c] = buffer_load4(rwq, (64 * sw + 16 * c + 4 * grp) * 4, 0);
    wk[c] = buffer_load4(rwk, (64 * sw + 16 * c + 4 * grp) * 4, 0);
  }

  // -------- the ring, the gate, and a first key tile on a guess. Wave w
  // walks key tiles kt_end - 1 - w, kt_end - 1 - w - NW, ... down to
  // kt_begin; the span (below) gives kt_end = qt + 1 whenever the row's last
  // active key is at or past the tile's last query (no right padding), so
  // the wave's first tile qt - w is loaded with Q, before the span is known,
  // and loaded again only if the guess was wrong.
  constexpr int rb = RB, rh = 16 * RB;
  f32x4 ring[6][4];
  f32x4 tcs[2], tsn[2];  // the tile's table entries (rotated pairs of key col)
  auto k_off = [&](int kt) -> int { return kt * KT + col < L ? ofs_t : koob; };
  auto load_k = [&](int slot, int sl, int kt) {
    const int vo = k_off(kt);
    kt = __builtin_amdgcn_readfirstlane(kt);
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        ring[slot][c][e] = buffer_load1(rk, vo, kt * KT * 4 + (64 * sl + 16 * c + e) * L4);
  };
  // V: features 16 J + col, keys k0 + 4 grp .. + 3 (L % 4 == 0: all in or out).
  const int ofs_v = (col * L + 4 * grp) * 4;
  auto load_v = [&](int slot, int g, int kt) {
    const int k = kt * KT + 4 * grp;
    const int vo = k < L ? ofs_v + kt * KT * 4 : koob;
#pragma unroll
    for (int j = 0; j < 4; ++j) ring[slot][j] = buffer_load4(rv, vo, (4 * g + j) * 16 * L4);
  };
  auto load_tile = [&](int kt) {
    load_k(0, 1, kt);
    load_k(1, 2, kt);
    load_k(2, 3, kt);
    load_k(3, 0, kt);
    load_v(4, 2 * h, kt);
    load_v(5, 2 * h + 1, kt);
  };
  // o * sigmoid(gate) (lib.rs:755-758) for features 16 (8 h + wave) + 4 grp
  // + r of query col; 0 for a dropped query (q < start).
  const int fb = 16 * (NBH * h + wave);
  float gt[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) gt[r] = buffer_load1(rg, ofs_q, q0 * 4 + (fb + r) * L4);
  // Q's table entries: at position q, loaded with Q, when nothing is
  // trimmed; after the span (position q - start) when rows are trimmed.
  f32x4 qcs[2], qsn[2];
  auto load_qtab = [&](int pos) {
#pragma unroll
    for (int b = 0; b < RB; ++b) {
      qcs[b] = *reinterpret_cast<const f32x4 *>(a.cos_t + (size_t)pos * rh + 16 * b + 4 * grp);
      qsn[b] = *reinterpret_cast<const f32x4 *>(a.sin_t + (size_t)pos * rh + 16 * b + 4 * grp);
    }
  };
  if constexpr (!TRIM) load_qtab(min(q, L - 1));
  // The mask's first 256 keys are loaded before the guessed tile, so that
  // waiting for them (loads complete in order) does not wait for the tile.
  const f32x4 mv0 = buffer_load4(rm, 4 * lane * 4, 0);  // past L: 0
  // Unconditional (tile 0 for a wave past the diagonal), so that the
  // compiler's waits after it count the same loads on every path.
  const int guess = max(qt - wave, 0);
  asm volatile("" ::: "memory");  // keeps the loads above ahead of the tile's
  load_tile(guess);

  // -------- the row's active span (mask != 0), every wave on its own; wave
  // 0 also keeps each key's flag in LDS for the walk (read after the Q-prep
  // barrier), so no load of the walk is waited for out of its order.
  int first, last;
  {
    int lo = 0x7fffffff, hi = -1;
    for (int k0 = 0; k0 < L; k0 += 256) {
      const f32x4 mv = k0 == 0 ? mv0 : buffer_load4(rm, (k0 + 4 * lane) * 4, 0);  // past L: 0
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        if (mv[t] != 0.0f) {
          lo = min(lo, k0 + 4 * lane + t);
          hi = max(hi, k0 + 4 * lane + t);
        }
        if (wave == 0 && k0 + 4 * lane + t < L) s_act[k0 + 4 * lane + t] = mv[t] != 0.0f;
      }
    }
    lo = wave_min(lo);
    hi = wave_max(hi);
    first = __builtin_amdgcn_readfirstlane(hi >= 0 ? lo : 0);
    last = __builtin_amdgcn_readfirstlane(hi);
  }
  const int start = (TRIM && last >= 0) ? first : 0;
  const bool q_live = q < L && q >= start;
  const int q_last = min(q0 + 15, L - 1);
  int kt_begin = 0, kt_end = 0;
  {
    const int kl = min(last, q_last);
    if (last >= 0 && first <= kl && q_last >= start) {
      kt_begin = first / KT;
      kt_end = kl / KT + 1;
    }
  }
  auto finish = [&](const f32x4 o) {
    if (q < L) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float x = q < start ? 0.0f : o[r] * fast_sigmoid(gt[r]);
        buffer_store1_nt(x, ro, ofs_t, q0 * 4 + (fb + r) * L4);
      }
    }
  };
  if (kt_begin >= kt_end) {  // no key at or before these queries: o = 0 (lib.rs:739-743)
    finish(f32x4{0.0f, 0.0f, 0.0f, 0.0f});
    return;
  }
  const int kt_first = kt_end - 1 - wave;  // this wave's first tile (none below kt_begin)
  auto load_tab = [&](int kt) {
    if (rb > 0) {
      const int pos = min(max(kt * KT + col - start, 0), L - 1);
#pragma unroll
      for (int b = 0; b < rb; ++b) {
        tcs[b] = *reinterpret_cast<const f32x4 *>(a.cos_t + (size_t)pos * rh + 16 * b + 4 * grp);
        tsn[b] = *reinterpret_cast<const f32x4 *>(a.sin_t + (size_t)pos * rh + 16 * b + 4 * grp);
      }
    }
  };
  if (kt_first >= kt_begin) {
    if (kt_first != guess) load_tile(kt_first);
    load_tab(kt_first);
  }

  // -------- Q: x (1 + w_q), RoPE, (1 + w_k) past rot_dim, into LDS; the sum
  // of squares over the four slices gives scale_q.
  float ssq = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) ssq += xq[i] * xq[i];
  ssq += __shfl_xor(ssq, 16);
  ssq += __shfl_xor(ssq, 32);
  if (prep && grp == 0) s_ssq[sw * 16 + col] = ssq;
  float qs[16];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int e = 0; e < 4; ++e) qs[4 * c + e] = xq[4 * c + e] * (1.0f + wq[c][e]);
  if constexpr (TRIM) load_qtab(min(max(q - start, 0), L - 1));
  if (rb > 0 && wave == 0) {  // slice 0 holds the rotated features
#pragma unroll
    for (int b = 0; b < rb; ++b) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x = qs[4 * b + e], y = qs[4 * (b + rb) + e];
        qs[4 * b + e] = rope_lo(x, y, qcs[b][e], qsn[b][e]);
        qs[4 * (b + rb) + e] = rope_hi(x, y, qcs[b][e], qsn[b][e]);
      }
    }
  }
  f32x4 *QL = reinterpret_cast<f32x4 *>(smem);
  if (prep) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const bool rotated = wave == 0 && c < 2 * rb;
      f32x4 y;
#pragma unroll
      for (int e = 0; e < 4; ++e) y[e] = q_live ? qs[4 * c + e] * (rotated ? 1.0f : 1.0f + wk[c][e]) : 0.0f;
      QL[(sw * 4 + c) * 64 + lane] = y;
    }
  }
  if (wave == 0 && col == 0) {
#pragma unroll
    for (int c = 0; c < 4; ++c) *reinterpret_cast<f32x4 *>(s_wkr + (c * 4 + grp) * 4) = wk[c] + 1.0f;
  }
  __syncthreads();
  const float c1q =
      a.c1 * rms_scale(s_ssq[col] + s_ssq[16 + col] + s_ssq[32 + col] + s_ssq[48 + col], HDP, a.eps);

  f32x4 O[4 * 2];  // O^T blocks 8 h .. 8 h + 7 (groups 2h, 2h + 1)
#pragma unroll
  for (int j = 0; j < 8; ++j) O[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float m = kNoMax, l = 0.0f;  // l: this lane's share of the row sum
  bool tainted = false;        // wave-uniform

  // Each piece is reloaded with the next tile's right after its MFMAs; at
  // the wave's last tile the "next" pieces re-read it (unconditional, so no
  // ring slot ever holds one of two values).
  for (int kt = kt_first; kt >= kt_begin; kt -= NW) {
    const int kn = kt - NW >= kt_begin ? kt - NW : kt;
    const int k0 = kt * KT;
    const bool act = k0 + col < L && s_act[k0 + col] != 0;
    f32x4 s0 = {0.0f, 0.0f, 0.0f, 0.0f}, s1 = {0.0f, 0.0f, 0.0f, 0.0f};
    float ssk = 0.0f;
    // S^T over K slices 1, 2, 3 (features past the rotated ones)
#pragma unroll
    for (int i = 0; i < 3; ++i) {
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float x = ring[i][c][e];
          ssk += x * x;
          const float y = QL[((i + 1) * 4 + c) * 64 + lane][e];
          if (c & 1)
            s1 = mfma_16x16x4(x, y, s1);
          else
            s0 = mfma_16x16x4(x, y, s0);
        }
      load_k(i, i + 1, kn);
    }
    // slice 0: sum of squares of the raw key, then x (1 + w_k) and RoPE on
    // the rotated blocks (0 .. 2 rb - 1)
    {
      f32x4(&k)[4] = ring[3];
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int e = 0; e < 4; ++e) ssk += k[c][e] * k[c][e];
#pragma unroll
      for (int c = 0; c < 4; ++c)
        if (c < 2 * rb) k[c] *= *reinterpret_cast<const f32x4 *>(s_wkr + (c * 4 + grp) * 4);
#pragma unroll
      for (int b = 0; b < rb; ++b) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float x = k[b][e], y = k[b + rb][e];
          k[b][e] = rope_lo(x, y, tcs[b][e], tsn[b][e]);
          k[b + rb][e] = rope_hi(x, y, tcs[b][e], tsn[b][e]);
        }
      }
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float y = QL[c * 64 + lane][e];
          if (c & 1)
            s1 = mfma_16x16x4(k[c][e], y, s1);
          else
            s0 = mfma_16x16x4(k[c][e], y, s0);
        }
    }
    load_k(3, 0, kn);
    load_tab(kn);
    // the key's scale (lanes col hold key col), to the S^T rows 4 grp + r
    ssk += __shfl_xor(ssk, 16);
    ssk += __shfl_xor(ssk, 32);
    const float sck = rms_scale(ssk, HDP, a.eps);
    const uint32_t abits = (uint32_t)__ballot(act && k0 + col >= start) & 0xffffu;
    const uint32_t w = q_live ? (abits & range_bits(0, q - k0)) : 0u;
    f32x4 s = s0 + s1;
#pragma unroll
    for (int r = 0; r < 4; ++r) s[r] *= c1q * __shfl(sck, 4 * grp + r);
    if (__ballot(q_live && w != 0xffffu) != 0) {
#pragma unroll
      for (int r = 0; r < 4; ++r) s[r] = ((w >> (4 * grp + r)) & 1u) ? s[r] : -INFINITY;
    }
    f32x4 ex;
    float rs = 0.0f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      ex[r] = fast_exp2(s[r] - m);
      rs += ex[r];
    }
    if (__builtin_expect(__ballot(q_live && !(rs <= kLazyLimit)) != 0, 0)) {
      const float mx = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
      const float mxs = pair_max(pair16_max(mx));
      const float mn = mxs > m + kRescaleSlack ? mxs : m;
      rs = 0.0f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        ex[r] = fast_exp2(s[r] - mn);
        rs += ex[r];
      }
      if (__ballot(q_live && !__builtin_isfinite(rs)) != 0) {
        tainted = true;
      } else {
        const float alpha = fast_exp2(m - mn);  // exactly 1 where the reference stays
#pragma unroll
        for (int j = 0; j < 8; ++j) O[j] *= alpha;
        l *= alpha;
        m = mn;
      }
    }
    l += rs;
    // P.V: the half's V groups in slots 4, 5, each reloaded after its MFMAs.
#pragma unroll
    for (int g = 0; g < 2; ++g) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          O[4 * g + j] = mfma_16x16x4(ring[4 + g][j][r], ex[r], O[4 * g + j]);
      load_v(4 + g, 2 * h + g, kn);
    }
    if (tainted) break;  // wave-uniform; the half is redone below
  }

  // -------- careful redo (rare): a wave's scores, or this half's O, went
  // non-finite; one wave redoes the tile with the reference's exact
  // semantics and stores this half's features.
  if (tid == 0) s_bad = 0;
  __syncthreads();
  bool bad = tainted;
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) bad |= q_live && !__builtin_isfinite(O[j][r]);
  if (__ballot(bad) != 0 && lane == 0) s_bad = 1;
  __syncthreads();
  if (s_bad != 0) {
    if (wave == 0)
      jeff_redo_wave<HDP, true, 2>(kernel_jeff_args(), nullptr, row, head, q0, kt_begin, kt_end,
                                   start, smem, 128 * h, 128 * h + 128);
    return;
  }

  // -------- merge: O = sum_w 2^(m_w - M) O_w / sum_w 2^(m_w - M) l_w; wave w
  // finishes O^T block 8 h + w. Every wave is past its walk (the barrier
  // above), so OM may cover the Q rows.
  f32x4 *OM = reinterpret_cast<f32x4 *>(smem);
#pragma unroll
  for (int j = 0; j < NBH; ++j) OM[(wave * NBH + j) * 64 + lane] = O[j];
  const float lt = pair_sum(pair16_sum(l));
  if (grp == 0) {
    s_m[wave * 16 + col] = m;
    s_l[wave * 16 + col] = lt;
  }
  __syncthreads();
  float M = s_m[col];
#pragma unroll
  for (int v = 1; v < NW; ++v) M = fmaxf(M, s_m[v * 16 + col]);
  float fac[NW], lsum = 0.0f;
#pragma unroll
  for (int v = 0; v < NW; ++v) {
    fac[v] = fast_exp2(s_m[v * 16 + col] - M);  // 0 for a wave without keys (m = kNoMax)
    lsum += fac[v] * s_l[v * 16 + col];
  }
  const float inv = lsum > 0.0f ? fast_rcp(lsum) : 0.0f;
  f32x4 Of = OM[wave * 64 + lane] * fac[0];
#pragma unroll
  for (int v = 1; v < NW; ++v) Of += OM[(v * NBH + wave) * 64 + lane] * fac[v];
  Of *= inv;
  finish(Of);
}

// ---------------------------------------------------------- bf16 attention

// Tile data for one 32-key bf16 tile: finished K rows from the prep workspace
// and the V columns, all as 16-byte loads with clamped indices. LDS holds K
// as [key][d] and V as [d][key] (bf16).
template <int HDP, bool VEC>
struct JeffStageBf16 {
  static constexpr int KT = 32;
  static constexpr int KTASKS = KT * HDP / 8;  // 16-byte chunks of K
  static constexpr int VTASKS = HDP * KT / 8;  // 16-byte chunks of V
  static constexpr int KN = (KTASKS + 255) / 256;
  static constexpr int VN = (VTASKS + 255) / 256;
  u16x8 k[KN], v[VN];

  __device__ __forceinline__ void fetch(const uint16_t *kp_tile, const uint16_t *V, int L, int hd,
                                        int k0, int tid) {
#pragma unroll
    for (int i = 0; i < KN; ++i) {
      const int e = min(tid + 256 * i, KTASKS - 1);
      const int kk = min(e / (HDP / 8), L - 1 - k0);
      k[i] = reinterpret_cast<const u16x8 *>(kp_tile)[kk * (HDP / 8) + e % (HDP / 8)];
    }
#pragma unroll
    for (int i = 0; i < VN; ++i) {
      const int e = min(tid + 256 * i, VTASKS - 1);
      const int d = min(e / (KT / 8), hd - 1), g = e % (KT / 8);
      const uint16_t *src = V + (size_t)L * d;
      const int key = k0 + 8 * g;
      if (VEC) {
        v[i] = *reinterpret_cast<const u16x8 *>(src + min(key, L - 8));
      } else {
#pragma unroll
        for (int t = 0; t < 8; ++t) v[i][t] = src[min(key + t, L - 1)];
      }
    }
  }

  __device__ __forceinline__ int commit(uint16_t *Ks, uint16_t *Vs, int tid, int k0, int L, int hd) {
    constexpr int KSB = HDP + 8, VSB = KT + 8;
    const u16x8 z = {0, 0, 0, 0, 0, 0, 0, 0};
    int nonfinite = 0;
#pragma unroll
    for (int i = 0; i < KN; ++i) {
      const int e = tid + 256 * i;
      const int kk = e / (HDP / 8), c = e % (HDP / 8);
      if (e < KTASKS) *reinterpret_cast<u16x8 *>(&Ks[kk * KSB + 8 * c]) = k0 + kk < L ? k[i] : z;
    }
#pragma unroll
    for (int i = 0; i < VN; ++i) {
      const int e = tid + 256 * i;
      const int d = e / (KT / 8), g = e % (KT / 8);
      if (e >= VTASKS) continue;
      u16x8 x = v[i];
      const int key = k0 + 8 * g;
      if (VEC && key + 8 > L) {  // the clamped load was shifted back: realign
        const int sh = key - (L - 8);
        u16x8 y = z;
#pragma unroll
        for (int t = 0; t < 8; ++t)
          if (t + sh < 8) y[t] = x[t + sh];
        x = y;
      }
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const bool live = d < hd && key + t < L;
        const bool fin = bf16_finite(x[t]);
        nonfinite |= live && !fin;
        x[t] = (live && fin) ? x[t] : (unsigned short)0;
      }
      *reinterpret_cast<u16x8 *>(&Vs[d * VSB + 8 * g]) = x;
    }
    return nonfinite;
  }
};

// LDS bytes of the bf16 kernel's workgroup (two K/V tiles or the Q scratch).
template <int HDP>
__host__ __device__ constexpr int jeff_bf16_smem_bytes() {
  constexpr int KT = 32, KSB = HDP + 8, VSB = KT + 8;
  constexpr int TILE_BYTES = 2 * (KT * KSB + HDP * VSB) * 2;
  constexpr int QSCR_BYTES = kWavesPerGroup * kJeffWaveQueries * (HDP + 1) * 4;
  return TILE_BYTES > QSCR_BYTES ? TILE_BYTES : QSCR_BYTES;
}

// Same arithmetic as jeff_attention_f32_kernel with q, k, v and gate in bf16:
// normalized/rotated q and k, scaled by powers of two (norm_weight_exp), are
// rounded to fp16 for S^T on v_mfma_f32_16x16x32_f16, and the probabilities
// to bf16 for P.V on v_mfma_f32_16x16x32_bf16 (V stays bf16); the row sum l
// adds the rounded probabilities; softmax, accumulation and output stay f32.
// A 32-key tile is two 16-key S^T blocks (lane group g holds keys 4g + r and
// 16 + 4g + r of its query), which together are exactly the B operand of one
// P.V MFMA per 16-row block of O^T.
// Whether jeff_bf16_wide_kernel flagged (non-finite values) a query tile of
// redo_qt queries that unit (bx, by, bz) of the bf16 grid covers, for any
// head of its group.
__device__ __forceinline__ bool jeff_bf16_unit_flagged(const JeffArgs &a, const int *redo,
                                                       int redo_qt, int bx, int by, int bz) {
  const int hg = a.heads_per_group, QT = kJeffWaveQueries * (kWavesPerGroup / hg);
  const int L = a.L, qa = bx * QT;
  const int nqt = (L + redo_qt - 1) / redo_qt;
  const int t_lo = qa / redo_qt, t_hi = (min(qa + QT, L) - 1) / redo_qt;
  int any = 0;
  for (int h = by * hg; h < by * hg + hg; ++h)
    for (int t = t_lo; t <= t_hi; ++t) any |= redo[((size_t)bz * a.heads + h) * nqt + t];
  return any != 0;
}

// One workgroup's unit (bx, by, bz) of the grid (query tile, head group,
// row); smem_raw: jeff_bf16_smem_bytes() of LDS, s_span: two ints.
template <int HDP, bool VEC>
__device__ __forceinline__ void jeff_bf16_unit(const JeffArgs &a, const uint16_t *__restrict__ kp,
                                               const int bx, const int by, const int bz,
                                               unsigned char *smem_raw, int *s_span) {
  constexpr int KT = 32;
  constexpr int QS8 = HDP / 32;  // bf16x8 B operands of Q per lane
  constexpr int NB = HDP / 16;   // 16-row blocks of O^T
  constexpr int KSB = HDP + 8, VSB = KT + 8;
  constexpr int KBUF = KT * KSB, VBUF = HDP * VSB;  // uint16 elements
  constexpr int QP = HDP + 1;
  uint16_t *const lds16 = reinterpret_cast<uint16_t *>(smem_raw);
  float *const qscr = reinterpret_cast<float *>(smem_raw);

  // The thread index goes through an opaque move: the exact pass runs units
  // in a loop, and what is derived from the index stays inside the unit
  // instead of being hoisted (and held live) across the whole loop.
  int tid;
  asm volatile("v_mov_b32 %0, %1" : "=v"(tid) : "v"((int)threadIdx.x));
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform, in a scalar register
  const int col = lane & 15, grp = lane >> 4;
  const int hg = a.heads_per_group, qsubs = kWavesPerGroup / hg;
  const int row = bz;
  const int head = by * hg + wave % hg;
  const int kvh = min(head / a.groups, a.kv_heads - 1);
  const int L = a.L, hd = a.hd, rh = a.rot_half;
  const int QT = kJeffWaveQueries * qsubs;
  const int qa = bx * QT;
  const int q = qa + (wave / hg) * kJeffWaveQueries + col;
  const bool qin = q < L;
  const float *maskr = a.mask + (size_t)row * L;
  const uint16_t *Q = static_cast<const uint16_t *>(a.q) + row * a.q_row + (size_t)head * hd * L;
  const uint16_t *Gt = static_cast<const uint16_t *>(a.gate) + row * a.q_row + (size_t)head * hd * L;
  const uint16_t *V = static_cast<const uint16_t *>(a.v) + row * a.kv_row + (size_t)kvh * a.kv_head;
  const uint16_t *KP = kp + ((size_t)row * a.kv_heads + kvh) * L * HDP;
  float *OUT = a.out + row * a.q_row + (size_t)head * hd * L;
  const bool rope = a.cos_t != nullptr && rh > 0;

  if (tid == 0) {
    s_span[0] = 0x7fffffff;
    s_span[1] = -1;
  }
  __syncthreads();
  scan_active(maskr, L, tid, lane, s_span);
  __syncthreads();
  const int first = s_span[0], last = s_span[1];
  const int start = (a.trim && last >= 0) ? first : 0;
  int kt_begin = 0, kt_end = 0;
  {
    const int kl = min(last, min(qa + QT, L) - 1);
    if (last >= 0 && first <= kl) {
      kt_begin = first / KT;
      kt_end = kl / KT + 1;
    }
  }

  // -------- Q: RMSNorm + partial RoPE in f32 (wave-local LDS phases), then
  // scaled by 2^-e_q and rounded to fp16 (the prepared keys are fp16 with
  // 2^-e_k): lane (col, grp) holds Q[q][32*s + 8*grp + e] in qb[s].
  const int eq = norm_weight_exp(a.q_norm, hd, lane);
  const float qsig = ldexpf(1.0f, -eq);
  const float c1 = ldexpf(a.c1, eq + norm_weight_exp(a.k_norm, hd, lane));
  f16x8 qb[QS8];
  const bool q_live = qin && q >= start;
  {
    float *qw = qscr + wave * (kJeffWaveQueries * QP);
    float *qs = qw + col * QP;
    constexpr int QQ = HDP / 4;
    float ss = 0.0f;
    const int qc = q_live ? q : 0;
#pragma unroll
    for (int s = 0; s < QQ; ++s) {
      const int d = grp * QQ + s;
      const float x = bf16_to_f32(Q[qc + (size_t)L * (d < hd ? d : hd - 1)]);
      const float y = (q_live && d < hd) ? x : 0.0f;
      qs[d] = y;
      ss += y * y;
    }
    ss += __shfl_xor(ss, 16);
    ss += __shfl_xor(ss, 32);
    const float scale = rms_scale(ss, hd, a.eps);
#pragma unroll 16
    for (int s = 0; s < QQ; ++s) {
      const int d = grp * QQ + s;
      const float wq = a.q_norm[min(d, hd - 1)];
      const float y = rms_apply(qs[d], scale, wq);
      qs[d] = d < hd ? y : 0.0f;
    }
    if (rope) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const int q0 = qa + (wave / hg) * kJeffWaveQueries;
      for (int e0 = 0; e0 < kJeffWaveQueries * rh; e0 += 64 * 8) {
        float c[8], sn[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int e = min(e0 + lane + 64 * u, kJeffWaveQueries * rh - 1);
          const int qi = e / rh, i = e - qi * rh;
          const int pos = min(max(q0 + qi - start, 0), L - 1);
          c[u] = a.cos_t[(size_t)pos * rh + i];
          sn[u] = a.sin_t[(size_t)pos * rh + i];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int e = e0 + lane + 64 * u;
          const int qi = e / rh, i = e - qi * rh;
          const int qq = q0 + qi;
          if (e < kJeffWaveQueries * rh && qq < L && qq >= start) {
            const float x = qw[qi * QP + i], y = qw[qi * QP + i + rh];
            qw[qi * QP + i] = rope_lo(x, y, c[u], sn[u]);
            qw[qi * QP + i + rh] = rope_hi(x, y, c[u], sn[u]);
          }
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int s = 0; s < QS8; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) qb[s][e] = (_Float16)(qs[32 * s + 8 * grp + e] * qsig);
  }
  __syncthreads();  // the Q scratch becomes the K/V buffers

  auto mask_of = [&](int kt) -> float { return maskr[min(kt * KT + (lane & 31), L - 1)]; };
  auto keep_word = [&](int kt, float mv) -> uint32_t {
    const int k0 = kt * KT;
    const int kc = k0 + (lane & 31);
    const bool act = kc < L && kc >= start && mv != 0.0f;
    const uint32_t abits = (uint32_t)__ballot(act);  // lanes 0..31 = keys of the tile
    return q_live ? (abits & range_bits(0, q - k0)) : 0u;
  };

  f32x4 O[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) O[j][r] = 0.0f;
  float m = -INFINITY, l = 0.0f;

  JeffStageBf16<HDP, VEC> st;
  int nonfinite = 0;
  uint32_t w = 0u;
  float m_next = 0.0f;
  if (kt_begin < kt_end) {
    const float m0 = mask_of(kt_begin);
    st.fetch(KP + (size_t)kt_begin * KT * HDP, V, L, hd, kt_begin * KT, tid);
    nonfinite = st.commit(lds16, lds16 + 2 * KBUF, tid, kt_begin * KT, L, hd);
    w = keep_word(kt_begin, m0);
  }
  int nf = __syncthreads_or(nonfinite);
  int any_nf = 0;

  for (int kt = kt_begin; kt < kt_end; ++kt) {
    const int cur = (kt - kt_begin) & 1;
    const bool more = kt + 1 < kt_end;
    if (more) {
      m_next = mask_of(kt + 1);
      st.fetch(KP + (size_t)(kt + 1) * KT * HDP, V, L, hd, (kt + 1) * KT, tid);
    }
    const uint16_t *Kc = lds16 + cur * KBUF;
    const uint16_t *Vc = lds16 + 2 * KBUF + cur * VBUF;

    if (__ballot(w != 0u) != 0) {
      f32x4 s0, s1;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        s0[r] = 0.0f;
        s1[r] = 0.0f;
      }
      const uint16_t *k0row = Kc + col * KSB + 8 * grp;
      const uint16_t *k1row = Kc + (16 + col) * KSB + 8 * grp;
#pragma unroll
      for (int st8 = 0; st8 < QS8; ++st8) {
        const f16x8 ka = *reinterpret_cast<const f16x8 *>(k0row + 32 * st8);
        const f16x8 kb = *reinterpret_cast<const f16x8 *>(k1row + 32 * st8);
        s0 = mfma_16x16x32_f16(ka, qb[st8], s0);
        s1 = mfma_16x16x32_f16(kb, qb[st8], s1);
      }
      // The probabilities are summed as the bf16 values P.V consumes.
      const float alpha = softmax_tile16<true>(s0, s1, w, grp, c1, m, l);
      if (alpha != 1.0f) {
#pragma unroll
        for (int j = 0; j < NB; ++j) O[j] *= alpha;
      }
      bf16x8 pb;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        pb[r] = (__bf16)s0[r];
        pb[4 + r] = (__bf16)s1[r];
      }
      // A operand of block j: V[keys 4g+0..3 and 16+4g+0..3][d = 16*j + col].
      const uint16_t *v0 = Vc + col * VSB + 4 * grp;
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const u16x4 lo = *reinterpret_cast<const u16x4 *>(v0 + j * 16 * VSB);
        const u16x4 hi = *reinterpret_cast<const u16x4 *>(v0 + j * 16 * VSB + 16);
        u16x8 vv;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          vv[e] = lo[e];
          vv[4 + e] = hi[e];
        }
        O[j] = mfma_16x16x32_bf16(__builtin_bit_cast(bf16x8, vv), pb, O[j]);
        if ((j & 7) == 7) __builtin_amdgcn_sched_barrier(0);
      }
    }
    any_nf |= nf;
    nonfinite = 0;
    if (more)
      nonfinite = st.commit(lds16 + (cur ^ 1) * KBUF, lds16 + 2 * KBUF + (cur ^ 1) * VBUF, tid,
                            (kt + 1) * KT, L, hd);
    nf = __syncthreads_or(nonfinite);
    if (more) w = keep_word(kt + 1, m_next);
  }

  // -------- non-finite values of kept keys (rare), as in the f32 kernel
  uint32_t special[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) special[j] = 0u;
  if (any_nf) {
    const int k_lo = kt_begin * KT, k_hi = min(kt_end * KT, L);
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int d = j * 16 + 4 * grp + r;
        uint32_t f = 0u;
        if (q_live && d < hd) {
#pragma nounroll
          for (int k = k_lo; k < k_hi && k <= q; ++k) {
            if (k < start || maskr[k] == 0.0f) continue;
            const float v = bf16_to_f32(V[k + (size_t)L * d]);
            if (!__builtin_isfinite(v)) f |= __builtin_isnan(v) ? 1u : (v > 0.0f ? 2u : 4u);
          }
        }
        special[j] |= f << (8 * r);
      }
  }

  float lt = l + __shfl_xor(l, 16);
  lt += __shfl_xor(lt, 32);
  const float inv = lt > 0.0f ? fast_rcp(lt) : 0.0f;
  if (qin) {
    const bool dropped = a.trim && q < start;
    f32x4 gv[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int d = j * 16 + 4 * grp + r;
        gv[j][r] = bf16_to_f32(Gt[q + (size_t)L * (d < hd ? d : hd - 1)]);
      }
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int d = j * 16 + 4 * grp + r;
        float o = O[j][r] * inv;
        const uint32_t f = (special[j] >> (8 * r)) & 7u;
        if (f) o = ((f & 1u) || f == 6u) ? __builtin_nanf("") : (f == 2u ? INFINITY : -INFINITY);
        if (d < hd)
          __builtin_nontemporal_store(dropped ? 0.0f : o * fast_sigmoid(gv[j][r]), &OUT[q + (size_t)L * d]);
      }
  }
}

template <int HDP, bool VEC>
__global__ __launch_bounds__(256, 2) void jeff_attention_bf16_kernel(const JeffArgs a,
                                                                     const uint16_t *__restrict__ kp) {
  __shared__ __attribute__((aligned(16))) unsigned char smem_raw[jeff_bf16_smem_bytes<HDP>()];
  __shared__ int s_span[2];
  jeff_bf16_unit<HDP, VEC>(a, kp, blockIdx.x, blockIdx.y, blockIdx.z, smem_raw, s_span);
}

// The exact pass after jeff_bf16_wide_kernel: the same units over a grid of
// gx x gy x gz, each run only where the wide kernel flagged one of its
// query tiles. A resident grid of workgroups walks the units (workgroup p
// takes p, p + gridDim.x, ...; the flags of up to 64 of them read in one
// round trip), so a call with nothing flagged costs one dispatch round of
// flag reads rather than a full grid of workgroups.
template <int HDP, bool VEC>
__global__ __launch_bounds__(256, 2) void jeff_bf16_exact_kernel(const JeffArgs a,
                                                                 const uint16_t *__restrict__ kp,
                                                                 const int *__restrict__ redo,
                                                                 int redo_qt, int gx, int gy,
                                                                 int gz) {
  __shared__ __attribute__((aligned(16))) unsigned char smem_raw[jeff_bf16_smem_bytes<HDP>()];
  __shared__ int s_span[2];
  const int n = gx * gy * gz, lane = threadIdx.x & 63, stride = gridDim.x;
  for (int v0 = blockIdx.x; v0 < n; v0 += 64 * stride) {
    // Lane k reads the flags of unit v0 + k*stride, all at once; every wave
    // gets the same ballot, so the loop below is uniform over the workgroup.
    const int v = v0 + lane * stride;
    const bool f = v < n && jeff_bf16_unit_flagged(a, redo, redo_qt, v % gx, (v / gx) % gy,
                                                   v / (gx * gy));
    uint64_t m = __ballot(f);
    while (m != 0) {
      const int u = v0 + (int)__builtin_ctzll(m) * stride;
      m &= m - 1;
      __syncthreads();  // the previous unit is done with the LDS
      jeff_bf16_unit<HDP, VEC>(a, kp, u % gx, (u / gx) % gy, u / (gx * gy), smem_raw, s_span);
    }
  }
}

// ----------------------------------------------------------------- launchers

// Workspace: the prepared keys (per row and kv head, keys rounded up to 16
// for the split-head kernel's padded blocks), then one (first, last) key
// span per row and the rows' active-key bits (32 keys per word).
static size_t jeff_kp_main_bytes(const JeffArgs &a, int rows, int hd_pad, bool bf16) {
  const size_t Lp = ((size_t)a.L + 15) & ~(size_t)15;
  const size_t b = (size_t)rows * a.kv_heads * Lp * hd_pad * (bf16 ? 2 : 4);
  return (b + 255) & ~(size_t)255;
}

template <int HDP>
static hipError_t launch_jeff_f32_hd(const JeffArgs &a, int rows, float *kp, hipStream_t stream,
                                     const KernelEvents &ev) {
  dim3 pgrid((a.L + kKeyTile - 1) / kKeyTile, a.kv_heads, rows);
  // Query tiles of 16 in causal pairs, kJeffF32Waves / heads_per_group tiles
  // (half as many pairs) per workgroup.
  const int nq = (a.L + kJeffWaveQueries - 1) / kJeffWaveQueries;
  const int pairs_per_group = kJeffF32Waves / a.heads_per_group / 2;
  const int npairs = (nq + 1) / 2;
  dim3 grid((npairs + pairs_per_group - 1) / pairs_per_group, a.heads / a.heads_per_group, rows);
  // 16-byte accesses along tokens need L % 4 == 0 and aligned bases; buffer
  // offsets need one head's (hd, L) block and one kv head's K rows within
  // 2 GiB.
  const uintptr_t bases = reinterpret_cast<uintptr_t>(a.q) | reinterpret_cast<uintptr_t>(a.v) |
                          reinterpret_cast<uintptr_t>(a.gate) | reinterpret_cast<uintptr_t>(a.out);
  const bool vec = a.L % 4 == 0 && (bases & 15) == 0 &&
                   ((size_t)a.L + 15) * (size_t)HDP * 4 < ((size_t)1 << 31);
  if constexpr (HDP == 256) {
    // Grids of at most two workgroups per CU (one row of C4 is 128) take
    // the fused kernel: one launch, no K prep, every query tile's key range
    // on eight wavefronts. Larger grids keep the K prep and the split-head
    // kernel, which holds four workgroups per CU (the fused kernel's 256
    // registers per wave allow two) and reads each prepared key tile with
    // 1 KB loads instead of normalizing it again for every query tile.
    const int rb = a.cos_t == nullptr ? 0 : (a.rot_half % 16 == 0 ? a.rot_half / 16 : -1);
    const long items = (long)nq * rows * a.heads;
    const bool div_ok = (uint64_t)rows * a.heads * a.heads <= ((uint64_t)1 << 32);
    // Grids of at most half the CUs (one C4 row per call) run each item as
    // two workgroups, one per half of the output features.
    if (vec && div_ok && a.hd == 256 && rb >= 0 && rb <= 2 && a.L <= kJeffHalfMaxL &&
        2 * items <= (a.cus > 0 ? a.cus : 1)) {
      const dim3 hgrid((unsigned)(rows * a.heads), (unsigned)nq, 2u);
      void (*const kern[3][2])(JeffArgs, int) = {
          {jeff_fused_half_f32_kernel<0, false>, jeff_fused_half_f32_kernel<0, true>},
          {jeff_fused_half_f32_kernel<1, false>, jeff_fused_half_f32_kernel<1, true>},
          {jeff_fused_half_f32_kernel<2, false>, jeff_fused_half_f32_kernel<2, true>}};
      hipExtLaunchKernelGGL(kern[rb][a.trim ? 1 : 0], hgrid, dim3(512), 0, stream, ev.start,
                            ev.stop, 0, a, rows);
      return hipGetLastError();
    }
    if (vec && div_ok && a.hd == 256 && rb >= 0 && rb <= 2 &&
        items <= 2L * (a.cus > 0 ? a.cus : 1)) {
      constexpr int NW = kJeffFusedWaves;
      const dim3 fgrid((unsigned)(rows * a.heads), (unsigned)nq);
      if (rb == 0)
        hipExtLaunchKernelGGL((jeff_fused_f32_kernel<NW, 0>), fgrid, dim3(NW * 64), 0, stream,
                              ev.start, ev.stop, 0, a, rows);
      else if (rb == 1)
        hipExtLaunchKernelGGL((jeff_fused_f32_kernel<NW, 1>), fgrid, dim3(NW * 64), 0, stream,
                              ev.start, ev.stop, 0, a, rows);
      else
        hipExtLaunchKernelGGL((jeff_fused_f32_kernel<NW, 2>), fgrid, dim3(NW * 64), 0, stream,
                              ev.start, ev.stop, 0, a, rows);
      return hipGetLastError();
    }
    // Buffer offsets of the split kernel: one head's (hd, L) block and one
    // kv head's padded K blocks within 2 GiB (checked above, L + 15 < 2^21).
    if (vec && div_ok) {
      int *spans = reinterpret_cast<int *>(reinterpret_cast<char *>(kp) +
                                           jeff_kp_main_bytes(a, rows, HDP, false));
      uint32_t *kbits = reinterpret_cast<uint32_t *>(spans + 2 * rows);
      const dim3 sp((a.L + 31) / 32, a.kv_heads, rows);
      hipExtLaunchKernelGGL(jeff_k_prep_split_kernel, sp, dim3(256), 0, stream, ev.start, nullptr,
                            0, a, kp, spans, kbits);
      hipError_t e = hipGetLastError();
      if (e != hipSuccess) return e;
      const dim3 sgrid(rows * a.heads, nq);
      hipExtLaunchKernelGGL((jeff_split_f32_kernel<HDP>), sgrid, dim3(256), 0, stream, nullptr,
                            ev.stop, 0, a, kp, spans, kbits, rows);
      return hipGetLastError();
    }
  }
  hipExtLaunchKernelGGL((jeff_k_prep_kernel<HDP, float>), pgrid, dim3(256), 0, stream, ev.start,
                        nullptr, 0, a, kp, nullptr);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const dim3 block(kJeffF32Waves * 64);
  if (vec)
    hipExtLaunchKernelGGL((jeff_attention_f32_kernel<HDP, true>), grid, block, 0, stream, nullptr,
                          ev.stop, 0, a, kp);
  else
    hipExtLaunchKernelGGL((jeff_attention_f32_kernel<HDP, false>), grid, block, 0, stream, nullptr,
                          ev.stop, 0, a, kp);
  return hipGetLastError();
}

hipError_t launch_jeff_attention_f32(const JeffArgs &a, int rows, int hd_pad, void *kp,
                                     hipStream_t stream, const KernelEvents &ev) {
  float *k = static_cast<float *>(kp);
  switch (hd_pad) {
    case 32: return launch_jeff_f32_hd<32>(a, rows, k, stream, ev);
    case 64: return launch_jeff_f32_hd<64>(a, rows, k, stream, ev);
    case 128: return launch_jeff_f32_hd<128>(a, rows, k, stream, ev);
    case 256: return launch_jeff_f32_hd<256>(a, rows, k, stream, ev);
    default: return hipErrorInvalidValue;
  }
}

// bf16 at head dim 256: the flags of jeff_bf16_wide_kernel follow.
size_t jeff_bf16_flags_offset(const JeffArgs &a, int rows) {
  const size_t b = jeff_kp_main_bytes(a, rows, 256, true) + (size_t)rows * 2 * sizeof(int) +
                   (size_t)rows * ((a.L + 31) / 32) * sizeof(uint32_t);
  return (b + 255) & ~(size_t)255;
}

size_t jeff_kp_bytes(const JeffArgs &a, int rows, int hd_pad, bool bf16) {
  if (bf16 && hd_pad == 256 && jeff_bf16_wide_fits(a))
    return jeff_bf16_flags_offset(a, rows) + jeff_bf16_wide_flag_count(a, rows) * sizeof(int);
  return jeff_kp_main_bytes(a, rows, hd_pad, bf16) + (size_t)rows * 2 * sizeof(int) +
         (size_t)rows * ((a.L + 31) / 32) * sizeof(uint32_t);
}

template <int HDP>
static hipError_t launch_jeff_bf16_hd(const JeffArgs &a, int rows, uint16_t *kp,
                                      hipStream_t stream, const KernelEvents &ev) {
  dim3 pgrid((a.L + kKeyTile - 1) / kKeyTile, a.kv_heads, rows);
  // The wide bf16 kernel takes the rows' active key bits from the prep.
  const bool wide = HDP == 256 && jeff_bf16_wide_fits(a);
  uint32_t *kbits =
      wide ? reinterpret_cast<uint32_t *>(reinterpret_cast<char *>(kp) +
                                          jeff_kp_main_bytes(a, rows, HDP, true) +
                                          (size_t)rows * 2 * sizeof(int))
           : nullptr;
  hipExtLaunchKernelGGL((jeff_k_prep_kernel<HDP, uint16_t>), pgrid, dim3(256), 0, stream, ev.start,
                        nullptr, 0, a, kp, kbits);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int qsubs = kWavesPerGroup / a.heads_per_group;
  const int qt = kJeffWaveQueries * qsubs;
  dim3 grid((a.L + qt - 1) / qt, a.heads / a.heads_per_group, rows);
  // 16-byte V loads along tokens need L % 8 == 0 and an aligned base.
  const bool vec = a.L % 8 == 0 && (reinterpret_cast<uintptr_t>(a.v) & 15) == 0;
  if constexpr (HDP == 256) {
    // The 32x32x16 kernel, then the exact pass over the query tiles it
    // flagged (non-finite values) on a resident grid (two workgroups per CU).
    if (jeff_bf16_wide_fits(a)) {
      int *flags = reinterpret_cast<int *>(reinterpret_cast<char *>(kp) + jeff_bf16_flags_offset(a, rows));
      e = launch_jeff_bf16_wide(a, rows, kp, kbits, flags, stream);
      if (e != hipSuccess) return e;
      const int redo_qt = jeff_bf16_wide_query_tile(a);
      const long units = (long)grid.x * grid.y * grid.z;
      const long slots = 2L * (a.cus > 0 ? a.cus : 1);
      const dim3 egrid((unsigned)(units < slots ? units : slots));
      if (vec)
        hipExtLaunchKernelGGL((jeff_bf16_exact_kernel<HDP, true>), egrid, dim3(256), 0, stream,
                              nullptr, ev.stop, 0, a, kp, flags, redo_qt, (int)grid.x,
                              (int)grid.y, (int)grid.z);
      else
        hipExtLaunchKernelGGL((jeff_bf16_exact_kernel<HDP, false>), egrid, dim3(256), 0, stream,
                              nullptr, ev.stop, 0, a, kp, flags, redo_qt, (int)grid.x,
                              (int)grid.y, (int)grid.z);
      return hipGetLastError();
    }
  }
  if (vec)
    hipExtLaunchKernelGGL((jeff_attention_bf16_kernel<HDP, true>), grid, dim3(256), 0, stream,
                          nullptr, ev.stop, 0, a, kp);
  else
    hipExtLaunchKernelGGL((jeff_attention_bf16_kernel<HDP, false>), grid, dim3(256), 0, stream,
                          nullptr, ev.stop, 0, a, kp);
  return hipGetLastError();
}

hipError_t launch_jeff_attention_bf16(const JeffArgs &a, int rows, int hd_pad, void *kp,
                                      hipStream_t stream, const KernelEvents &ev) {
  uint16_t *k = static_cast<uint16_t *>(kp);
  switch (hd_pad) {
    case 32: return launch_jeff_bf16_hd<32>(a, rows, k, stream, ev);
    case 64: return launch_jeff_bf16_hd<64>(a, rows, k, stream, ev);
    case 128: return launch_jeff_bf16_hd<128>(a, rows, k, stream, ev);
    case 256: return launch_jeff_bf16_hd<256>(a, rows, k, stream, ev);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace tfd
