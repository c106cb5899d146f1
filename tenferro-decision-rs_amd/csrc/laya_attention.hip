// Laya fused split + RoPE + masked attention on gfx950 f32 matrix cores.
//
// Arithmetic follows cpu-kernels laya_attention_block_with_workspace
// (crates/cpu-kernels/src/lib.rs:843-1156): RoPE on q and k from a host-built
// f32 table (874-888), s = (q.k) * (1/sqrt(hd)) (1124), masked softmax
// (1111-1136), out = sum p*v with p == 0 never multiplying a value (1143-1151),
// NaN for a query that keeps no key (1025-1033, 1143-1151).
//
// One workgroup = 4 wavefronts = 128 queries of one (batch, head). Each
// wavefront owns 32 queries and walks 32-key tiles:
//   S^T (32 keys x 32 queries) = K_tile * Q^T      (hd/2 MFMA 32x32x2)
//   O^T (hd x 32 queries)     += V_tile^T * P^T     (hd/32 x 16 MFMA 32x32x2)
// Computing S^T rather than S puts each lane's 16 probabilities exactly where
// the B operand of the P.V product wants them, so no shuffles sit between the
// two products. Q (rotated) stays in registers for the whole walk; K (rotated
// while staged) and V tiles go through LDS and are shared by the 4 waves.
// Key tiles outside the workgroup's key span are never visited; a wave whose
// 32 queries keep nothing in a tile skips its MFMAs.
#include "tfd_device.hpp"
#include "tfd_internal.hpp"

namespace tfd {

// ---------------------------------------------------------------- keep bits

// Packs the (L, L, B) byte keep tensor into one 32-bit word per
// (batch, key tile, query): bit j set when key 32*kt + j is kept.
__global__ __launch_bounds__(256) void laya_keep_bits_kernel(const uint8_t *__restrict__ keep,
                                                             uint32_t *__restrict__ bits, int L,
                                                             int nkt) {
  const int q = blockIdx.x * blockDim.x + threadIdx.x;
  const int kt = blockIdx.y, b = blockIdx.z;
  if (q >= L) return;
  const uint8_t *base = keep + (size_t)L * L * b + q;
  const int k0 = kt * kKeyTile;
  const int n = min(kKeyTile, L - k0);
  uint8_t v[kKeyTile];
#pragma unroll
  for (int kk = 0; kk < kKeyTile; ++kk)  // unconditional (clamped) loads: all in flight at once
    v[kk] = base[(size_t)L * (k0 + min(kk, n - 1))];
#pragma unroll
  for (int kk = 0; kk < kKeyTile; ++kk) v[kk] = kk < n ? v[kk] : 0;
  uint32_t w = 0;
#pragma unroll
  for (int kk = 0; kk < kKeyTile; ++kk) w |= (uint32_t)(v[kk] != 0) << kk;
  bits[((size_t)b * nkt + kt) * L + q] = w;
}

// ------------------------------------------------------------------ helpers

// Element dd of the head's RoPE-rotated row (lib.rs:991-1010): pairs
// (i, i + half) for i < half, x[i]*c - x[i+half]*s and x[i]*s + x[i+half]*c,
// evaluated without contraction like the reference. dd >= hd pads with 0.
__device__ __forceinline__ float rope_elem(const float *row, int dd, int hd, int half,
                                           const float *cr, const float *sr) {
#pragma clang fp contract(off)
  // Branch-free with clamped indices so that a caller's loads over many dd
  // are all issued before the first is waited on.
  const int dc = dd < hd ? dd : hd - 1;
  const float x = row[dc];
  if (cr == nullptr) return dd < hd ? x : 0.0f;
  const bool lo = dc < half, hi = !lo && dc < 2 * half;
  const int i = lo ? dc : (hi ? dc - half : 0);
  const int partner = lo ? dc + half : (hi ? dc - half : dc);
  const float y = row[partner];
  const float c = half > 0 ? cr[i] : 1.0f, s = half > 0 ? sr[i] : 0.0f;
  const float r = lo ? x * c - y * s : (hi ? y * s + x * c : x);
  return dd < hd ? r : 0.0f;
}

// ------------------------------------------------------------------ staging

// x*c - y*s and x*s + y*c elementwise, uncontracted like the reference.
__device__ __forceinline__ f32x4 rot_lo(f32x4 x, f32x4 y, f32x4 c, f32x4 s) {
#pragma clang fp contract(off)
  return x * c - y * s;
}
__device__ __forceinline__ f32x4 rot_hi(f32x4 x, f32x4 y, f32x4 c, f32x4 s) {
#pragma clang fp contract(off)
  return x * s + y * c;
}

__device__ __forceinline__ bool all_finite(f32x4 v) {
  return __builtin_isfinite(v[0]) && __builtin_isfinite(v[1]) && __builtin_isfinite(v[2]) &&
         __builtin_isfinite(v[3]);
}

// One K/V tile's global data held in registers between the prefetch (issued
// before the previous tile's products) and the LDS commit (after them).
//
// VEC (hd == HDP, hd % 8 == 0, 16-byte aligned rows): a K task is one
// (key, chunk c) with its RoPE partner chunk c + half/4 and the table chunks,
// all 16-byte loads; a V task is one (key, chunk). Otherwise (any hd) the
// commit loads and rotates element by element and the prefetch is empty.
template <int HDP, bool VEC>
struct LayaStage {
  static constexpr int KTASKS = kKeyTile * HDP / 8;
  static constexpr int VTASKS = kKeyTile * HDP / 4;
  static constexpr int KN = VEC ? (KTASKS + 255) / 256 : 1;
  static constexpr int VN = VEC ? (VTASKS + 255) / 256 : 1;
  f32x4 ka[KN], kb[KN], c[KN], s[KN];
  f32x4 v[VN];

  __device__ __forceinline__ void fetch(const LayaArgs &a, const float *xb, size_t tok, int k0,
                                        int tid) {
    if constexpr (VEC) {
      // Every load is unconditional with a clamped (in-bounds) index, so all
      // of them are in flight together; out-of-range keys are zeroed at
      // commit time.
      const int hh = a.half;
#pragma unroll
      for (int i = 0; i < KN; ++i) {
        const int task = min(tid + 256 * i, KTASKS - 1);
        const int key = min(k0 + task / (HDP / 8), a.L - 1), cp = task % (HDP / 8);
        const float *row = xb + (size_t)key * tok + a.d;
        ka[i] = *reinterpret_cast<const f32x4 *>(row + 4 * cp);
        kb[i] = *reinterpret_cast<const f32x4 *>(row + 4 * cp + hh);
        if (a.cos_t) {
          c[i] = *reinterpret_cast<const f32x4 *>(a.cos_t + (size_t)key * hh + 4 * cp);
          s[i] = *reinterpret_cast<const f32x4 *>(a.sin_t + (size_t)key * hh + 4 * cp);
        } else {
          c[i] = f32x4{1.0f, 1.0f, 1.0f, 1.0f};
          s[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
      }
#pragma unroll
      for (int i = 0; i < VN; ++i) {
        const int task = min(tid + 256 * i, VTASKS - 1);
        const int key = min(k0 + task / (HDP / 4), a.L - 1), ch = task % (HDP / 4);
        v[i] = *reinterpret_cast<const f32x4 *>(xb + (size_t)key * tok + 2 * a.d + 4 * ch);
      }
    }
  }

  // Writes the tile to LDS (K rotated); returns 1 if a V value is NaN or inf.
  __device__ __forceinline__ int commit(const LayaArgs &a, const float *xb, size_t tok, int k0,
                                        int tid, float *Ks, float *Vs) {
    constexpr int KS = HDP + 4, VS = HDP + 8;
    int nonfinite = 0;
    if constexpr (VEC) {
      const int hh = a.half;
      const bool rope = a.cos_t != nullptr;
      const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int i = 0; i < KN; ++i) {
        const int task = tid + 256 * i;
        if (task < KTASKS) {
          const int kk = task / (HDP / 8), cp = task % (HDP / 8);
          const bool live = k0 + kk < a.L;
          f32x4 lo = ka[i], hi = kb[i];
          if (rope) {
            lo = rot_lo(ka[i], kb[i], c[i], s[i]);
            hi = rot_hi(ka[i], kb[i], c[i], s[i]);
          }
          lo = live ? lo : z;
          hi = live ? hi : z;
          *reinterpret_cast<f32x4 *>(&Ks[kk * KS + 4 * cp]) = lo;
          *reinterpret_cast<f32x4 *>(&Ks[kk * KS + hh + 4 * cp]) = hi;
        }
      }
#pragma unroll
      for (int i = 0; i < VN; ++i) {
        const int task = tid + 256 * i;
        if (task < VTASKS) {
          const int kk = task / (HDP / 4), ch = task % (HDP / 4);
          const f32x4 x = k0 + kk < a.L ? v[i] : z;
          nonfinite |= !all_finite(x);
          *reinterpret_cast<f32x4 *>(&Vs[kk * VS + 4 * ch]) = x;
        }
      }
    } else {
      const int L = a.L, hd = a.hd, hh = a.half;
      const bool rope = a.cos_t != nullptr;
      for (int e = tid; e < kKeyTile * HDP; e += 256) {
        const int kk = e / HDP, dd = e % HDP;
        const int key = k0 + kk;
        float kv = 0.0f, vv = 0.0f;
        if (key < L && dd < hd) {
          const float *row = xb + (size_t)key * tok;
          const float *cr = rope ? a.cos_t + (size_t)key * hh : nullptr;
          const float *sr = rope ? a.sin_t + (size_t)key * hh : nullptr;
          kv = rope_elem(row + a.d, dd, hd, hh, cr, sr);
          vv = row[2 * a.d + dd];
          nonfinite |= !__builtin_isfinite(vv);
        }
        Ks[kk * KS + dd] = kv;
        Vs[kk * VS + dd] = vv;
      }
    }
    return nonfinite;
  }
};

// ------------------------------------------------------------------- kernel

template <int HDP, int MODE, bool VEC>
__global__ __launch_bounds__(256) void laya_attention_kernel(const LayaArgs a) {
  constexpr int KS = HDP + 4;  // K row stride (floats): 16-byte rows, conflict-free b128 reads
  constexpr int VS = HDP + 8;  // V row stride: the two lane halves read rows 4 apart
  constexpr int QS = HDP / 2;  // Q registers per lane
  constexpr int NB = HDP / 32; // 32-row blocks of O^T
  __shared__ __attribute__((aligned(16))) float Ks[2][kKeyTile * KS];
  __shared__ __attribute__((aligned(16))) float Vs[2][kKeyTile * VS];
  __shared__ int s_span[3];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 31, half = lane >> 5;
  const int head = blockIdx.y, b = blockIdx.z;
  const int L = a.L, hd = a.hd, hh = a.half, nkt = a.nkt;
  const int qg0 = blockIdx.x * kLayaGroupQueries;
  const int q = qg0 + wave * kWaveQueries + col;
  const bool qin = q < L;
  const size_t tok = 3 * (size_t)a.d;
  const float *xb = a.qkv + (size_t)b * L * tok + (size_t)head * hd;
  const bool rope = a.cos_t != nullptr;

  // -------- key span of the workgroup
  if (tid == 0) {
    s_span[0] = 0x7fffffff;
    s_span[1] = -1;
    s_span[2] = 0;
  }
  __syncthreads();
  if (MODE == kMaskBits) {
    int lo = 0x7fffffff, hi = -1;
    for (int i0 = 0; i0 < kLayaGroupQueries * nkt; i0 += 256 * 8) {
      uint32_t word[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {  // 8 loads in flight per thread
        const int i = i0 + tid + 256 * u;
        const int qq = qg0 + (i & (kLayaGroupQueries - 1));
        const int kt = i / kLayaGroupQueries;
        const bool ok = i < kLayaGroupQueries * nkt && qq < L;
        const uint32_t x = a.bits[((size_t)b * nkt + min(kt, nkt - 1)) * L + min(qq, L - 1)];
        word[u] = ok ? x : 0u;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int kt = (i0 + tid + 256 * u) / kLayaGroupQueries;
        if (word[u] != 0u) {
          lo = min(lo, kt);
          hi = max(hi, kt);
        }
      }
    }
    lo = wave_min(lo);
    hi = wave_max(hi);
    if (lane == 0) {
      atomicMin(&s_span[0], lo);
      atomicMax(&s_span[1], hi);
    }
  } else {
    const uint8_t *vb = a.valid + (size_t)b * L;
    int lo = 0x7fffffff, hi = -1, padded = 0;
    for (int k0 = 0; k0 < L; k0 += 256 * 8) {
      uint8_t v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int k = k0 + tid + 256 * u;
        const uint8_t x = vb[min(k, L - 1)];
        v[u] = k < L ? x : 0;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int k = k0 + tid + 256 * u;
        if (v[u]) {
          lo = min(lo, k);
          hi = max(hi, k);
        }
      }
    }
    if (tid < kLayaGroupQueries) {
      const int qq = qg0 + tid;
      padded = (qq < L && !vb[qq]) ? 1 : 0;
    }
    lo = wave_min(lo);
    hi = wave_max(hi);
    padded = wave_max(padded);
    if (lane == 0) {
      atomicMin(&s_span[0], lo);
      atomicMax(&s_span[1], hi);
      atomicMax(&s_span[2], padded);
    }
  }
  __syncthreads();
  int kt_begin = 0, kt_end = 0;
  if (MODE == kMaskBits) {
    if (s_span[1] >= 0) {
      kt_begin = s_span[0];
      kt_end = s_span[1] + 1;
    }
  } else {
    int kf = s_span[0], kl = s_span[1];
    // A padded query keeps every valid key (build_mask), so only a tile of
    // valid queries narrows to the window.
    if (a.window >= 0 && s_span[2] == 0 && kl >= 0) {
      kf = max(kf, qg0 - a.window);
      kl = min(kl, min(qg0 + kLayaGroupQueries - 1, L - 1) + a.window);
    }
    if (kl >= 0 && kf <= kl) {
      kt_begin = kf / kKeyTile;
      kt_end = kl / kKeyTile + 1;
    }
  }

  // -------- Q: rotated, in registers. Lane (col, half) holds
  // Q[q][half*QS + s] for s < QS, the B operand of step s.
  float qreg[QS];
  {
    const int qq = qin ? q : 0;
    const float *row = xb + (size_t)qq * tok;
    if constexpr (VEC) {
      // hd == HDP: this lane's half of the row and its RoPE partner half are
      // the two halves of the row; 16-byte loads, all in flight together.
      f32x4 lo[QS / 4], hi[QS / 4], cs[QS / 4], sn[QS / 4];
#pragma unroll
      for (int c = 0; c < QS / 4; ++c) {
        lo[c] = reinterpret_cast<const f32x4 *>(row)[c];
        hi[c] = reinterpret_cast<const f32x4 *>(row + QS)[c];
        cs[c] = f32x4{1.0f, 1.0f, 1.0f, 1.0f};
        sn[c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        if (rope) {
          cs[c] = reinterpret_cast<const f32x4 *>(a.cos_t + (size_t)qq * hh)[c];
          sn[c] = reinterpret_cast<const f32x4 *>(a.sin_t + (size_t)qq * hh)[c];
        }
      }
#pragma unroll
      for (int c = 0; c < QS / 4; ++c) {
        f32x4 v = half ? hi[c] : lo[c];
        if (rope) v = half ? rot_hi(lo[c], hi[c], cs[c], sn[c]) : rot_lo(lo[c], hi[c], cs[c], sn[c]);
#pragma unroll
        for (int e = 0; e < 4; ++e) qreg[4 * c + e] = qin ? v[e] : 0.0f;
      }
    } else {
      const float *cr = rope ? a.cos_t + (size_t)qq * hh : nullptr;
      const float *sr = rope ? a.sin_t + (size_t)qq * hh : nullptr;
#pragma unroll
      for (int s = 0; s < QS; ++s)
        qreg[s] = qin ? rope_elem(row, half * QS + s, hd, hh, cr, sr) : 0.0f;
    }
  }
  bool q_valid = false;
  if (MODE == kMaskStruct) {
    const uint8_t x = a.valid[(size_t)b * L + min(q, L - 1)];
    q_valid = qin && x != 0;
  }

  // This lane's keep word for key tile kt (bit j: key 32*kt + j). The raw
  // word or validity byte is fetched one tile ahead (mask_of) and turned into
  // the word (keep_word) only when the tile comes up, so waiting on it never
  // stalls the tile prefetch issued beside it.
  auto mask_of = [&](int kt) -> uint32_t {
    if (MODE == kMaskBits) return a.bits[((size_t)b * nkt + kt) * L + min(q, L - 1)];
    return a.valid[(size_t)b * L + min(kt * kKeyTile + col, L - 1)];
  };
  auto keep_word = [&](int kt, uint32_t x) -> uint32_t {
    uint32_t w = 0u;
    if (MODE == kMaskBits) {
      w = qin ? x : 0u;
    } else {
      const int k0 = kt * kKeyTile;
      const int key = k0 + col;
      const bool kv = key < L && x != 0;
      const uint32_t vbits = (uint32_t)__ballot(kv);  // lanes 0..31 = keys of the tile
      if (qin) {
        w = vbits;
        if (a.window >= 0 && q_valid) w &= range_bits(q - a.window - k0, q + a.window - k0);
      }
    }
    return w;
  };

  f32x16 O[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) O[j][r] = 0.0f;
  float m = -INFINITY, l = 0.0f;

  // -------- software pipeline: tile kt+1 is fetched into registers before
  // the products of tile kt and committed to the other LDS buffer after
  // them; one barrier per tile.
  LayaStage<HDP, VEC> st;
  int nonfinite = 0;
  uint32_t w = 0u;
  uint32_t m_next = 0u;
  if (kt_begin < kt_end) {
    const uint32_t m0 = mask_of(kt_begin);
    st.fetch(a, xb, tok, kt_begin * kKeyTile, tid);
    nonfinite = st.commit(a, xb, tok, kt_begin * kKeyTile, tid, Ks[0], Vs[0]);
    w = keep_word(kt_begin, m0);
  }
  int nf = __syncthreads_or(nonfinite);

  for (int kt = kt_begin; kt < kt_end; ++kt) {
    const int cur = (kt - kt_begin) & 1;
    const bool more = kt + 1 < kt_end;
    if (more) {
      m_next = mask_of(kt + 1);
      st.fetch(a, xb, tok, (kt + 1) * kKeyTile, tid);
    }
    const float *Kc = Ks[cur];
    const float *Vc = Vs[cur];

    if (__ballot(w != 0u) != 0) {  // wave-uniform: skip tiles this wave never keeps
      f32x16 s;
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = 0.0f;
      const f32x4 *krow = reinterpret_cast<const f32x4 *>(&Kc[col * KS + half * QS]);
#pragma unroll
      for (int c = 0; c < QS / 4; ++c) {
        const f32x4 kv = krow[c];
        s = mfma_32x32x2(kv[0], qreg[4 * c + 0], s);
        s = mfma_32x32x2(kv[1], qreg[4 * c + 1], s);
        s = mfma_32x32x2(kv[2], qreg[4 * c + 2], s);
        s = mfma_32x32x2(kv[3], qreg[4 * c + 3], s);
      }
      const float alpha = softmax_tile(s, w, half, a.c1, m, l);
      if (alpha != 1.0f) {
#pragma unroll
        for (int j = 0; j < NB; ++j) O[j] *= alpha;
      }
      if (!nf) {
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            O[j] = mfma_32x32x2(Vc[acc_row(r, half) * VS + j * 32 + col], s[r], O[j]);
      } else {
        // A value in this tile is NaN or infinite: accumulate key by key and
        // skip zero probabilities, as the reference's scalar path does
        // (lib.rs:1143-1151), so a masked non-finite value never leaks.
        for (int kk = 0; kk < kKeyTile; ++kk) {
          const float p = tile_prob(s, kk, col);
          if (p == 0.0f) continue;
#pragma unroll
          for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) O[j][r] += p * Vc[kk * VS + j * 32 + acc_row(r, half)];
        }
      }
    }
    nonfinite = 0;
    if (more) nonfinite = st.commit(a, xb, tok, (kt + 1) * kKeyTile, tid, Ks[cur ^ 1], Vs[cur ^ 1]);
    nf = __syncthreads_or(nonfinite);
    if (more) w = keep_word(kt + 1, m_next);
  }

  // -------- normalize and store: out[feat + d + hidden*(q + L*b)]
  // 0/0 gives NaN for a query that kept nothing, as the reference does.
  const float lt = l + __shfl_xor(l, 32);
  const float inv = lt > 0.0f ? fast_rcp(lt) : __builtin_nanf("");
  if (qin) {
    float *orow = a.out + ((size_t)b * L + q) * a.d + (size_t)head * hd;
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int dd = j * 32 + acc_row(r, half);
        if (dd < hd) orow[dd] = O[j][r] * inv;
      }
  }
}

// Writes zeros (a kernel rather than a memset, so callers may capture it in a
// graph).
__global__ __launch_bounds__(256) void fill_zero_kernel(float *__restrict__ out, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    out[i] = 0.0f;
}

// ----------------------------------------------------------------- launchers

hipError_t launch_fill_zero(float *out, size_t n, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  size_t blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, out, n);
  return hipGetLastError();
}

hipError_t launch_laya_keep_bits(const uint8_t *keep, uint32_t *bits, int L, int B, int nkt,
                                 hipStream_t stream) {
  dim3 grid((L + 255) / 256, nkt, B);
  hipLaunchKernelGGL(laya_keep_bits_kernel, grid, dim3(256), 0, stream, keep, bits, L, nkt);
  return hipGetLastError();
}

template <int HDP, bool VEC>
static hipError_t launch_laya_hd(const LayaArgs &a, int heads, int batch, int mode,
                                 hipStream_t stream) {
  dim3 grid((a.L + kLayaGroupQueries - 1) / kLayaGroupQueries, heads, batch);
  if (mode == kMaskBits)
    hipLaunchKernelGGL((laya_attention_kernel<HDP, kMaskBits, VEC>), grid, dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL((laya_attention_kernel<HDP, kMaskStruct, VEC>), grid, dim3(256), 0, stream,
                       a);
  return hipGetLastError();
}

template <int HDP>
static hipError_t launch_laya_pick(const LayaArgs &a, int heads, int batch, int mode,
                                   hipStream_t stream) {
  // 16-byte row loads need hd == HDP, hd % 8 == 0 (RoPE halves in whole
  // chunks), a row stride of whole chunks and an aligned base.
  const bool vec = a.hd == HDP && a.hd % 8 == 0 && a.d % 4 == 0 &&
                   (reinterpret_cast<uintptr_t>(a.qkv) & 15) == 0;
  return vec ? launch_laya_hd<HDP, true>(a, heads, batch, mode, stream)
             : launch_laya_hd<HDP, false>(a, heads, batch, mode, stream);
}

hipError_t launch_laya_attention(const LayaArgs &a, int heads, int batch, int hd_pad, int mode,
                                 hipStream_t stream) {
  switch (hd_pad) {
    case 32: return launch_laya_pick<32>(a, heads, batch, mode, stream);
    case 64: return launch_laya_pick<64>(a, heads, batch, mode, stream);
    case 128: return launch_laya_pick<128>(a, heads, batch, mode, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace tfd
