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
// (batch, key tile, query): bit j set when key 32*kt + j is kept. Also
// writes the tile map: byte (b*nkt + kt)*ng + g is 1 when any of queries
// 64g..64g+63 keeps a key of tile kt (ng = ceil(L/64)), from which the
// attention workgroups read their key spans.
__global__ __launch_bounds__(256) void laya_keep_bits_kernel(const uint8_t *__restrict__ keep,
                                                             uint32_t *__restrict__ bits,
                                                             uint8_t *__restrict__ any, int L,
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
  // A wave is 64 consecutive queries starting at a multiple of 64; its lane
  // 0 is active whenever the wave is.
  const bool some = __ballot(w != 0u) != 0;
  if ((threadIdx.x & 63) == 0) any[((size_t)b * nkt + kt) * ((L + 63) / 64) + q / 64] = some;
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
// at the top of a step) and the LDS commit (interleaved with that step's P.V
// products).
//
// VEC (hd == HDP, hd % 8 == 0, 16-byte aligned rows): a K task is one
// (key, chunk c) with its RoPE partner chunk c + half/4 (and, with ROPE, the
// table chunks), all 16-byte loads; a V task is one (key, chunk). Otherwise
// (any hd) the commit loads and rotates element by element and the prefetch
// is empty.
template <int HDP, bool VEC, bool ROPE>
struct LayaStage {
  static constexpr int KTASKS = kKeyTile * HDP / 8;
  static constexpr int VTASKS = kKeyTile * HDP / 4;
  static constexpr int KN = VEC ? (KTASKS + 255) / 256 : 1;
  static constexpr int VN = VEC ? (VTASKS + 255) / 256 : 1;
  static constexpr int CN = ROPE ? KN : 1;
  f32x4 ka[KN], kb[KN], c[CN], s[CN];
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
        if constexpr (ROPE) {
          c[i] = *reinterpret_cast<const f32x4 *>(a.cos_t + (size_t)key * hh + 4 * cp);
          s[i] = *reinterpret_cast<const f32x4 *>(a.sin_t + (size_t)key * hh + 4 * cp);
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

  // The VEC commit in pieces a caller can spread between other work:
  // pieces [0, 2*KN) write K chunks (even: the low half of task i/2, odd:
  // the high half), pieces [2*KN, 2*KN + VN) write V chunks. Each returns 1
  // if it wrote a NaN or infinite V value.
  static constexpr int PIECES = 2 * KN + VN;
  __device__ __forceinline__ int commit_piece(int piece, const LayaArgs &a, int k0, int tid,
                                              float *Ks, float *Vs) {
    constexpr int KS = HDP + 4, VS = HDP + 8;
    const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
    if (piece < 2 * KN) {
      const int i = piece / 2;
      const int task = tid + 256 * i;
      if (KTASKS % 256 == 0 || task < KTASKS) {
        const int kk = task / (HDP / 8), cp = task % (HDP / 8);
        const bool live = k0 + kk < a.L;
        f32x4 x;
        if (piece % 2 == 0) {
          x = ka[i];
          if constexpr (ROPE) x = rot_lo(ka[i], kb[i], c[i], s[i]);
        } else {
          x = kb[i];
          if constexpr (ROPE) x = rot_hi(ka[i], kb[i], c[i], s[i]);
        }
        x = live ? x : z;
        *reinterpret_cast<f32x4 *>(&Ks[kk * KS + (piece % 2) * a.half + 4 * cp]) = x;
      }
      return 0;
    }
    const int i = piece - 2 * KN;
    const int task = tid + 256 * i;
    int nonfinite = 0;
    if (VTASKS % 256 == 0 || task < VTASKS) {
      const int kk = task / (HDP / 4), ch = task % (HDP / 4);
      const f32x4 x = k0 + kk < a.L ? v[i] : z;
      nonfinite = !all_finite(x);
      *reinterpret_cast<f32x4 *>(&Vs[kk * VS + 4 * ch]) = x;
    }
    return nonfinite;
  }

  // Writes the tile to LDS (K rotated); returns 1 if a V value is NaN or inf.
  __device__ __forceinline__ int commit(const LayaArgs &a, const float *xb, size_t tok, int k0,
                                        int tid, float *Ks, float *Vs) {
    constexpr int KS = HDP + 4, VS = HDP + 8;
    int nonfinite = 0;
    if constexpr (VEC) {
      const int hh = a.half;
      const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int i = 0; i < KN; ++i) {
        const int task = tid + 256 * i;
        if (KTASKS % 256 == 0 || task < KTASKS) {  // blockDim is 256
          const int kk = task / (HDP / 8), cp = task % (HDP / 8);
          const bool live = k0 + kk < a.L;
          f32x4 lo = ka[i], hi = kb[i];
          if constexpr (ROPE) {
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
        if (VTASKS % 256 == 0 || task < VTASKS) {
          const int kk = task / (HDP / 4), ch = task % (HDP / 4);
          const f32x4 x = k0 + kk < a.L ? v[i] : z;
          nonfinite |= !all_finite(x);
          *reinterpret_cast<f32x4 *>(&Vs[kk * VS + 4 * ch]) = x;
        }
      }
    } else {
      const int L = a.L, hd = a.hd, hh = a.half;
      for (int e = tid; e < kKeyTile * HDP; e += 256) {
        const int kk = e / HDP, dd = e % HDP;
        const int key = k0 + kk;
        float kv = 0.0f, vv = 0.0f;
        if (key < L && dd < hd) {
          const float *row = xb + (size_t)key * tok;
          const float *cr = ROPE ? a.cos_t + (size_t)key * hh : nullptr;
          const float *sr = ROPE ? a.sin_t + (size_t)key * hh : nullptr;
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

// Output of the fast softmax step on one S^T tile (see the kernel).
struct LayaSoft {
  f32x16 p;
  float rs, mn;
  bool need;
};

// ------------------------------------------------------------------- kernel

// Scheduling hints for one straight-line block: `n` repeats of one MFMA
// followed by up to `v` VALU instructions (the compiler fills what exists).
template <int n, int v>
__device__ __forceinline__ void interleave_mfma_valu() {
#pragma unroll
  for (int i = 0; i < n; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x002, v, 0);
  }
}

template <int HDP, int MODE, bool VEC, bool ROPE>
__global__ __launch_bounds__(256, 2) void laya_attention_kernel(const LayaArgs a) {
  constexpr int KS = HDP + 4;  // K row stride (floats): 16-byte rows, conflict-free b128 reads
  constexpr int VS = HDP + 8;  // V row stride: the two lane halves read rows 4 apart
  constexpr int QS = HDP / 2;  // Q registers per lane
  constexpr int NB = HDP / 32; // 32-row blocks of O^T
  constexpr int GQ = kLayaGroupQueries;
  constexpr int NBUF = 3;      // tiles t (V read), t+1 (K read), t+2 (being written)
  __shared__ __attribute__((aligned(16))) float Ks[NBUF][kKeyTile * KS];
  __shared__ __attribute__((aligned(16))) float Vs[NBUF][kKeyTile * VS];
  __shared__ int s_nf[NBUF][kWavesPerGroup];  // per-wave non-finite V flags, by buffer

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 31, half = lane >> 5;
  const int head = blockIdx.y, b = blockIdx.z;
  const int L = a.L, hd = a.hd, hh = a.half, nkt = a.nkt;
  const int qg0 = blockIdx.x * GQ;
  const int q = qg0 + wave * kWaveQueries + col;
  const bool qin = q < L;
  const size_t tok = 3 * (size_t)a.d;
  const float *xb = a.qkv + (size_t)b * L * tok + (size_t)head * hd;

  // -------- Q: rotated, in registers. Lane (col, half) holds
  // Q[q][half*QS + s] for s < QS, the B operand of step s. The loads are
  // issued first so that they overlap the span scan.
  float qreg[QS];
  f32x4 qlo[VEC ? QS / 4 : 1], qhi[VEC ? QS / 4 : 1], qcs[VEC && ROPE ? QS / 4 : 1],
      qsn[VEC && ROPE ? QS / 4 : 1];
  const int qq = qin ? q : 0;
  if constexpr (VEC) {
    // hd == HDP: this lane's half of the row and its RoPE partner half are
    // the two halves of the row; 16-byte loads, all in flight together.
    const float *row = xb + (size_t)qq * tok;
#pragma unroll
    for (int c = 0; c < QS / 4; ++c) {
      qlo[c] = reinterpret_cast<const f32x4 *>(row)[c];
      qhi[c] = reinterpret_cast<const f32x4 *>(row + QS)[c];
      if constexpr (ROPE) {
        qcs[c] = reinterpret_cast<const f32x4 *>(a.cos_t + (size_t)qq * hh)[c];
        qsn[c] = reinterpret_cast<const f32x4 *>(a.sin_t + (size_t)qq * hh)[c];
      }
    }
  }

  // -------- key span of the workgroup, computed by every wave on its own
  // (identical results, no barrier): the tiles [kt_begin, kt_end) that hold
  // a key some query of the workgroup may keep. It may be a superset; a wave
  // skips the products of tiles its queries keep nothing of.
  int kt_begin = 0, kt_end = 0;
  if (MODE == kMaskBits) {
    const int ng = (L + 63) / 64, g0 = qg0 / 64;
    const uint8_t *anyb = a.any + (size_t)b * nkt * ng;
    int lo = 0x7fffffff, hi = -1;
    for (int k0 = 0; k0 < nkt; k0 += 64 * 4) {
      uint8_t f[4][GQ / 64];
#pragma unroll
      for (int u = 0; u < 4; ++u)  // clamped loads, all in flight together
#pragma unroll
        for (int g = 0; g < GQ / 64; ++g)
          f[u][g] = anyb[(size_t)min(k0 + lane + 64 * u, nkt - 1) * ng + min(g0 + g, ng - 1)];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int kt = k0 + lane + 64 * u;
        bool some = false;
#pragma unroll
        for (int g = 0; g < GQ / 64; ++g) some |= g0 + g < ng && f[u][g] != 0;
        if (kt < nkt && some) {
          lo = min(lo, kt);
          hi = max(hi, kt);
        }
      }
    }
    lo = wave_min(lo);
    hi = wave_max(hi);
    if (hi >= 0) {
      kt_begin = lo;
      kt_end = hi + 1;
    }
  } else {
    // build_mask (laya-infer model.rs:465-490): a valid query keeps the
    // valid keys of its window, a padded query every valid key. With a
    // window and no padded query in the group the window bounds the span;
    // otherwise it runs from the first to the last valid key of the row.
    const uint8_t *vb = a.valid + (size_t)b * L;
    int padded = 0;
#pragma unroll
    for (int u = 0; u < GQ / 64; ++u) {
      const int qx = qg0 + lane + 64 * u;
      const uint8_t x = vb[min(qx, L - 1)];
      padded |= qx < L && x == 0;
    }
    padded = __ballot(padded) != 0;
    int kf = 0, kl = -1;
    if (a.window >= 0 && !padded) {
      kf = max(0, qg0 - a.window);
      kl = min(L - 1, min(qg0 + GQ - 1, L - 1) + a.window);
    } else {
      int lo = 0x7fffffff, hi = -1;
      for (int k0 = 0; k0 < L; k0 += 64 * 8) {
        uint8_t v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = vb[min(k0 + lane + 64 * u, L - 1)];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int k = k0 + lane + 64 * u;
          if (k < L && v[u]) {
            lo = min(lo, k);
            hi = max(hi, k);
          }
        }
      }
      kf = wave_min(lo);
      kl = wave_max(hi);
    }
    if (kl >= 0 && kf <= kl) {
      kt_begin = kf / kKeyTile;
      kt_end = kl / kKeyTile + 1;
    }
  }

  if constexpr (VEC) {
#pragma unroll
    for (int c = 0; c < QS / 4; ++c) {
      f32x4 v = half ? qhi[c] : qlo[c];
      if constexpr (ROPE)
        v = half ? rot_hi(qlo[c], qhi[c], qcs[c], qsn[c]) : rot_lo(qlo[c], qhi[c], qcs[c], qsn[c]);
#pragma unroll
      for (int e = 0; e < 4; ++e) qreg[4 * c + e] = qin ? v[e] : 0.0f;
    }
  } else {
    const float *row = xb + (size_t)qq * tok;
    const float *cr = ROPE ? a.cos_t + (size_t)qq * hh : nullptr;
    const float *sr = ROPE ? a.sin_t + (size_t)qq * hh : nullptr;
#pragma unroll
    for (int s = 0; s < QS; ++s)
      qreg[s] = qin ? rope_elem(row, half * QS + s, hd, hh, cr, sr) : 0.0f;
  }
  bool q_valid = false;
  if (MODE == kMaskStruct) {
    const uint8_t x = a.valid[(size_t)b * L + min(q, L - 1)];
    q_valid = qin && x != 0;
  }

  // This lane's keep word for key tile kt (bit j: key 32*kt + j); 0 past the
  // span. The raw word or validity byte is fetched two tiles ahead (mask_of)
  // and turned into the word (keep_word) only after that step's barrier, so
  // waiting on it never stalls the tile prefetch issued beside it.
  auto mask_of = [&](int kt) -> uint32_t {
    if (MODE == kMaskBits)
      return a.bits[((size_t)b * nkt + min(kt, nkt - 1)) * L + min(q, L - 1)];
    return a.valid[(size_t)b * L + min(kt * kKeyTile + col, L - 1)];
  };
  auto keep_word = [&](int kt, uint32_t x) -> uint32_t {
    uint32_t w = 0u;
    if (kt >= kt_end) return 0u;
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
  float m = kNoMax, l = 0.0f;
  const float c1 = a.c1;

  // S^T of one staged tile: K rows from LDS against the Q registers.
  auto scores = [&](const float *Kc) {
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
    return s;
  };
  auto pv = [&](const float *Vc, const f32x16 &p) {
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        O[j] = mfma_32x32x2(Vc[acc_row(r, half) * VS + j * 32 + col], p[r], O[j]);
  };

  // -------- software pipeline over three LDS buffers. Step t: prefetch tile
  // t+2 into registers; S(t+1) on the matrix cores while the vector ALUs run
  // the softmax of S(t); P(t).V(t) on the matrix cores while tile t+2 is
  // committed to LDS; one barrier. Whether a wave staged a NaN or infinite
  // value travels in s_nf[buffer][wave].
  const int nt = kt_end - kt_begin;
  LayaStage<HDP, VEC, ROPE> st;
  auto publish = [&](int slot, int nonfin) {
    const int wnf = __ballot(nonfin) != 0;
    if (lane == 0) s_nf[slot][wave] = wnf;
  };
  auto read_nf = [&](int slot) {
    int f = 0;
#pragma unroll
    for (int i = 0; i < kWavesPerGroup; ++i) f |= s_nf[slot][i];
    return f;
  };
  uint32_t w0 = 0u, w1 = 0u;  // keep words of tiles t and t+1
  int nf0 = 0, nf1 = 0;       // non-finite values in tiles t and t+1
  {
    LayaStage<HDP, VEC, ROPE> st1;
    uint32_t x0 = 0u, x1 = 0u;
    if (nt > 0) {
      x0 = mask_of(kt_begin);
      st.fetch(a, xb, tok, kt_begin * kKeyTile, tid);
    }
    if (nt > 1) {
      x1 = mask_of(kt_begin + 1);
      st1.fetch(a, xb, tok, (kt_begin + 1) * kKeyTile, tid);
    }
    int f0 = 0, f1 = 0;
    if (nt > 0) f0 = st.commit(a, xb, tok, kt_begin * kKeyTile, tid, Ks[0], Vs[0]);
    if (nt > 1) f1 = st1.commit(a, xb, tok, (kt_begin + 1) * kKeyTile, tid, Ks[1], Vs[1]);
    publish(0, f0);
    publish(1, f1);
    __syncthreads();
    nf0 = read_nf(0);
    nf1 = read_nf(1);
    if (nt > 0) w0 = keep_word(kt_begin, x0);
    if (nt > 1) w1 = keep_word(kt_begin + 1, x1);
  }

  f32x16 s_cur;
#pragma unroll
  for (int r = 0; r < 16; ++r) s_cur[r] = 0.0f;
  if (nt > 0 && __ballot(w0 != 0u) != 0) s_cur = scores(Ks[0]);

  // Fast walk: finite scores and values. Its only accumulator updates are
  // the P.V products and a wave-uniform rescale. A wave leaves it (without
  // touching O, m or l) at the first tile with a non-finite kept score or
  // value and finishes in the careful walk below; both walks commit the same
  // tiles and run the same barriers, so waves may be in different walks.
  int t = 0, cb = 0;
  uint32_t m2 = 0u;
  for (; t < nt; ++t) {
    if (nf0) break;  // workgroup-uniform
    const int nb = cb == NBUF - 1 ? 0 : cb + 1, fb = nb == NBUF - 1 ? 0 : nb + 1;
    const bool more1 = t + 1 < nt, more2 = t + 2 < nt;
    if (more2) {
      m2 = mask_of(kt_begin + t + 2);
      st.fetch(a, xb, tok, (kt_begin + t + 2) * kKeyTile, tid);
    }
    const bool act = __ballot(w0 != 0u) != 0;            // wave-uniform
    const bool act1 = more1 && __ballot(w1 != 0u) != 0;  // wave-uniform
    LayaSoft so;
    if (act) {
      if (__ballot(qin && w0 != 0xffffffffu) != 0) {
        // A tile some query of the wave keeps only in part: mask it.
#pragma unroll
        for (int r = 0; r < 16; ++r)
          s_cur[r] = ((w0 >> acc_row(r, half)) & 1u) ? s_cur[r] : -INFINITY;
      }
      // The tile max and the exponent reference, ahead of the fused block
      // (the cross-lane swap would otherwise fence the exponentials off from
      // the MFMAs they are meant to overlap).
      float mx = s_cur[0];
#pragma unroll
      for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s_cur[r]);
      const float mxs = pair_max(mx) * c1;
      so.need = mxs > m + kRescaleSlack;
      so.mn = so.need ? mxs : m;
    }
    f32x16 s_nx;
    if (act && act1) {
      // S(t+1) interleaved with the exponentials of S(t), in a fixed order
      // (sched_barrier fences): each MFMA is followed by its share of the
      // vector work, which runs while the matrix core is busy; the K operand
      // for the next 4 MFMAs is read one group ahead.
      so.rs = 0.0f;
#pragma unroll
      for (int r = 0; r < 16; ++r) s_nx[r] = 0.0f;
      const f32x4 *krow = reinterpret_cast<const f32x4 *>(&Ks[nb][col * KS + half * QS]);
      constexpr int STEP = QS / 16;  // MFMAs per exponential
      f32x4 kv = krow[0];
#pragma unroll
      for (int c = 0; c < QS / 4; ++c) {
        const f32x4 kvn = krow[c + 1 < QS / 4 ? c + 1 : c];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int k = 4 * c + i;
          s_nx = mfma_32x32x2(kv[i], qreg[k], s_nx);
          if (k % STEP == 0) {
            const int r = k / STEP;
            so.p[r] = fast_exp2(__builtin_fmaf(s_cur[r], c1, -so.mn));
            so.rs += so.p[r];
          }
          __builtin_amdgcn_sched_barrier(0);
        }
        kv = kvn;
      }
    } else if (act) {
      so.rs = 0.0f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        so.p[r] = fast_exp2(__builtin_fmaf(s_cur[r], c1, -so.mn));
        so.rs += so.p[r];
      }
    } else if (act1) {
      s_nx = scores(Ks[nb]);
    }
    if (act) {
      if (__ballot(!__builtin_isfinite(so.rs)) != 0) break;
      if (__ballot(so.need) != 0) {
        const float alpha = fast_exp2(m - so.mn);  // exactly 1 where the reference stays
#pragma unroll
        for (int j = 0; j < NB; ++j) O[j] *= alpha;
        l *= alpha;
      }
      l += so.rs;
      m = so.mn;
    }
    int f2 = 0;
    if (act && more2) {
      if constexpr (VEC) {
        // P(t).V(t) with the commit of tile t+2 spread over its first MFMAs
        // (fixed order, as above); the two O^T blocks alternate so that
        // consecutive MFMAs are independent, and each V operand is read four
        // MFMAs ahead.
        const float *Vc = Vs[cb];
        const int k2 = (kt_begin + t + 2) * kKeyTile;
        constexpr int NM = NB * 16;
        constexpr int NP = LayaStage<HDP, VEC, ROPE>::PIECES;
        constexpr int PSTEP = NM / NP >= 2 ? 2 : 1;
        auto vop = [&](int idx) {
          return Vc[acc_row(idx / NB, half) * VS + (idx % NB) * 32 + col];
        };
        float vq[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) vq[i] = vop(i);
#pragma unroll
        for (int idx = 0; idx < NM; ++idx) {
          const float vcur = vq[idx % 4];
          if (idx + 4 < NM) vq[idx % 4] = vop(idx + 4);
          O[idx % NB] = mfma_32x32x2(vcur, so.p[idx / NB], O[idx % NB]);
          if (idx % PSTEP == 0 && idx / PSTEP < NP)
            f2 |= st.commit_piece(idx / PSTEP, a, k2, tid, Ks[fb], Vs[fb]);
          __builtin_amdgcn_sched_barrier(0);
        }
      } else {
        pv(Vs[cb], so.p);
        f2 = st.commit(a, xb, tok, (kt_begin + t + 2) * kKeyTile, tid, Ks[fb], Vs[fb]);
      }
    } else if (act) {
      pv(Vs[cb], so.p);
    } else if (more2) {
      f2 = st.commit(a, xb, tok, (kt_begin + t + 2) * kKeyTile, tid, Ks[fb], Vs[fb]);
    }
    publish(fb, f2);
    __syncthreads();
    nf0 = nf1;
    nf1 = read_nf(fb);
    w0 = w1;
    w1 = more2 ? keep_word(kt_begin + t + 2, m2) : 0u;
    if (act1) s_cur = s_nx;
    cb = nb;
  }

  // Careful walk, from the tile where the fast walk stopped: the reference's
  // masked softmax with an exact running max (non-finite scores weigh 0, a
  // +inf score empties the row) and, for a tile holding a non-finite value,
  // key-by-key accumulation that skips zero probabilities.
  for (; t < nt; ++t) {
    const int nb = cb == NBUF - 1 ? 0 : cb + 1, fb = nb == NBUF - 1 ? 0 : nb + 1;
    const bool more2 = t + 2 < nt;
    if (more2) {
      m2 = mask_of(kt_begin + t + 2);
      st.fetch(a, xb, tok, (kt_begin + t + 2) * kKeyTile, tid);
    }
    if (__ballot(w0 != 0u) != 0) {
      f32x16 p = scores(Ks[cb]);
      const float alpha = softmax_tile(p, qin ? w0 : 0u, half, c1, m, l);
      // alpha == 0: every earlier probability is 0 against the new max, so
      // earlier (possibly infinite) values drop out as in the reference.
#pragma unroll
      for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) O[j][r] = alpha == 0.0f ? 0.0f : O[j][r] * alpha;
      const float *Vc = Vs[cb];
      if (!nf0) {
        pv(Vc, p);
      } else {
        // The reference's scalar path (lib.rs:1143-1151): a masked
        // non-finite value never leaks.
        for (int kk = 0; kk < kKeyTile; ++kk) {
          const float pk = tile_prob(p, kk, col);
          if (pk == 0.0f) continue;
#pragma unroll
          for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) O[j][r] += pk * Vc[kk * VS + j * 32 + acc_row(r, half)];
        }
      }
    }
    int f2 = 0;
    if (more2) f2 = st.commit(a, xb, tok, (kt_begin + t + 2) * kKeyTile, tid, Ks[fb], Vs[fb]);
    publish(fb, f2);
    __syncthreads();
    nf0 = nf1;
    nf1 = read_nf(fb);
    w0 = w1;
    w1 = more2 ? keep_word(kt_begin + t + 2, m2) : 0u;
    cb = nb;
  }

  // -------- normalize and store: out[feat + d + hidden*(q + L*b)]
  // 0/0 gives NaN for a query that kept nothing, as the reference does.
  const float lt = pair_sum(l);
  const float inv = lt > 0.0f ? fast_rcp(lt) : __builtin_nanf("");
  if (qin) {
    float *orow = a.out + ((size_t)b * L + q) * a.d + (size_t)head * hd;
    if constexpr (VEC) {
      // Accumulators 4g..4g+3 are dims j*32 + 8g + 4*half + 0..3: one
      // 16-byte store each.
#pragma unroll
      for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 v = {O[j][4 * g] * inv, O[j][4 * g + 1] * inv, O[j][4 * g + 2] * inv,
                           O[j][4 * g + 3] * inv};
          *reinterpret_cast<f32x4 *>(orow + j * 32 + 8 * g + 4 * half) = v;
        }
    } else {
#pragma unroll
      for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int dd = j * 32 + acc_row(r, half);
          if (dd < hd) orow[dd] = O[j][r] * inv;
        }
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

hipError_t launch_laya_keep_bits(const uint8_t *keep, uint32_t *bits, uint8_t *any, int L, int B,
                                 int nkt, hipStream_t stream) {
  dim3 grid((L + 255) / 256, nkt, B);
  hipLaunchKernelGGL(laya_keep_bits_kernel, grid, dim3(256), 0, stream, keep, bits, any, L, nkt);
  return hipGetLastError();
}

template <int HDP, bool VEC, bool ROPE>
static hipError_t launch_laya_hd(const LayaArgs &a, int heads, int batch, int mode,
                                 hipStream_t stream) {
  dim3 grid((a.L + kLayaGroupQueries - 1) / kLayaGroupQueries, heads, batch);
  if (mode == kMaskBits)
    hipLaunchKernelGGL((laya_attention_kernel<HDP, kMaskBits, VEC, ROPE>), grid, dim3(256), 0,
                       stream, a);
  else
    hipLaunchKernelGGL((laya_attention_kernel<HDP, kMaskStruct, VEC, ROPE>), grid, dim3(256), 0,
                       stream, a);
  return hipGetLastError();
}

template <int HDP>
static hipError_t launch_laya_pick(const LayaArgs &a, int heads, int batch, int mode,
                                   hipStream_t stream) {
  // 16-byte row loads need hd == HDP, hd % 8 == 0 (RoPE halves in whole
  // chunks), a row stride of whole chunks and aligned bases.
  const bool vec = a.hd == HDP && a.hd % 8 == 0 && a.d % 4 == 0 &&
                   (reinterpret_cast<uintptr_t>(a.qkv) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(a.out) & 15) == 0;
  const bool rope = a.cos_t != nullptr;
  if (vec)
    return rope ? launch_laya_hd<HDP, true, true>(a, heads, batch, mode, stream)
                : launch_laya_hd<HDP, true, false>(a, heads, batch, mode, stream);
  return rope ? launch_laya_hd<HDP, false, true>(a, heads, batch, mode, stream)
              : launch_laya_hd<HDP, false, false>(a, heads, batch, mode, stream);
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
