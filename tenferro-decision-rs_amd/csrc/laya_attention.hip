// Laya fused split + RoPE + masked attention on gfx950 f32 matrix cores.
//
// Arithmetic follows cpu-kernels laya_attention_block_with_workspace
// (crates/cpu-kernels/src/lib.rs:843-1156): RoPE on q and k from a host-built
// f32 table (874-888), s = (q.k) * (1/sqrt(hd)) (1124), masked softmax
// (1111-1136), out = sum p*v with p == 0 never multiplying a value (1143-1151),
// NaN for a query that keeps no key (1025-1033, 1143-1151).
//
// One workgroup = 4 wavefronts = 64 queries of one (batch, head). Each
// wavefront owns 16 queries and walks 32-key tiles as two 16-key blocks:
//   S^T (16 keys x 16 queries) = K_blk * Q^T       (hd/4 MFMA 16x16x4 per block)
//   O^T (hd x 16 queries)     += V_tile^T * P^T     (hd/16 x 8 MFMA 16x16x4)
// Computing S^T rather than S puts each lane's 8 probabilities exactly where
// the B operand of the P.V product wants them, so no shuffles sit between the
// two products. Q (rotated) stays in registers for the whole walk; K (rotated
// while staged) and V tiles go through LDS and are shared by the 4 waves.
// Key tiles outside the workgroup's key span are never visited; a wave whose
// 16 queries keep nothing in a tile skips its MFMAs. Small workgroups (four
// per CU) keep the per-tile critical path short and the work per CU even
// when rows differ in length.
#include <type_traits>

#include "tfd_device.hpp"
#include "tfd_internal.hpp"

namespace tfd {

// ---------------------------------------------------------------- keep bits

// Packs the (L, L, B) byte keep tensor into one 32-bit word per
// (batch, key tile, query): bit j set when key 32*kt + j is kept. Also
// writes the tile map: byte (b*ng + g)*laya_map_row(nkt) + kt is 1 when any
// of queries 64g..64g+63 keeps a key of tile kt (ng = ceil(L/64)); the
// attention workgroups read their group's row with scalar loads.
// Placement plan of a one-round attention grid (laya_xcd_layout, kMaskBits):
// the item and key span of workgroup p, computed from the whole tile map by
// one wave (every workgroup derives the same plan). Workgroup p runs on XCD
// x = p % 8, CU c = (p / 8) % 32 of it, round t = p / 256 (S = grid / 256
// rounds). As in the fixed layout, XCD x runs the items r in [x*M, x*M + M)
// of every batch row (M = heads*nqb / 8; a head's keys are read by at most
// two XCDs). Which CU runs which of them follows the row's cost, the widest
// key span over its 64-query groups: the XCD's items sorted by cost, longest
// first, are dealt out in snake order for rounds 0 .. S-2, and the last round
// gives the largest remaining items to the least loaded CUs. Every XCD holds
// the same multiset of row costs, so one CU order serves all eight. Only the
// work of a CU changes, never a result. `scratch` holds B*ng + 96 ints of
// LDS. Returns {row, item head*nqb + qb, kt_begin, kt_end}, uniform.
__device__ int4 laya_plan_item(const uint8_t *__restrict__ any, int L, int nkt, int B, int H,
                               int p, int *scratch, FastDiv ngdiv, FastDiv mdiv) {
  const int lane = threadIdx.x & 63;
  const int ng = (L + 63) >> 6, G = B * ng;
  const int M = (H * ng) >> 3, S = (B * M) >> 5;  // both exact in this layout
  int *s_span = scratch, *s_cost = scratch + G, *s_rows = s_cost + 32, *s_load = s_rows + 32;
  auto wave_sync = [] {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
  if (lane < 32) s_cost[lane] = 0;
  wave_sync();
  for (int g = lane; g < G; g += 64) {  // the span of every (row, 64-query group)
    const uint4 *row = reinterpret_cast<const uint4 *>(any + (size_t)g * laya_map_row(nkt));
    int lo = -1, hi = -1;
    for (int t0 = 0; t0 < nkt; t0 += 16) {
      const uint4 v = row[t0 / 16];  // 16 flags; rows are padded to 64 bytes
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = t0 + 4 * i;
        uint32_t x = w[i];
        if (t + 4 > nkt) x = t >= nkt ? 0u : x & ((1u << (8 * (nkt - t))) - 1u);
        if (x != 0u) {
          if (lo < 0) lo = t + (int)__builtin_ctz(x) / 8;
          hi = t + (31 - (int)__builtin_clz(x)) / 8;
        }
      }
    }
    s_span[g] = lo < 0 ? 0 : lo | ((hi + 1) << 16);
    if (lo >= 0) atomicMax(&s_cost[ngdiv.div((uint32_t)g)], hi + 1 - lo);
  }
  wave_sync();
  if (lane < B) {  // rows by cost, longest first (ties: lower row first)
    const int cb = s_cost[lane];
    int rank = 0;
    for (int o = 0; o < B; ++o) rank += s_cost[o] > cb || (s_cost[o] == cb && o < lane);
    s_rows[rank] = lane;
  }
  wave_sync();
  auto snake = [](int t, int c) { return 32 * t + ((t & 1) ? 31 - c : c); };
  if (lane < 32) {  // CU `lane`'s load after the snake rounds
    int load = 0;
    for (int t = 0; t < S - 1; ++t) load += s_cost[s_rows[mdiv.div((uint32_t)snake(t, lane))]];
    s_load[lane] = load;
  }
  wave_sync();
  const int x = p & 7, c = (p >> 3) & 31, t = p >> 8;
  int pos = snake(t, c);
  if (t == S - 1) {  // last round: this CU's place by load, least loaded first
    const int lc = s_load[c];
    const bool before = lane < 32 && (s_load[lane] < lc || (s_load[lane] == lc && lane < c));
    pos = 32 * t + __builtin_popcountll(__ballot(before));
  }
  const int pm = (int)mdiv.div((uint32_t)pos);
  const int b = s_rows[pm];
  const int r = x * M + (pos - pm * M);
  const int sp = s_span[b * ng + (r - (int)ngdiv.div((uint32_t)r) * ng)];
  return make_int4(b, r, sp & 0xffff, sp >> 16);
}

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
  if ((threadIdx.x & 63) == 0)
    any[((size_t)b * ((L + 63) / 64) + q / 64) * laya_map_row(nkt) + kt] = some;
}

// The structured mask (valid (L, B) + window, laya-infer model.rs:465-490)
// in the attention kernel's terms, for a grid that gets the placement plan:
// words[b*nkt + kt], bit j set when key 32*kt + j is valid (the keys any
// query of row b may keep; the kernel applies the window per query), and the
// tile map in laya_keep_bits_kernel's layout: flag (b, g, kt) is 1 when some
// query of 64-query group g keeps a key of tile kt. A valid query keeps the
// valid keys within the window (all valid keys without one), a padded query
// every valid key; so a group with a padded query, or any group without a
// window, keeps every tile holding a valid key, and otherwise the tiles
// holding a valid key within the window of the group's first or last query.
// One wave per (row b, group g): lane l reads query 64g + l, then the row's
// keys 64 at a time (all loads independent); the g == 0 wave also writes the
// row's words.
__global__ __launch_bounds__(64) void laya_valid_prep_kernel(const uint8_t *__restrict__ valid,
                                                             uint32_t *__restrict__ words,
                                                             uint8_t *__restrict__ any, int L,
                                                             int nkt, int window) {
  const int ng = (L + 63) / 64, g = blockIdx.x, b = blockIdx.y;
  const int lane = threadIdx.x;
  const uint8_t *vb = valid + (size_t)b * L;
  const int q0 = 64 * g, q1 = min(q0 + 63, L - 1);
  const bool padded = __ballot(q0 + lane < L && vb[min(q0 + lane, L - 1)] == 0) != 0;
  int lo = 0, hi = L - 1;  // keys some query of the group may keep
  if (window >= 0 && !padded) {
    lo = max(0, q0 - window);
    hi = min(L - 1, q1 + window);
  }
  uint8_t *row = any + ((size_t)b * ng + g) * laya_map_row(nkt);
  for (int c0 = 0; c0 < ng; c0 += 8) {
    uint8_t x[8];  // eight 64-key chunks in flight at once
#pragma unroll
    for (int u = 0; u < 8; ++u) x[u] = vb[min(64 * (c0 + u) + lane, L - 1)];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int c = c0 + u, k = 64 * c + lane;
      const bool v = k < L && x[u] != 0;
      const uint64_t kept = __ballot(v && k >= lo && k <= hi);
      const uint64_t vm = __ballot(v);
      if (lane < 2 && 2 * c + lane < nkt) {  // lane t: tile 2c + t (bits 32t .. 32t + 31)
        row[2 * c + lane] = (uint32_t)(kept >> (32 * lane)) != 0u;
        if (g == 0) words[(size_t)b * nkt + 2 * c + lane] = (uint32_t)(vm >> (32 * lane));
      }
    }
  }
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

// One K/V tile's global data held in registers between the prefetch (issued
// before the previous tile's products) and the LDS commit (after them). LDS
// holds K as [key][d] (row stride KS) and V transposed, [d][key] (row stride
// VS), so that the P.V product reads four consecutive keys of one feature
// with one 16-byte read.
//
// VEC (hd == HDP, hd % 8 == 0, 16-byte aligned rows, the batch row within
// 2 GiB): buffer loads; a K task is one (key, chunk c) with its RoPE partner
// chunk c + half/4 (and, with ROPE, the table chunks); a V task is one
// feature of four consecutive keys, four 4-byte loads (a wave reads whole
// key rows) that land as one 16-byte [d][key .. key + 3] LDS row piece.
// Keys at or past L read as 0. Otherwise (any hd) the commit loads and
// rotates element by element and the prefetch is empty.
template <int HDP, bool VEC, bool ROPE, int NT = 256>  // NT: threads that stage a tile
struct LayaStage {
  static constexpr int KS = HDP + 4;        // conflict-free 16-byte row reads
  static constexpr int VS = kKeyTile + 4;   // 16 lanes of 16-byte row pieces: conflict-free
  static constexpr int KBUF = kKeyTile * KS, VBUF = HDP * VS;
  static constexpr int KTASKS = kKeyTile * HDP / 8;
  static constexpr int VTASKS = (kKeyTile / 4) * HDP;
  static constexpr int KN = VEC ? (KTASKS + NT - 1) / NT : 1;
  static constexpr int VN = VEC ? (VTASKS + NT - 1) / NT : 1;
  static constexpr int CN = ROPE ? KN : 1;
  f32x4 ka[KN], kb[KN], c[CN], s[CN];
  f32x4 v[VN];
  // Resources and per-lane byte offsets, fixed for the walk.
  __amdgpu_buffer_rsrc_t rk, rv, rc, rs;
  int ok[KN], oc[KN], ov[VN];
  int hh4, tok4;

  __device__ __forceinline__ void init(const LayaArgs &a, const float *xb, size_t tok, int tid) {
    if constexpr (VEC) {
      const int L = a.L, hh = a.half;
      const uint32_t row_bytes = (uint32_t)(((size_t)(L - 1) * tok + a.hd) * 4);
      rk = buffer_rsrc(xb + a.d, row_bytes);
      rv = buffer_rsrc(xb + 2 * a.d, row_bytes);
      if constexpr (ROPE) {
        rc = buffer_rsrc(a.cos_t, (uint32_t)((size_t)L * hh * 4));
        rs = buffer_rsrc(a.sin_t, (uint32_t)((size_t)L * hh * 4));
      }
#pragma unroll
      for (int i = 0; i < KN; ++i) {
        const int task = min(tid + NT * i, KTASKS - 1);
        const int kk = task / (HDP / 8), cp = task % (HDP / 8);
        ok[i] = (int)(((size_t)kk * tok + 4 * cp) * 4);
        oc[i] = (kk * hh + 4 * cp) * 4;
      }
#pragma unroll
      for (int i = 0; i < VN; ++i) {
        const int task = min(tid + NT * i, VTASKS - 1);
        const int dd = task % HDP, kq = task / HDP;
        ov[i] = (int)(((size_t)(4 * kq) * tok + dd) * 4);
      }
      hh4 = hh * 4;
      tok4 = (int)(tok * 4);
    }
  }

  __device__ __forceinline__ void fetch(int k0) {
    if constexpr (VEC) {
      const int sk = k0 * tok4, sc = k0 * hh4;
#pragma unroll
      for (int i = 0; i < KN; ++i) {
        ka[i] = buffer_load4(rk, ok[i], sk);
        kb[i] = buffer_load4(rk, ok[i], sk + hh4);
        if constexpr (ROPE) {
          c[i] = buffer_load4(rc, oc[i], sc);
          s[i] = buffer_load4(rs, oc[i], sc);
        }
      }
#pragma unroll
      for (int i = 0; i < VN; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) v[i][e] = buffer_load1(rv, ov[i], sk + e * tok4);
    }
  }

  // Writes the tile to LDS (K rotated, V transposed).
  __device__ __forceinline__ void commit(const LayaArgs &a, const float *xb, size_t tok, int k0,
                                         int tid, float *Ks, float *Vs) {
    if constexpr (VEC) {
      const int hh = a.half;
#pragma unroll
      for (int i = 0; i < KN; ++i) {
        const int task = tid + NT * i;
        if (KTASKS % NT == 0 || task < KTASKS) {
          const int kk = task / (HDP / 8), cp = task % (HDP / 8);
          f32x4 lo = ka[i], hi = kb[i];
          if constexpr (ROPE) {
            lo = rot_lo(ka[i], kb[i], c[i], s[i]);
            hi = rot_hi(ka[i], kb[i], c[i], s[i]);
          }
          *reinterpret_cast<f32x4 *>(&Ks[kk * KS + 4 * cp]) = lo;
          *reinterpret_cast<f32x4 *>(&Ks[kk * KS + hh + 4 * cp]) = hi;
        }
      }
#pragma unroll
      for (int i = 0; i < VN; ++i) {
        const int task = tid + NT * i;
        if (VTASKS % NT == 0 || task < VTASKS) {
          const int dd = task % HDP, kq = task / HDP;
          *reinterpret_cast<f32x4 *>(&Vs[dd * VS + 4 * kq]) = v[i];
        }
      }
    } else {
      const int L = a.L, hd = a.hd, hh = a.half;
      for (int e = tid; e < kKeyTile * HDP; e += NT) {
        const int kk = e / HDP, dd = e % HDP;
        const int key = k0 + kk;
        float kv = 0.0f, vv = 0.0f;
        if (key < L && dd < hd) {
          const float *row = xb + (size_t)key * tok;
          const float *cr = ROPE ? a.cos_t + (size_t)key * hh : nullptr;
          const float *sr = ROPE ? a.sin_t + (size_t)key * hh : nullptr;
          kv = rope_elem(row + a.d, dd, hd, hh, cr, sr);
          vv = row[2 * a.d + dd];
        }
        Ks[kk * KS + dd] = kv;
        Vs[dd * VS + kk] = vv;
      }
    }
  }
};

// ------------------------------------------------------------------- kernel

// The careful path for one wave's 16 queries (rare: NaN or inf among its
// kept scores or values), recomputed from global memory without barriers
// and written to out: the reference's masked softmax with an exact running
// max (non-finite scores weigh 0, a +inf score empties the row,
// lib.rs:1111-1136) and key-by-key accumulation that skips zero
// probabilities (lib.rs:1143-1151). Kept out of line so that its registers
// never weigh on the walk. Pw: 32 x 17 floats of LDS owned by the wave.
template <int HDP, int MODE, bool ROPE>
__device__ __noinline__ void laya_redo_wave(const LayaArgs *ap, int b, int head, int q0,
                                            int kt_begin, int kt_end, float *Pw) {
  const LayaArgs &a = *ap;
  constexpr int QS = HDP / 4, NB = HDP / 16, PS = 17;
  const int lane = threadIdx.x & 63, col = lane & 15, grp = lane >> 4;
  const int L = a.L, hd = a.hd, hh = a.half, nkt = a.nkt;
  const int q = q0 + col;
  const bool qin = q < L;
  const size_t tok = 3 * (size_t)a.d;
  const float *xb = a.qkv + (size_t)b * L * tok + (size_t)head * hd;
  const int qq = qin ? q : 0;
  float qreg[QS];
  {
    const float *row = xb + (size_t)qq * tok;
    const float *cr = ROPE ? a.cos_t + (size_t)qq * hh : nullptr;
    const float *sr = ROPE ? a.sin_t + (size_t)qq * hh : nullptr;
#pragma unroll
    for (int x = 0; x < QS; ++x) qreg[x] = qin ? rope_elem(row, grp * QS + x, hd, hh, cr, sr) : 0.0f;
  }
  bool q_valid = false;
  if (MODE == kMaskStruct) q_valid = qin && a.valid[(size_t)b * L + qq] != 0;
  f32x4 O[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) O[j][r] = 0.0f;
  float m = kNoMax, l = 0.0f;
#pragma unroll 1
  for (int kt = kt_begin; kt < kt_end; ++kt) {
    const int k0 = kt * kKeyTile;
    uint32_t wk = 0u;
    if (MODE == kMaskBits) {
      const uint32_t x = a.bits[((size_t)b * nkt + kt) * L + qq];
      wk = qin ? x : 0u;
    } else if (MODE == kMaskRaw) {
      uint32_t x = 0u;
      for (int j = 0; j < kKeyTile && k0 + j < L; ++j)
        x |= (uint32_t)(a.keep[(size_t)b * L * L + (size_t)(k0 + j) * L + qq] != 0) << j;
      wk = qin ? x : 0u;
    } else {
      const int key = k0 + (lane & 31);
      const bool kv = key < L && a.valid[(size_t)b * L + min(key, L - 1)] != 0;
      const uint32_t vbits = (uint32_t)__ballot(kv);
      if (qin) {
        wk = vbits;
        if (a.window >= 0 && q_valid) wk &= range_bits(q - a.window - k0, q + a.window - k0);
      }
    }
    if (__ballot(wk != 0u) == 0) continue;
    f32x4 sb[2];
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
      const int key = k0 + 16 * blk + col;
      const int kc = min(key, L - 1);
      const float *krow = xb + (size_t)kc * tok + a.d;
      const float *cr = ROPE ? a.cos_t + (size_t)kc * hh : nullptr;
      const float *sr = ROPE ? a.sin_t + (size_t)kc * hh : nullptr;
      f32x4 p = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int x = 0; x < QS; ++x) {
        const float kx = rope_elem(krow, grp * QS + x, hd, hh, cr, sr);
        p = mfma_16x16x4(key < L ? kx : 0.0f, qreg[x], p);
      }
      sb[blk] = p;
    }
    const float alpha = softmax_tile16(sb[0], sb[1], wk, grp, a.c1, m, l);
    // alpha == 0: every earlier probability is 0 against the new max, so
    // earlier (possibly infinite) values drop out as in the reference.
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) O[j][r] = alpha == 0.0f ? 0.0f : O[j][r] * alpha;
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      Pw[(4 * grp + r) * PS + col] = sb[0][r];
      Pw[(16 + 4 * grp + r) * PS + col] = sb[1][r];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll 1
    for (int kk = 0; kk < kKeyTile; ++kk) {
      const float pk = Pw[kk * PS + col];
      if (pk == 0.0f) continue;  // only kept keys inside the row get here
      const float *vrow = xb + (size_t)(k0 + kk) * tok + 2 * a.d;
#pragma unroll
      for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int dd = 16 * j + 4 * grp + r;
          if (dd < hd) O[j][r] += pk * vrow[dd];
        }
    }
    __builtin_amdgcn_wave_barrier();
  }
  const float lt = pair_sum(pair16_sum(l));
  const float inv = lt > 0.0f ? fast_rcp(lt) : __builtin_nanf("");
  if (qin) {
    float *orow = a.out + ((size_t)b * L + q) * a.d + (size_t)head * hd;
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int dd = 16 * j + 4 * grp + r;
        if (dd < hd) orow[dd] = O[j][r] * inv;
      }
  }
}

// Occupancy target (laya_groups_per_cu): four workgroups (16 waves) per CU
// where LDS and registers allow it. On gfx950 the f32 MFMAs and the vector
// ALU share the SIMD (they never run at the same time), so the walk keeps its
// vector work per tile small and relies on other waves to cover memory and
// barrier waits.
template <int HDP, int MODE, bool VEC, bool ROPE, bool VW, int TEAMS, int QW>
__global__ __launch_bounds__(64 * QW * TEAMS, TEAMS == 1 ? laya_groups_per_cu(HDP) : 1) void laya_attention_kernel(
    const LayaArgs a) {
  static_assert(QW == 4 || (QW == 2 && TEAMS > 1), "16 queries per wave, 4 or 2 waves per team");
  constexpr int NT = 64 * QW;  // threads per team
  using Stage = LayaStage<HDP, VEC, ROPE, NT>;
  constexpr int KS = Stage::KS, VS = Stage::VS;
  constexpr int QS = HDP / 4;   // Q registers per lane (4 lane groups split hd)
  constexpr int NB = HDP / 16;  // 16-row blocks of O^T
  constexpr int GQ = kLayaWaveQueries * QW;  // queries per workgroup
  // TEAMS > 1 (grids of at most one workgroup per CU): TEAMS teams of four
  // waves, each with its own K/V buffers, walk every TEAMS-th key tile of
  // the workgroup's span and merge their (m, l, O) once at the end.
  constexpr int TB = 2 * (Stage::KBUF + Stage::VBUF);  // floats per team
  static_assert(TEAMS == 1 || (TEAMS - 1) * 4 * (4 * (HDP / 16) + 2) * 64 + 4 * kKeyTile * 17 <= TEAMS * TB,
                "merge data and the redo rows fit in the teams' K/V buffers");
  __shared__ __attribute__((aligned(16))) float smem[TEAMS * TB];
  const int team = TEAMS == 1 ? 0 : __builtin_amdgcn_readfirstlane((int)threadIdx.x / NT);
  auto Ks = [&](int i) { return smem + team * TB + i * Stage::KBUF; };
  auto Vs = [&](int i) { return smem + team * TB + 2 * Stage::KBUF + i * Stage::VBUF; };

  const int tid = TEAMS == 1 ? (int)threadIdx.x : (int)(threadIdx.x & (NT - 1)), lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform, in a scalar register
  const int col = lane & 15, grp = lane >> 4;
  const int L = a.L, hd = a.hd, hh = a.half, nkt = a.nkt;
  // Work item (batch row b, head, 64-query block qb). The dispatcher hands
  // workgroup p to XCD p % 8 (each XCD has its own L2) and, while all fit,
  // to CU slot p % (CUs): when the counts allow it (laya_xcd_layout), each
  // XCD gets an equal share of every batch row (consecutive (head, block)
  // items, so a head's keys and values are read by at most two XCDs). The
  // placement plan, when a tile map is given (laya_keep_bits_kernel's, or
  // laya_valid_prep_kernel's for the structured mask), also balances the key
  // tiles per CU and carries the item's key span; otherwise the workgroups of a CU come
  // from different rows (r, r + 3, r + 6). Beyond one dispatch round,
  // workgroups start where others end and the grid order is the better
  // schedule.
  int b = blockIdx.z, head = blockIdx.y, qb = blockIdx.x;
  int kt_begin = 0, kt_end = 0;
  const int nqb = gridDim.x, H = gridDim.y, B = gridDim.z;
  // The launcher decides the layout (laya_xcd_layout, laya_planned) and
  // supplies the divisions by nqb and by M.
  const bool xcd = TEAMS == 1 && QW == 4 && a.layout >= 1;
  const bool planned = TEAMS == 1 && QW == 4 && a.layout == 2;
  {
    const int p = blockIdx.x + nqb * (blockIdx.y + H * blockIdx.z);
    if (planned) {
      __shared__ int4 s_item;
      if (wave == 0) {
        const int4 e = laya_plan_item(a.any, L, nkt, B, H, p, reinterpret_cast<int *>(smem),
                                      a.ngdiv, a.mdiv);
        if (lane == 0) s_item = e;
      }
      __syncthreads();
      const int4 e = s_item;
      b = __builtin_amdgcn_readfirstlane(e.x);
      const int ey = __builtin_amdgcn_readfirstlane(e.y);
      head = (int)a.ngdiv.div((uint32_t)ey);
      qb = ey - head * nqb;
      kt_begin = e.z;
      kt_end = e.w;
    } else if (xcd) {
      // B divides 32 in this layout (a power of two).
      const int M = (H * nqb) >> 3;  // items of a batch row per XCD
      const int lb = __builtin_ctz((unsigned)B);
      const int x = p & 7, j = p >> 3;
      const int t = j >> 5, c = j & 31;  // round, CU of the XCD
      const int row = (c + 3 * t) & (B - 1);
      const int k = t * (32 >> lb) + (c >> lb);  // item of that row on this XCD
      const int r = x * M + k;
      b = row;
      head = (int)a.ngdiv.div((uint32_t)r);
      qb = r - head * nqb;
    }
  }
  const int qg0 = qb * GQ;
  const int q0w = qg0 + wave * kLayaWaveQueries;
  const int q = q0w + col;
  const bool qin = q < L;
  const size_t tok = 3 * (size_t)a.d;
  const float *xb = a.qkv + (size_t)b * L * tok + (size_t)head * hd;

  // -------- key span of the workgroup: the tiles [kt_begin, kt_end) that
  // hold a key some query of the workgroup may keep (it may be a superset; a
  // wave skips the products of tiles its queries keep nothing of). Every
  // wave computes it on its own from ballots (identical scalar results, no
  // barrier). Its bytes are read before anything else, so that waiting for
  // them never waits for the Q rows issued after them.
  const int ng = (L + 63) / 64;
  // kMaskBits: the workgroup's 64 queries are exactly tile-map group qg0 / 64.
  const uint8_t *anyb = a.any + ((size_t)b * ng + qg0 / 64) * laya_map_row(nkt);
  const uint8_t *vb = a.valid + (size_t)b * L;  // kMaskStruct
  const __amdgpu_buffer_rsrc_t rkeep =  // kMaskRaw: this batch row's keep bytes
      buffer_rsrc(MODE == kMaskRaw ? a.keep + (size_t)b * L * L : nullptr,
                  MODE == kMaskRaw ? (uint32_t)((size_t)L * L) : 0u);
  bool padded = false;
  if (MODE == kMaskStruct) {
    const int qx = qg0 + lane;
    const bool mine = lane < GQ;  // lane = one of the workgroup's queries
    const uint8_t xv = vb[min(qx, L - 1)];
    padded = __ballot(mine && qx < L && xv == 0) != 0;
    // A caller that reads only some queries' outputs (the model forward)
    // skips groups without one. Every wave takes the same branch before any
    // barrier, so the workgroup leaves as a whole.
    if (a.qneed != nullptr &&
        __ballot(mine && qx < L && a.qneed[(size_t)b * L + min(qx, L - 1)] != 0) == 0)
      return;
  }

  // -------- Q: rotated, in registers. Lane (col, grp) holds
  // Q[q][grp*QS + x] for x < QS, the B operand of step x.
  float qreg[QS];
  const int qq = qin ? q : 0;
  const int d0 = grp * QS;
  // VEC (hd == HDP): the wave's 16 Q rows are loaded along the rows, so that
  // every load instruction reads whole cache lines once: task (t, p) is
  // token q0w + t with its chunk pair (p, p + hd/8), the two 16-byte pieces
  // that RoPE rotates together, plus table chunk p of that token. The
  // rotated rows go to the wave's staging rows in LDS (the second K/V
  // buffer, unused until the walk's first barrier has passed) and come back
  // in the MFMA layout after the loads.
  constexpr int QT = 16 * HDP / 8 / 64;  // tasks per lane
  constexpr int QSR = HDP + 4;           // staging row stride: conflict-free 16-byte accesses
  f32x4 qlo4[VEC ? QT : 1], qhi4[VEC ? QT : 1], qc4[VEC && ROPE ? QT : 1], qs4[VEC && ROPE ? QT : 1];
  float *qst = nullptr;
  if constexpr (VEC) {
    static_assert(2 * 16 * QSR <= Stage::KBUF && 2 * 16 * QSR <= Stage::VBUF,
                  "Q staging: two waves per second K or V buffer");
    qst = (wave < 2 ? Ks(1) : Vs(1)) + (wave & 1) * 16 * QSR;
#pragma unroll
    for (int i = 0; i < QT; ++i) {
      const int task = lane + 64 * i, pp = task % (HDP / 8), t = task / (HDP / 8);
      const int tq = min(q0w + t, L - 1);
      const float *row = xb + (size_t)tq * tok + 4 * pp;
      qlo4[i] = *reinterpret_cast<const f32x4 *>(row);
      qhi4[i] = *reinterpret_cast<const f32x4 *>(row + hh);
      if constexpr (ROPE) {
        qc4[i] = *reinterpret_cast<const f32x4 *>(a.cos_t + (size_t)tq * hh + 4 * pp);
        qs4[i] = *reinterpret_cast<const f32x4 *>(a.sin_t + (size_t)tq * hh + 4 * pp);
      }
    }
  }

  // Lowest / highest set lane index of a ballot over 64 items starting at k0.
  int lo = 0x7fffffff, hi = -1;
  auto span_add = [&](uint64_t mk, int k0) {
    if (mk != 0) {
      lo = min(lo, k0 + (int)__builtin_ctzll(mk));
      hi = max(hi, k0 + 63 - (int)__builtin_clzll(mk));
    }
  };
  if (planned) {
    // the span came with the plan entry
  } else if (MODE == kMaskRaw) {
    // Every tile for now: the first tiles are fetched on that guess while
    // the workgroup scans its queries' keep bytes for the real span (below).
    kt_begin = 0;
    kt_end = nkt;
  } else if (MODE == kMaskBits) {
    // The group's row of the tile map, 64 flags (16 words) per scalar load.
    const uint32_t *anyw = reinterpret_cast<const uint32_t *>(anyb);
    for (int t0 = 0; t0 < nkt; t0 += 64) {
      uint32_t x[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) x[i] = anyw[t0 / 4 + i];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int t = t0 + 4 * i;  // flags t .. t + 3, one per byte
        uint32_t v = x[i];
        if (t + 4 > nkt) v = t >= nkt ? 0u : v & ((1u << (8 * (nkt - t))) - 1u);
        if (v != 0u) {
          lo = min(lo, t + (int)__builtin_ctz(v) / 8);
          hi = max(hi, t + (31 - (int)__builtin_clz(v)) / 8);
        }
      }
    }
    if (hi >= 0) {
      kt_begin = lo;
      kt_end = hi + 1;
    }
  } else {
    // build_mask (laya-infer model.rs:465-490): a valid query keeps the
    // valid keys of its window, a padded query every valid key. With a
    // window and no padded query in the group the window bounds the span;
    // otherwise it runs from the first to the last valid key of the row.
    int kf = 0, kl = -1;
    if (a.window >= 0 && !padded) {
      kf = max(0, qg0 - a.window);
      kl = min(L - 1, min(qg0 + GQ - 1, L - 1) + a.window);
    } else {
      for (int k0 = 0; k0 < L; k0 += 64 * 8) {
        uint8_t v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = vb[min(k0 + lane + 64 * u, L - 1)];
#pragma unroll
        for (int u = 0; u < 8; ++u)
          span_add(__ballot(k0 + lane + 64 * u < L && v[u] != 0), k0 + 64 * u);
      }
      kf = lo;
      kl = hi;
    }
    if (kl >= 0 && kf <= kl) {
      kt_begin = kf / kKeyTile;
      kt_end = kl / kKeyTile + 1;
    }
  }
  // Ballot results are uniform already; say so for the walk's scalar
  // counters and offsets.
  kt_begin = __builtin_amdgcn_readfirstlane(kt_begin);
  kt_end = __builtin_amdgcn_readfirstlane(kt_end);
  // This team's tiles: those of [kt_begin, kt_end) with kt % TEAMS == team,
  // from tb in steps of TEAMS (a choice that depends on the tile index only,
  // not on the span, so that two spans of the same keep pattern give the
  // same sums); every team runs the same number of steps (one barrier each).
  int tb = kt_begin, te = kt_end, kt_stop = kt_end;
  auto team_span = [&]() {
    tb = kt_begin + ((team - kt_begin) % TEAMS + TEAMS) % TEAMS;
    te = kt_end;
    kt_stop = kt_begin + (kt_end - kt_begin + TEAMS - 1) / TEAMS * TEAMS + (tb - kt_begin);
  };
  if constexpr (TEAMS > 1) team_span();

  // This lane's keep word for key tile kt (bit j: key 32*kt + j). The raw
  // word or validity byte is fetched one tile ahead (mask_of) and turned
  // into the word (keep_word) only after that tile's barrier, so waiting on
  // it never stalls the tile prefetch issued beside it.
  // kMaskStruct reads the rows' valid-key words (VW: the prep gave them,
  // planned grids), else the validity bytes of the tile's keys.
  constexpr bool vwords = MODE == kMaskStruct && VW;
  // kMaskRaw: lanes 0..31 fetch the keep bytes of key 32*kt + lane for the
  // wave's 16 queries (one 16-byte piece of that key's row; a key past L
  // reads 0), turned into the 16 queries' words by ballots.
  using MaskT = typename std::conditional<MODE == kMaskRaw, uint4, uint32_t>::type;
  auto raw_of = [&](int kt) -> uint4 {
    const int key = kt * kKeyTile + (lane & 31);
    const f32x4 v = buffer_load4(rkeep, key * L + q0w, 0);
    return make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                      __float_as_uint(v[3]));
  };
  auto mask_of = [&](int kt) -> MaskT {
    if constexpr (MODE == kMaskRaw) {
      return raw_of(kt);
    } else {
      if (MODE == kMaskBits)
        return a.bits[((size_t)b * nkt + min(kt, nkt - 1)) * L + min(q, L - 1)];
      if (vwords) return a.bits[(size_t)b * nkt + min(kt, nkt - 1)];  // uniform
      return a.valid[(size_t)b * L + min(kt * kKeyTile + (lane & 31), L - 1)];
    }
  };

  // The first tile's loads go out before the Q rotation waits for its rows.
  Stage st;
  st.init(a, xb, tok, tid);
  MaskT m0{};
  if (tb < te) {
    m0 = mask_of(tb);
    st.fetch(tb * kKeyTile);
  }
  // kMaskRaw: the lowest and highest key any query of the workgroup keeps,
  // per wave (lane = key; a piece that runs past the last query reads the
  // next key's bytes, which can only widen the span).
  __shared__ int s_rspan[MODE == kMaskRaw ? 2 * TEAMS * QW : 1];
  if constexpr (MODE == kMaskRaw) {
    const int wg = (int)(threadIdx.x >> 6), nw = (int)(blockDim.x >> 6);
    for (int k0 = wg * 64; k0 < L; k0 += nw * 64) {  // lo, hi: still empty here
      const int k = k0 + lane;
      uint32_t any = 0u;
#pragma unroll
      for (int c = 0; c < GQ / 16; ++c) {
        const f32x4 v = buffer_load4(rkeep, k * L + qg0 + 16 * c, 0);
        any |= __float_as_uint(v[0]) | __float_as_uint(v[1]) | __float_as_uint(v[2]) |
               __float_as_uint(v[3]);
      }
      span_add(__ballot(k < L && any != 0u), k0);
    }
    if (lane == 0) {
      s_rspan[2 * wg] = lo;
      s_rspan[2 * wg + 1] = hi;
    }
  }

  if constexpr (VEC) {
#pragma unroll
    for (int i = 0; i < QT; ++i) {
      const int task = lane + 64 * i, pp = task % (HDP / 8), t = task / (HDP / 8);
      f32x4 lo = qlo4[i], hi = qhi4[i];
      if constexpr (ROPE) {
        lo = rot_lo(qlo4[i], qhi4[i], qc4[i], qs4[i]);
        hi = rot_hi(qlo4[i], qhi4[i], qc4[i], qs4[i]);
      }
      *reinterpret_cast<f32x4 *>(qst + t * QSR + 4 * pp) = lo;
      *reinterpret_cast<f32x4 *>(qst + t * QSR + hh + 4 * pp) = hi;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int c = 0; c < QS / 4; ++c) {
      const f32x4 v = *reinterpret_cast<const f32x4 *>(qst + col * QSR + d0 + 4 * c);
#pragma unroll
      for (int e = 0; e < 4; ++e) qreg[4 * c + e] = qin ? v[e] : 0.0f;
    }
  } else {
    const float *row = xb + (size_t)qq * tok;
    const float *cr = ROPE ? a.cos_t + (size_t)qq * hh : nullptr;
    const float *sr = ROPE ? a.sin_t + (size_t)qq * hh : nullptr;
#pragma unroll
    for (int x = 0; x < QS; ++x) qreg[x] = qin ? rope_elem(row, d0 + x, hd, hh, cr, sr) : 0.0f;
  }
  bool q_valid = false;
  if (MODE == kMaskStruct) {
    const uint8_t x = a.valid[(size_t)b * L + min(q, L - 1)];
    q_valid = qin && x != 0;
  }

  auto keep_word = [&](int kt, MaskT x) -> uint32_t {
    uint32_t w = 0u;
    if constexpr (MODE == kMaskRaw) {
      // Query q0w + c keeps key 32*kt + j when byte c of lane j's piece is
      // non-zero: one ballot per query, and this lane takes its query's.
      const uint32_t words[4] = {x.x, x.y, x.z, x.w};
      const bool kl = lane < kKeyTile;
#pragma unroll
      for (int c = 0; c < 16; ++c) {
        const uint32_t mk = (uint32_t)__ballot(kl && ((words[c / 4] >> (8 * (c % 4))) & 0xffu) != 0u);
        w = col == c ? mk : w;
      }
      w = qin ? w : 0u;
    } else if (MODE == kMaskBits) {
      w = qin ? x : 0u;
    } else {
      const int k0 = kt * kKeyTile;
      // The tile's valid keys (lanes 0..31 of the ballot = keys of the tile).
      const uint32_t vbits = vwords ? x : (uint32_t)__ballot(k0 + (lane & 31) < L && x != 0);
      if (qin) {
        w = vbits;
        if (a.window >= 0 && q_valid) w &= range_bits(q - a.window - k0, q + a.window - k0);
      }
    }
    return w;
  };

  f32x4 O[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) O[j][r] = 0.0f;
  float m = kNoMax, l = 0.0f;  // l: this lane's share of the row sum
  const float c1 = a.c1;

  // -------- the walk: tile kt+1 is fetched into registers before the
  // products of tile kt and committed to the other LDS buffer after them;
  // one barrier per tile. A 32-key tile is two S^T blocks: s0 holds keys
  // 4*grp + r, s1 keys 16 + 4*grp + r of query col.
  //
  // Exponents are exp2(fma(s, c1, -m)) against a reference m (log2 units)
  // that moves only when needed: a tile is first exponentiated against the
  // current m, and only if some lane's 8 terms sum to more than 2^11 (or to
  // NaN / inf: every term is then checked for a max more than kRescaleSlack
  // above m) is the tile max taken, m moved to it and the accumulators
  // rescaled. Terms stay below 2^11; O / l is unchanged. Non-finite inputs
  // are kept off this path: a wave whose kept scores sum to NaN or inf
  // stops computing (it still stages tiles and meets the barriers), a NaN or
  // inf value reaches O and stays there, and either way the wave redoes its
  // queries with the reference's exact semantics after the walk.
  uint32_t w = 0u;
  MaskT m_next{};
  if (tb < te) {
    st.commit(a, xb, tok, tb * kKeyTile, tid, Ks(0), Vs(0));
    w = keep_word(tb, m0);
  }
  __syncthreads();
  if constexpr (MODE == kMaskRaw) {
    // The real span (uniform): a shorter end only trims the walk; a later
    // start puts other tiles first, which are fetched and committed now.
    int rlo = 0x7fffffff, rhi = -1;
    for (int i = 0; i < (int)(blockDim.x >> 6); ++i) {
      rlo = min(rlo, s_rspan[2 * i]);
      rhi = max(rhi, s_rspan[2 * i + 1]);
    }
    const int nb = rhi >= 0 ? rlo / kKeyTile : 0, ne = rhi >= 0 ? rhi / kKeyTile + 1 : 0;
    const bool moved = __builtin_amdgcn_readfirstlane(nb) != kt_begin;
    kt_begin = __builtin_amdgcn_readfirstlane(nb);
    kt_end = __builtin_amdgcn_readfirstlane(ne);
    team_span();
    if (moved) {
      w = 0u;
      if (tb < te) {
        m0 = mask_of(tb);
        st.fetch(tb * kKeyTile);
        st.commit(a, xb, tok, tb * kKeyTile, tid, Ks(0), Vs(0));
        w = keep_word(tb, m0);
      }
      __syncthreads();
    }
  }
  // Nothing may still be in flight when the walk starts: otherwise the
  // compiler can carry a prologue load's register into the loop's wait
  // bookkeeping and make every tile's first product wait for the prefetch of
  // the next tile (costs nothing here: the first tile's commit has waited).
  __builtin_amdgcn_s_waitcnt(0);
  bool tainted = false;  // wave-uniform
  int cur = 0;
  for (int kt = tb; kt < kt_stop; kt += TEAMS) {
    const bool act = TEAMS == 1 || kt < te;  // a team with fewer tiles idles at its last step
    const bool more = kt + TEAMS < te;
    if (more) {
      m_next = mask_of(kt + TEAMS);
      st.fetch((kt + TEAMS) * kKeyTile);
    }
    if (act && !tainted && __ballot(w != 0u) != 0) {  // wave-uniform
      // S^T: K rows from LDS against the Q registers, two independent chains.
      f32x4 s0 = {0.0f, 0.0f, 0.0f, 0.0f}, s1 = {0.0f, 0.0f, 0.0f, 0.0f};
      {
        const float *Kc = Ks(cur);
        const f32x4 *k0p = reinterpret_cast<const f32x4 *>(&Kc[col * KS + d0]);
        const f32x4 *k1p = reinterpret_cast<const f32x4 *>(&Kc[(16 + col) * KS + d0]);
#pragma unroll
        for (int c = 0; c < QS / 4; ++c) {
          const f32x4 x0 = k0p[c], x1 = k1p[c];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            s0 = mfma_16x16x4(x0[e], qreg[4 * c + e], s0);
            s1 = mfma_16x16x4(x1[e], qreg[4 * c + e], s1);
          }
        }
      }
      if (__ballot(qin && w != 0xffffffffu) != 0) {
        // A tile some query of the wave keeps only in part: mask it.
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          s0[r] = ((w >> (4 * grp + r)) & 1u) ? s0[r] : -INFINITY;
          s1[r] = ((w >> (16 + 4 * grp + r)) & 1u) ? s1[r] : -INFINITY;
        }
      }
      f32x4 e0, e1;
      float rs = 0.0f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        e0[r] = fast_exp2(__builtin_fmaf(s0[r], c1, -m));
        e1[r] = fast_exp2(__builtin_fmaf(s1[r], c1, -m));
        rs += e0[r] + e1[r];
      }
      bool ok = true;
      if (__ballot(qin && !(rs <= kLazyLimit)) != 0) {
        // Move the reference where the tile max exceeds it by more than the
        // slack (the first tile always: m starts at kNoMax).
        const float mx = fmaxf(fmaxf(fmaxf(s0[0], s0[1]), fmaxf(s0[2], s0[3])),
                               fmaxf(fmaxf(s1[0], s1[1]), fmaxf(s1[2], s1[3])));
        const float mxs = pair_max(pair16_max(mx)) * c1;
        const bool need = mxs > m + kRescaleSlack;
        const float mn = need ? mxs : m;
        rs = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          e0[r] = fast_exp2(__builtin_fmaf(s0[r], c1, -mn));
          e1[r] = fast_exp2(__builtin_fmaf(s1[r], c1, -mn));
          rs += e0[r] + e1[r];
        }
        if (__ballot(qin && !__builtin_isfinite(rs)) != 0) {
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
        // A operand of block j: V[key 4*grp + r (+16)][d = 16*j + col], one
        // 16-byte read per 4 keys.
        const float *vb = &Vs(cur)[col * VS + 4 * grp];
#pragma unroll
        for (int j = 0; j < NB; ++j) {
          const f32x4 va = *reinterpret_cast<const f32x4 *>(vb + j * 16 * VS);
          const f32x4 vc = *reinterpret_cast<const f32x4 *>(vb + j * 16 * VS + 16);
#pragma unroll
          for (int r = 0; r < 4; ++r) O[j] = mfma_16x16x4(va[r], e0[r], O[j]);
#pragma unroll
          for (int r = 0; r < 4; ++r) O[j] = mfma_16x16x4(vc[r], e1[r], O[j]);
        }
      }
    }
    if (more) st.commit(a, xb, tok, (kt + TEAMS) * kKeyTile, tid, Ks(cur ^ 1), Vs(cur ^ 1));
    __syncthreads();
    if (more) w = keep_word(kt + TEAMS, m_next);
    cur ^= 1;
  }

  // -------- careful redo (rare): NaN / inf among this wave's kept scores
  // or values. Every wave's LDS reads of the walk precede its last barrier,
  // so the wave may now use its own slice of the LDS block.
  bool bad = false;
#pragma unroll
  for (int j = 0; j < NB; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) bad |= !__builtin_isfinite(O[j][r]);
  bool redo = tainted || __ballot(qin && bad) != 0;
  if constexpr (TEAMS > 1) {
    // Teams 1 .. TEAMS-1 hand their (m, l, O) for the same queries to team
    // 0 through LDS (the K/V buffers: every wave is past the walk's last
    // barrier), with their redo flags; team 0 merges them, or redoes the
    // whole span when any part met a non-finite value.
    constexpr int MF = 4 * NB + 2;  // floats per lane: O, m, l
    __shared__ int s_redo[TEAMS * 4];
    float *mg = smem + ((team - 1) * 4 + wave) * MF * 64;
    if (team > 0) {
#pragma unroll
      for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) mg[(4 * j + r) * 64 + lane] = O[j][r];
      mg[4 * NB * 64 + lane] = m;
      mg[(4 * NB + 1) * 64 + lane] = l;
    }
    if (lane == 0) s_redo[team * 4 + wave] = redo ? 1 : 0;
    __syncthreads();
    if (team > 0) return;
#pragma unroll
    for (int t = 1; t < TEAMS; ++t) redo |= s_redo[t * 4 + wave] != 0;
    if (!redo) {
      float M = m;
#pragma unroll
      for (int t = 1; t < TEAMS; ++t) M = fmaxf(M, smem[((t - 1) * 4 + wave) * MF * 64 + 4 * NB * 64 + lane]);
      const float f0 = fast_exp2(m - M);  // 1 for the part that holds the max
      l *= f0;
#pragma unroll
      for (int j = 0; j < NB; ++j) O[j] *= f0;
#pragma unroll
      for (int t = 1; t < TEAMS; ++t) {
        const float *src = smem + ((t - 1) * 4 + wave) * MF * 64;
        const float ft = fast_exp2(src[4 * NB * 64 + lane] - M);
        l += ft * src[(4 * NB + 1) * 64 + lane];
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) O[j][r] += ft * src[(4 * j + r) * 64 + lane];
      }
    }
  }
  if (redo) {
    // The kernel's LayaArgs (its first parameter, at offset 0 of the kernel
    // argument segment): passing the struct by value would copy it to
    // scratch.
    laya_redo_wave<HDP, MODE, ROPE>((const LayaArgs *)__builtin_amdgcn_kernarg_segment_ptr(), b,
                                    head, q0w, kt_begin, kt_end,
                                    smem + (TEAMS > 1 ? (TEAMS - 1) * 4 * (4 * NB + 2) * 64 : 0) +
                                        wave * kKeyTile * 17);
    return;
  }

  // -------- normalize and store: out[feat + d + hidden*(q + L*b)]
  // 0/0 gives NaN for a query that kept nothing, as the reference does.
  const float lt = pair_sum(pair16_sum(l));
  const float inv = lt > 0.0f ? fast_rcp(lt) : __builtin_nanf("");
  if (qin) {
    float *orow = a.out + ((size_t)b * L + q) * a.d + (size_t)head * hd;
    if constexpr (VEC) {
      // Block j holds dims 16j + 4*grp + 0..3: one 16-byte store each,
      // non-temporal: nothing in this kernel reads the output again, and
      // dirty L2 lines would be written back at the kernel's end (C2 kernel
      // 44.1 -> 42.7 us).
#pragma unroll
      for (int j = 0; j < NB; ++j)
        __builtin_nontemporal_store(O[j] * inv,
                                    reinterpret_cast<f32x4 *>(orow + 16 * j + 4 * grp));
    } else {
#pragma unroll
      for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int dd = 16 * j + 4 * grp + r;
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

__global__ __launch_bounds__(256) void add_row_bias_kernel(float *__restrict__ c,
                                                           const float *__restrict__ b, int m,
                                                           size_t total) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (size_t)gridDim.x * blockDim.x)
    c[i] += b[i % (size_t)m];
}

// ----------------------------------------------------------------- launchers

hipError_t launch_fill_zero(float *out, size_t n, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  size_t blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, out, n);
  return hipGetLastError();
}

hipError_t launch_add_row_bias(float *c, const float *b, int m, size_t n, hipStream_t stream) {
  const size_t total = (size_t)m * n;
  if (total == 0) return hipSuccess;
  size_t blocks = (total + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(add_row_bias_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, c, b, m,
                     total);
  return hipGetLastError();
}

hipError_t launch_laya_keep_bits(const uint8_t *keep, uint32_t *bits, uint8_t *any, int L, int B,
                                 int nkt, hipStream_t stream) {
  dim3 grid((L + 255) / 256, nkt, B);
  hipLaunchKernelGGL(laya_keep_bits_kernel, grid, dim3(256), 0, stream, keep, bits, any, L, nkt);
  return hipGetLastError();
}

hipError_t launch_laya_valid_prep(const uint8_t *valid, uint32_t *words, uint8_t *any, int L,
                                  int B, int nkt, int window, hipStream_t stream) {
  hipLaunchKernelGGL(laya_valid_prep_kernel, dim3((unsigned)((L + 63) / 64), (unsigned)B),
                     dim3(64), 0, stream, valid, words, any, L, nkt, window);
  return hipGetLastError();
}

template <int HDP, bool VEC, bool ROPE, int TEAMS, int QW>
static hipError_t launch_laya_teams(const LayaArgs &a, dim3 grid, int mode, hipStream_t stream,
                                    const KernelEvents &ev) {
  const dim3 block(64 * QW * TEAMS);
  if constexpr (TEAMS > 1) {
    if (mode == kMaskRaw) {
      hipExtLaunchKernelGGL((laya_attention_kernel<HDP, kMaskRaw, VEC, ROPE, false, TEAMS, QW>),
                            grid, block, 0, stream, ev.start, ev.stop, 0, a);
      return hipGetLastError();
    }
  }
  if (mode == kMaskRaw) return hipErrorInvalidValue;  // only the teams variant packs keep bytes
  if (mode == kMaskBits)
    hipExtLaunchKernelGGL((laya_attention_kernel<HDP, kMaskBits, VEC, ROPE, false, TEAMS, QW>),
                          grid, block, 0, stream, ev.start, ev.stop, 0, a);
  else if (a.bits != nullptr)
    hipExtLaunchKernelGGL((laya_attention_kernel<HDP, kMaskStruct, VEC, ROPE, true, TEAMS, QW>),
                          grid, block, 0, stream, ev.start, ev.stop, 0, a);
  else
    hipExtLaunchKernelGGL((laya_attention_kernel<HDP, kMaskStruct, VEC, ROPE, false, TEAMS, QW>),
                          grid, block, 0, stream, ev.start, ev.stop, 0, a);
  return hipGetLastError();
}

template <int HDP, bool VEC, bool ROPE>
static hipError_t launch_laya_hd(const LayaArgs &a, int heads, int batch, int mode,
                                 hipStream_t stream, const KernelEvents &ev) {
  const unsigned ng = (a.L + kLayaGroupQueries - 1) / kLayaGroupQueries;
  // A grid of at most one 64-query workgroup per CU would leave each CU one
  // wave per SIMD walking every key tile of its span, latency-bound: split
  // the span over teams of waves instead (four teams at hd <= 64, two at
  // 128, as the teams' K/V buffers fit in LDS), and where even half the CUs
  // would suffice, give each workgroup 32 queries (two waves per team), so
  // that every CU gets one.
  const long groups = (long)ng * heads * batch;
  if (!laya_teams_grid(a.L, heads, batch, a.nkt, a.cus) && mode == kMaskRaw)
    return hipErrorInvalidValue;
  if (a.cus > 0 && a.nkt > 1 && groups * 2 <= a.cus) {
    const dim3 grid((a.L + 2 * kLayaWaveQueries - 1) / (2 * kLayaWaveQueries), heads, batch);
    return launch_laya_teams<HDP, VEC, ROPE, laya_teams(HDP), 2>(a, grid, mode, stream, ev);
  }
  const dim3 grid(ng, heads, batch);
  if (laya_teams_grid(a.L, heads, batch, a.nkt, a.cus))
    return launch_laya_teams<HDP, VEC, ROPE, laya_teams(HDP), 4>(a, grid, mode, stream, ev);
  LayaArgs b = a;
  b.layout = 0;
  if (laya_xcd_layout((int)ng, heads, batch, laya_groups_per_cu(HDP), a.cus))
    b.layout = (a.any != nullptr && (int)ng * batch <= kLayaPlanMax) ? 2 : 1;
  b.ngdiv = FastDiv::make(ng);
  b.mdiv = FastDiv::make((uint32_t)(heads * (int)ng / 8 > 0 ? heads * (int)ng / 8 : 1));
  return launch_laya_teams<HDP, VEC, ROPE, 1, 4>(b, grid, mode, stream, ev);
}

template <int HDP>
static hipError_t launch_laya_pick(const LayaArgs &a, int heads, int batch, int mode,
                                   hipStream_t stream, const KernelEvents &ev) {
  // 16-byte row loads need hd == HDP, hd % 8 == 0 (RoPE halves in whole
  // chunks), a row stride of whole chunks and aligned bases.
  // Buffer loads also need one batch row of qkv within 2 GiB.
  const bool vec = a.hd == HDP && a.hd % 8 == 0 && a.d % 4 == 0 &&
                   (reinterpret_cast<uintptr_t>(a.qkv) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(a.out) & 15) == 0 &&
                   (size_t)a.L * 3 * (size_t)a.d * 4 < ((size_t)1 << 31);
  const bool rope = a.cos_t != nullptr;
  if (vec)
    return rope ? launch_laya_hd<HDP, true, true>(a, heads, batch, mode, stream, ev)
                : launch_laya_hd<HDP, true, false>(a, heads, batch, mode, stream, ev);
  return rope ? launch_laya_hd<HDP, false, true>(a, heads, batch, mode, stream, ev)
              : launch_laya_hd<HDP, false, false>(a, heads, batch, mode, stream, ev);
}

hipError_t launch_laya_attention(const LayaArgs &a, int heads, int batch, int hd_pad, int mode,
                                 hipStream_t stream, const KernelEvents &ev) {
  switch (hd_pad) {
    case 32: return launch_laya_pick<32>(a, heads, batch, mode, stream, ev);
    case 64: return launch_laya_pick<64>(a, heads, batch, mode, stream, ev);
    case 128: return launch_laya_pick<128>(a, heads, batch, mode, stream, ev);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace tfd
