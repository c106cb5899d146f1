// Jeff full attention, bf16 variant at head dim 256 (cpu-kernels
// jeff_full_attention_into, crates/cpu-kernels/src/lib.rs:609-763, with q, k,
// v and gate held in bf16), on the 32x32x16 matrix cores of gfx950: S^T on
// fp16 operands (normalized, rotated q and k scaled by powers of two,
// norm_weight_exp), P.V on bf16 operands (V as given). fp16 rounds q and k
// 8x finer than bf16: with bf16 scores a query that keeps two keys missed
// 1e-2 by up to 22% (V ~ N(0, 1)); the row sum adds the bf16-rounded
// probabilities P.V consumes, so the output is a convex combination of V.
//
// One workgroup = 8 wavefronts on one kv head, one workgroup per CU (two
// wavefronts per SIMD, 256 registers each), in two groups of four. A group
// owns one query tile: hw of the GQA group's query heads (4 when the group
// size allows it) x 4/hw sub-tiles of 32 queries; the workgroup's two tiles
// form a causal pair (2p, 2p + 1), so both walk about the same keys and
// share every 32-key tile of K and V staged in LDS. Each wavefront owns one
// block of 32 queries of one head and walks the key tiles:
//   S^T (32 keys x 32 queries) = K_tile . Q^T  (16 MFMAs, K from LDS, Q^T in
//                                               registers as fp16 B operands)
//   online softmax in the log2 domain against a lazily moved reference
//   O^T (256 x 32) += V_tile^T . P^T           (16 MFMAs, V from LDS)
// The walk runs in phases separated by workgroup barriers. A wavefront's
// step k is an MFMA half (P.V of tile k - 1 interleaved with S^T of tile k:
// every MFMA of the single S^T accumulator chain is followed by an
// independent P.V MFMA, which covers the chain's result latency) and a
// vector half (the softmax of tile k). Group 1 runs one phase behind group
// 0, so on every SIMD one wavefront keeps the matrix core busy while the
// other one does its softmax (exponentials, sums, bf16 packing), and the two
// trade roles at every barrier. Left to chance, as with two independent
// workgroups per CU, the two wavefronts of a SIMD reach their MFMA chains
// together as often as not.
//
// K and V move from global memory straight into LDS (buffer_load_dwordx4
// ... lds, no staging registers), four tiles deep, chunk-major in blocks of
// 16 rows, so that every 128-bit operand read is free of bank conflicts and
// addressed from one register per lane; each of the 8 wavefronts moves 4 of
// a tile's 32 one-KB pieces. The probabilities leave the S^T accumulators in
// the B operand layout of the P.V product except for one lane-half exchange
// per 8 keys (v_permlane32_swap). (Two query blocks per wavefront, so that
// each operand read feeds two MFMAs, would need 64 queries x 256 features of
// O^T plus their Q operands: more than the 512 registers of one wavefront per
// SIMD.)
//
// Non-finite values take another route: a group whose kept scores sum to
// NaN/inf, or whose output came out non-finite (a NaN/inf value, also one
// multiplied by a zero probability), writes no output and raises its flags;
// jeff_bf16_exact_kernel then recomputes the flagged tiles with the
// reference's exact semantics (masked or zero-probability values never
// leak, NaN scores weigh 0, a +inf score empties its row).
#include "jeff_common.hpp"
#include "tfd_device.hpp"
#include "tfd_internal.hpp"

namespace tfd {

namespace {

constexpr int kWideHd = 256;      // head dim (fixed)
constexpr int kWideKeys = 32;     // keys per tile
constexpr int kWideWaves = 4;     // wavefronts per group (two groups)
constexpr int kWideQueries = 32;  // queries per wavefront
constexpr int kWideStages = 4;    // K/V tiles resident in LDS
// Staged tiles, 16-byte chunks (8 bf16): K as 2 blocks of 16 keys x 32
// chunks, V as 16 blocks of 16 features x 4 chunks, each block chunk-major
// (chunk c of row i at c * 256 + 16 * i within its block).
constexpr int kKBlock = 32 * 256;    // bytes of 16 keys x 256 features
constexpr int kKBuf = 2 * kKBlock;   // 16 KB
constexpr int kVBlock = 4 * 256;     // bytes of 16 features x 32 keys
constexpr int kVBuf = 16 * kVBlock;  // 16 KB
constexpr int kStage = kKBuf + kVBuf;
// A lane's 16 terms of a tile, taken against the current reference, summing
// to at most this (16 * 2^kRescaleSlack) need no new reference.
constexpr float kLazyLimit16 = 4096.0f;

__device__ __forceinline__ f32x16 mfma_32x32x16_bf16(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma_32x32x16_f16(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// This lane's index, recomputed where it is used (two vector instructions,
// opaque to the compiler): the walk needs it only for the last tile's
// clamped addresses, and a lane index kept live across the walk is what the
// compiler spills first.
__device__ __forceinline__ int lane_now() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

// Orders the scheduling region it ends (a straight run of n LDS operand
// reads, each feeding one MFMA, n > kReadAhead): kReadAhead reads, then
// alternately one MFMA and one read, then the last kReadAhead MFMAs. Left
// alone, the scheduler issues two reads at a time and every MFMA waits out
// the LDS latency of its operand.
constexpr int kReadAhead = 4;
template <int n>
__device__ __forceinline__ void pipeline_reads() {
  static_assert(n > kReadAhead, "more reads than the read-ahead");
  __builtin_amdgcn_sched_group_barrier(0x100, kReadAhead, 0);  // DS reads
#pragma unroll
  for (int i = 0; i < n - kReadAhead; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
  }
  __builtin_amdgcn_sched_group_barrier(0x008, kReadAhead, 0);
}

// Two f32 rounded to bf16 (nearest even, as f32_to_bf16) in one register,
// lo in the low half: one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, bf16x2));
}

// Sum of the 16 bf16 values packed two per word in g, in f32 (each half
// moved into the high half of a word is that value as an f32; two chains):
// the row sum of exactly the probabilities the P.V product consumes. (One
// v_dot2 per word against 1.0 does the same in fewer instructions but
// measured 4% slower on C5.)
__device__ __forceinline__ float sum_bf16x16(const uint32_t (&g)[8]) {
  float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    s0 += __uint_as_float(g[i] << 16);
    s1 += __uint_as_float(g[i] & 0xffff0000u);
  }
  return s0 + s1;
}

// Heads per group: 4, 2 or 1, whichever divides the GQA group size.
int wide_heads_per_group(const JeffArgs &a) {
  const int G = a.heads / a.kv_heads;
  return G % 4 == 0 ? 4 : (G % 2 == 0 ? 2 : 1);
}

}  // namespace

bool jeff_bf16_wide_fits(const JeffArgs &a) {
  const int G = a.kv_heads > 0 ? a.heads / a.kv_heads : 0;
  const bool rope_ok = a.cos_t == nullptr || a.rot_half == 16 || a.rot_half == 32;
  // Buffer loads address one (row, kv head)'s K and V with 32-bit offsets.
  const bool offsets_ok = (size_t)a.L * kWideHd * 2 < ((size_t)1 << 31);
  return a.hd == kWideHd && G >= 1 && a.heads == G * a.kv_heads && rope_ok && a.L >= 8 &&
         offsets_ok && a.L % 8 == 0 && (reinterpret_cast<uintptr_t>(a.v) & 15) == 0 &&
         (reinterpret_cast<uintptr_t>(a.q_norm) & 15) == 0;
}

int jeff_bf16_wide_query_tile(const JeffArgs &a) {
  return kWideQueries * (kWideWaves / wide_heads_per_group(a));
}

size_t jeff_bf16_wide_flag_count(const JeffArgs &a, int rows) {
  const int qt = jeff_bf16_wide_query_tile(a);
  return (size_t)rows * a.heads * ((a.L + qt - 1) / qt);
}

// Work item p: query tile pair qt2 (longest first), then unit u = (row, kv
// head, head group); the units of one pair are consecutive, so their K/V
// streams land on few XCDs and meet in L2. kbits: one bit per key, mask != 0
// (jeff_k_prep_kernel).
__global__ __launch_bounds__(512, 1) void jeff_bf16_wide_kernel(const JeffArgs a,
                                                                const uint16_t *__restrict__ kp,
                                                                const uint32_t *__restrict__ kbits,
                                                                int *__restrict__ flags, int rows,
                                                                int hw) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[kWideStages * kStage];
  __shared__ int s_flag[2];
  __shared__ int s_span[2];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // 0..7
  const int grp = wave >> 2, w4 = wave & 3;
  const int col = lane & 31, half = lane >> 5;
  const int L = a.L, G = a.heads / a.kv_heads;
  const int ngrp = G / hw;
  const int QT = kWideQueries * (kWideWaves / hw);
  const int nqt = (L + QT - 1) / QT, nqt2 = (nqt + 1) / 2;
  const int units = rows * a.kv_heads * ngrp;
  const int p = blockIdx.x;
  const int qt2 = nqt2 - 1 - p / units;
  const int u = p % units;
  const int row = u / (a.kv_heads * ngrp);
  const int kvh = (u / ngrp) % a.kv_heads;
  const int head = kvh * G + (u % ngrp) * hw + w4 % hw;
  const int qt = 2 * qt2 + grp;
  const int q0w = qt * QT + (w4 / hw) * kWideQueries;
  const int qv = q0w + col;

  const uint16_t *Qh =
      static_cast<const uint16_t *>(a.q) + row * a.q_row + (size_t)head * kWideHd * L;
  const uint16_t *Gh =
      static_cast<const uint16_t *>(a.gate) + row * a.q_row + (size_t)head * kWideHd * L;
  const uint16_t *Vh =
      static_cast<const uint16_t *>(a.v) + row * a.kv_row + (size_t)kvh * a.kv_head;
  const uint16_t *Kh = kp + ((size_t)row * a.kv_heads + kvh) * (size_t)L * kWideHd;
  float *Oh = a.out + row * a.q_row + (size_t)head * kWideHd * L;
  const int nw = (L + 31) / 32;
  const uint32_t *rbits = kbits + (size_t)row * nw;

  // -------- the row's active span (first and last key with mask != 0),
  // from its key bits; the walk covers its tiles up to the workgroup's last
  // query (causal).
  if (tid == 0) {
    s_span[0] = 0x7fffffff;
    s_span[1] = -1;
  }
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  {
    int lo = 0x7fffffff, hi = -1;
    for (int w = tid; w < nw; w += 2 * kWideWaves * 64) {
      const uint32_t b = rbits[w];
      if (b != 0) {
        lo = min(lo, 32 * w + __builtin_ctz(b));
        hi = max(hi, 32 * w + 31 - __builtin_clz(b));
      }
    }
    lo = wave_min(lo);
    hi = wave_max(hi);
    if (lane == 0) {
      atomicMin(&s_span[0], lo);
      atomicMax(&s_span[1], hi);
    }
  }
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  const int last = s_span[1], first = last >= 0 ? s_span[0] : 0;
  const int start = (a.trim && last >= 0) ? first : 0;
  const bool q_live = qv < L && qv >= start;
  const int q_last_wg = min((2 * qt2 + 2) * QT - 1, L - 1);
  int kt_begin = 0, kt_end = 0;
  if (last >= 0 && first <= min(last, q_last_wg)) {
    kt_begin = first / kWideKeys;
    kt_end = min(last, q_last_wg) / kWideKeys + 1;
  }
  // This wavefront's 32 queries: the last tile with a key at or before one
  // of them, and whether some / all of them are live.
  const int kt_w_end = q0w < L ? min(kt_end, min(last, q0w + 31) / kWideKeys + 1) : kt_begin;
  const bool w_live = q0w < L && q0w + 31 >= start;
  const bool w_full = q0w >= start && q0w + 32 <= L;

  // -------- Q: RMSNorm (lib.rs:676-691) and partial RoPE (692-709) in f32,
  // times 2^-e_q, rounded to fp16 B operands (the prepared keys are fp16
  // times 2^-e_k; norm_weight_exp): lane (col, half) holds features
  // 16s + 8*half + e of query qv in qb[s]. RoPE partners (i, i + rot/2) sit
  // in the same lane, rot/32 steps apart.
  const int eq = norm_weight_exp(a.q_norm, kWideHd, lane);
  const float qsig = ldexpf(1.0f, -eq);
  const float c1 = ldexpf(a.c1, eq + norm_weight_exp(a.k_norm, kWideHd, lane));
  f16x8 qb[16];
  const int rh = a.cos_t != nullptr ? a.rot_half : 0;
  {
    const int qc = min(qv, L - 1);
    float y[16][8];
    float ss = 0.0f;
#pragma unroll
    for (int s = 0; s < 16; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        y[s][e] = bf16_to_f32(Qh[(size_t)(16 * s + 8 * half + e) * L + qc]);
        ss += y[s][e] * y[s][e];
      }
    ss = pair_sum(ss);  // the other 128 features sit in lane ^ 32
    const float scale = rms_scale(ss, kWideHd, a.eps);
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      const f32x4 w0 = *reinterpret_cast<const f32x4 *>(a.q_norm + 16 * s + 8 * half);
      const f32x4 w1 = *reinterpret_cast<const f32x4 *>(a.q_norm + 16 * s + 8 * half + 4);
#pragma unroll
      for (int e = 0; e < 8; ++e) y[s][e] = rms_apply(y[s][e], scale, e < 4 ? w0[e] : w1[e - 4]);
    }
    const size_t pos = (size_t)min(max(qv - start, 0), L - 1) * (size_t)(rh > 0 ? rh : 1);
    auto rotate = [&](float (&lo)[8], float (&hi)[8], int s) {
      const int i0 = 16 * s + 8 * half;
      const f32x4 c0 = *reinterpret_cast<const f32x4 *>(a.cos_t + pos + i0);
      const f32x4 c1v = *reinterpret_cast<const f32x4 *>(a.cos_t + pos + i0 + 4);
      const f32x4 n0 = *reinterpret_cast<const f32x4 *>(a.sin_t + pos + i0);
      const f32x4 n1 = *reinterpret_cast<const f32x4 *>(a.sin_t + pos + i0 + 4);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float c = e < 4 ? c0[e] : c1v[e - 4], sn = e < 4 ? n0[e] : n1[e - 4];
        const float xl = lo[e], xh = hi[e];
        lo[e] = rope_lo(xl, xh, c, sn);
        hi[e] = rope_hi(xl, xh, c, sn);
      }
    };
    if (q_live && rh == 32) {
      rotate(y[0], y[2], 0);
      rotate(y[1], y[3], 1);
    } else if (q_live && rh == 16) {
      rotate(y[0], y[1], 0);
    }
#pragma unroll
    for (int s = 0; s < 16; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) qb[s][e] = (_Float16)(q_live ? y[s][e] * qsig : 0.0f);
  }

  // -------- staging of local tile j (keys 32 (kt_begin + j) ..) into buffer
  // j mod 4: a tile is 32 one-KB loads (K: 2 blocks x 8 instructions of 4
  // chunks; V: 16 blocks), wavefront w issues K instructions 2w, 2w + 1
  // (block i >> 3, chunks 4 (i & 7) ..) and V blocks 2w, 2w + 1. A lane
  // moves 16 bytes: row lane & 15, chunk lane >> 4 of its instruction.
  const int si = lane & 15, sc = lane >> 4;
  const uint32_t klane = (uint32_t)(si * kWideHd * 2 + sc * 16);
  const uint32_t vlane = (uint32_t)(si * L * 2 + sc * 16);
  const u32x4r rk = rsrc_words(Kh, (uint32_t)((size_t)L * kWideHd * 2));
  const u32x4r rv = rsrc_words(Vh, (uint32_t)((size_t)L * kWideHd * 2));
  auto buf = [&](int j) { return lds + (j & (kWideStages - 1)) * kStage; };
  auto stage = [&](int j) {
    unsigned char *Kb = buf(j);
    unsigned char *Vb = Kb + kKBuf;
    const int k0 = (kt_begin + j) * kWideKeys;
    if (k0 + kWideKeys <= L) {
#pragma unroll
      for (int n = 0; n < 2; ++n) {
        const int i = 2 * wave + n, B = i >> 3, c0 = 4 * (i & 7);
        load_lds16(rk, klane, (uint32_t)(((k0 + 16 * B) * kWideHd + 8 * c0) * 2),
                   Kb + B * kKBlock + c0 * 256);
      }
#pragma unroll
      for (int n = 0; n < 2; ++n) {
        const int B = 2 * wave + n;
        load_lds16(rv, vlane, (uint32_t)((16 * B * L + k0) * 2), Vb + B * kVBlock);
      }
    } else {
      // The last, partial tile: keys clamped to L - 1 (their scores are
      // masked), V chunks clamped to the last 8 keys.
      const int ln = lane_now(), li = ln & 15, lc = ln >> 4;
#pragma unroll
      for (int n = 0; n < 2; ++n) {
        const int i = 2 * wave + n, B = i >> 3, c0 = 4 * (i & 7);
        const int key = min(k0 + 16 * B + li, L - 1);
        load_lds16(rk, (uint32_t)((key * kWideHd + 8 * (c0 + lc)) * 2), 0u,
                   Kb + B * kKBlock + c0 * 256);
      }
#pragma unroll
      for (int n = 0; n < 2; ++n) {
        const int B = 2 * wave + n;
        load_lds16(rv, (uint32_t)(((16 * B + li) * L + min(k0 + 8 * lc, L - 8)) * 2), 0u,
                   Vb + B * kVBlock);
      }
    }
  };
  // Operand addresses: lane (col, half) reads K row col (block col >> 4),
  // chunks 2s + half, and V feature row col of each 32-feature block.
  const int kbase = (col >> 4) * kKBlock + half * 256 + (col & 15) * 16;
  const int vbase = (col >> 4) * kVBlock + half * 256 + (col & 15) * 16;

  f32x16 O[8];
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) O[j][r] = 0.0f;
  float m = kNoMax, l = 0.0f;
  bool tainted = false;  // wave-uniform
  f32x16 st = {};
  bf16x8 pb[2] = {};

  const int T = kt_end - kt_begin;
  if (T > 0) stage(0);
  if (T > 1) stage(1);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if (tid < 2) s_flag[tid] = 0;
  __syncthreads();

  // Steps this wavefront computes: tiles 0 .. kw - 1 of the walk (none
  // after a tile came out non-finite: the exact pass redoes the wavefront).
  int kw = w_live ? max(kt_w_end - kt_begin, 0) : 0;

  // -------- the softmax of local tile k (scores in st) into the P^T
  // operands pb (lib.rs:712-730), against the reference m. The row sum l
  // adds the bf16-rounded terms that P.V consumes, so that O / l is a convex
  // combination of V, as the reference's p = e / sum is (lib.rs:731-754).
  auto softmax = [&](int k) {
    const int kt = kt_begin + k, k0 = kt * kWideKeys;
    const uint32_t wact = rbits[kt];
    float e[16];
    uint32_t g[8];
    const uint32_t keep = q_live ? (wact & range_bits(0, qv - k0)) : 0u;
    const uint32_t kh = keep >> (4 * half);  // bit 8g + r: key 8g + 4*half + r
    const bool full = w_full && wact == 0xffffffffu && k0 + kWideKeys - 1 <= q0w;
    auto bit = [](uint32_t w, int r) { return ((w >> (8 * (r >> 2) + (r & 3))) & 1u) != 0u; };
    // Lane (col, half) holds S^T rows (keys) 8g + 4*half + r' of query col
    // in st[4g + r'].
    if (full) {
#pragma unroll
      for (int r = 0; r < 16; ++r) e[r] = fast_exp2(__builtin_fmaf(st[r], c1, -m));
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r)
        e[r] = bit(kh, r) ? fast_exp2(__builtin_fmaf(st[r], c1, -m)) : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) g[i] = pack_bf16x2(e[2 * i], e[2 * i + 1]);
    float rs = sum_bf16x16(g);
    if (__ballot(q_live && !(rs <= kLazyLimit16)) != 0) {
      // Rare: a score far above the reference (or non-finite). Move the
      // reference to the tile's maximum and redo the terms; -inf scores and
      // masked keys weigh 0. The keep bits go through an opaque copy so that
      // the common path above does not hold them.
      uint32_t kr;
      asm volatile("v_mov_b32 %0, %1" : "=v"(kr) : "v"(full ? 0xffffffffu : kh));
      auto kept = [&](int r) { return bit(kr, r); };
      float mx = -INFINITY;
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, kept(r) ? st[r] : -INFINITY);
      const float mxs = pair_max(mx) * c1;
      const float mn = mxs > m + kRescaleSlack ? mxs : m;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float x = st[r];
        e[r] = (!kept(r) || (__builtin_isinf(x) && x < 0.0f))
                   ? 0.0f
                   : fast_exp2(__builtin_fmaf(x, c1, -mn));
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) g[i] = pack_bf16x2(e[2 * i], e[2 * i + 1]);
      rs = sum_bf16x16(g);
      if (__ballot(q_live && !__builtin_isfinite(rs)) != 0) {
        tainted = true;
        kw = 0;
      } else if (__ballot(mn != m) != 0) {
        const float alpha = fast_exp2(m - mn);  // exactly 1 where m stays
        if (__ballot(l != 0.0f) != 0) {
#pragma unroll
          for (int j = 0; j < 8; ++j) O[j] *= alpha;
        }
        l *= alpha;
        m = mn;
      }
    }
    l += rs;
    // P^T as the B operand of O^T += V^T . P^T: lane (col, half) needs keys
    // 8*half .. 8*half + 7 of each 16-key half hh; it holds keys 4*half + r'
    // of each 8-key group. One permlane32 swap per pair of 8-key groups.
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      uint32_t w[4];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const auto r = __builtin_amdgcn_permlane32_swap(g[4 * hh + i], g[4 * hh + 2 + i],
                                                        false, false);
        w[i] = r[0];
        w[2 + i] = r[1];
      }
      pb[hh] = __builtin_bit_cast(
          bf16x8, (__attribute__((ext_vector_type(4))) uint32_t){w[0], w[1], w[2], w[3]});
    }
  };
  // The V operands of the first two P.V MFMAs of tile k (blocks O[0] and
  // O[1], first key half), read at the end of the vector half so that the
  // next MFMA half starts without waiting on LDS; tile k is complete then.
  bf16x8 vpre0, vpre1;
  auto pre_read = [&](int k) {
    const unsigned char *Vb = buf(k) + kKBuf;
    vpre0 = *reinterpret_cast<const bf16x8 *>(Vb + vbase);
    vpre1 = *reinterpret_cast<const bf16x8 *>(Vb + vbase + 2 * kVBlock);
  };
  // End of an MFMA half: this wavefront's loads of the next tile are in LDS
  // and its operand reads are done.
  auto mfma_end = [&]() {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  };

  // -------- the walk. Group 1 runs one phase behind group 0: one barrier
  // more before the walk, one fewer after it. Step k: the MFMA half (P.V of
  // tile k - 1 and S^T of tile k), then the vector half (staging tile k + 2
  // into the buffer tile k - 2 left, whose last reader, group 1's P.V, ran
  // in the phase before; the softmax of tile k). Each wavefront waits for
  // its share of tile k + 1 at the end of its MFMA half of step k, before
  // the barrier that precedes the tile's first read (group 0's S^T in step
  // k + 1). Every barrier is reached by all eight wavefronts: the number of
  // steps T is the workgroup's.
  if (grp == 1) asm volatile("s_barrier" ::: "memory");
  {
    const bool sk = 0 < kw;
    if (sk) {
      const unsigned char *Kb = buf(0);
      st = f32x16{};
#pragma unroll
      for (int s = 0; s < 16; ++s) {
        const f16x8 ka = *reinterpret_cast<const f16x8 *>(Kb + kbase + s * 512);
        st = mfma_32x32x16_f16(ka, qb[s], st);
      }
      pipeline_reads<16>();
    }
    mfma_end();
    if (2 < T) stage(2);
    if (sk) softmax(0);
    pre_read(0);
    asm volatile("s_barrier" ::: "memory");
  }
  for (int k = 1; k <= T; ++k) {
    const bool pv = k <= kw, sk = k < kw;
    if (pv) {
      // P.V(k - 1) and S^T(k) interleaved. Past this wavefront's last tile
      // (sk false) the S^T products read a stale buffer and are not used.
      const unsigned char *Vb = buf(k - 1) + kKBuf;
      const unsigned char *Kb = buf(k);
      // P.V order: O blocks (0, 1) of key half 0 from the pre-read, then
      // (0, 1) of half 1, (2, 3) of half 0, (2, 3) of half 1, ...
      constexpr int kPj[16] = {0, 1, 0, 1, 2, 3, 2, 3, 4, 5, 4, 5, 6, 7, 6, 7};
      constexpr int kPh[16] = {0, 0, 1, 1, 0, 0, 1, 1, 0, 0, 1, 1, 0, 0, 1, 1};
      st = f32x16{};
      O[0] = mfma_32x32x16_bf16(vpre0, pb[0], O[0]);
      O[1] = mfma_32x32x16_bf16(vpre1, pb[0], O[1]);
#pragma unroll
      for (int s = 0; s < 16; ++s) {
        const f16x8 ka = *reinterpret_cast<const f16x8 *>(Kb + kbase + s * 512);
        st = mfma_32x32x16_f16(ka, qb[s], st);
        if (s < 14) {
          const int q = s + 2;
          const bf16x8 va = *reinterpret_cast<const bf16x8 *>(Vb + vbase + kPj[q] * 2 * kVBlock +
                                                              kPh[q] * 512);
          O[kPj[q]] = mfma_32x32x16_bf16(va, pb[kPh[q]], O[kPj[q]]);
        }
      }
      // Four operand reads in flight: the two pre-read MFMAs go first.
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);  // DS reads
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // MFMA
#pragma unroll
      for (int i = 0; i < 26; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
    }
    mfma_end();
    if (k + 2 < T) stage(k + 2);
    if (sk) softmax(k);
    pre_read(k);
    asm volatile("s_barrier" ::: "memory");
  }
  if (grp == 0) asm volatile("s_barrier" ::: "memory");

  // -------- o / sum (0 when nothing was kept), sigmoid gate, store
  // (lib.rs:731-758). A non-finite output is left to the exact pass.
  bool bad = tainted;
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) bad |= q_live && !__builtin_isfinite(O[j][r]);
  if (__ballot(bad) != 0 && lane == 0) s_flag[grp] = 1;
  __syncthreads();
  const bool flagged = s_flag[grp] != 0;
  // One flag per (row, head, query tile): wavefronts 0 .. hw-1 of a group
  // hold its heads.
  if (lane == 0 && w4 < hw && qt < nqt)
    flags[((size_t)row * a.heads + head) * nqt + qt] = flagged ? 1 : 0;
  if (flagged || qv >= L) return;
  const float lt = pair_sum(l);
  const float inv = lt > 0.0f ? fast_rcp(lt) : 0.0f;
  const bool dropped = a.trim && qv < start;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    float gv[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int f = 32 * j + 8 * (r >> 2) + 4 * half + (r & 3);
      gv[r] = bf16_to_f32(Gh[(size_t)f * L + qv]);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int f = 32 * j + 8 * (r >> 2) + 4 * half + (r & 3);
      // Non-temporal: the output is not read again in the kernel.
      __builtin_nontemporal_store(dropped ? 0.0f : O[j][r] * inv * fast_sigmoid(gv[r]),
                                  &Oh[(size_t)f * L + qv]);
    }
  }
}

hipError_t launch_jeff_bf16_wide(const JeffArgs &a, int rows, const uint16_t *kp,
                                 const uint32_t *kbits, int *flags, hipStream_t stream) {
  const int hw = wide_heads_per_group(a);
  const int qt = jeff_bf16_wide_query_tile(a);
  const int units = rows * a.kv_heads * (a.heads / a.kv_heads / hw);
  const int nqt = (a.L + qt - 1) / qt;
  const unsigned grid = (unsigned)(units * ((nqt + 1) / 2));
  hipLaunchKernelGGL(jeff_bf16_wide_kernel, dim3(grid), dim3(512), 0, stream, a, kp, kbits, flags,
                     rows, hw);
  return hipGetLastError();
}

}  // namespace tfd
