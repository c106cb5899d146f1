// Jeff full attention, bf16 variant at head dim 256 (cpu-kernels
// jeff_full_attention_into, crates/cpu-kernels/src/lib.rs:609-763, with q, k,
// v and gate held in bf16), on the 32x32x16 bf16 matrix cores of gfx950.
//
// One workgroup = 4 wavefronts on one kv head: hw of the group's query heads
// (4 when the GQA group size allows it) x 4/hw sub-tiles of 32 queries, so a
// 32-key tile of K and V staged in LDS serves 128 (query, head) rows; two
// workgroups per CU (two wavefronts per SIMD, 256 registers each). Each
// wavefront owns one block of 32 queries of one head and walks the key
// tiles:
//   S^T (32 keys x 32 queries) = K_tile . Q^T  (16 MFMAs, K from LDS, Q^T in
//                                               registers as bf16 B operands)
//   online softmax in the log2 domain against a lazily moved reference
//   O^T (256 x 32) += V_tile^T . P^T           (16 MFMAs, V from LDS)
// with four operand reads from LDS kept in flight ahead of each MFMA chain.
// The probabilities leave the S^T accumulators in the B operand layout of
// the P.V product except for one lane-half exchange per 8 keys
// (v_permlane32_swap). K and V move from global memory straight into LDS
// (buffer_load_dwordx4 ... lds, no staging registers), double-buffered,
// chunk-major in blocks of 16 rows, so that every 128-bit operand read is
// free of bank conflicts and addressed from one register per lane. (Two
// query blocks per wavefront, so that each operand read feeds two MFMAs,
// would need 64 queries x 256 features of O^T plus their Q operands: more
// than the 512 registers of one wavefront per SIMD.)
//
// Non-finite values take another route: a workgroup whose kept scores sum to
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

constexpr int kWideHd = 256;     // head dim (fixed)
constexpr int kWideKeys = 32;    // keys per tile
constexpr int kWideWaves = 4;    // wavefronts per workgroup
constexpr int kWideBlocks = 1;   // 32-query blocks per wavefront
constexpr int kWideQueries = 32 * kWideBlocks;  // queries per wavefront
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

// 16 bytes at byte voff + soff of buffer r into LDS: lane i of the wavefront
// writes lds_base + 16*i (lds_base and soff the same for the whole
// wavefront). The buffer form keeps the per-lane address in one 32-bit
// register (the global form needs a 64-bit address per load, which the
// compiler ends up spilling, and every reload's wait would then also wait
// for the loads to LDS issued before it).
__device__ __forceinline__ void load_lds16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                           unsigned char *lds_base) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds_base,
                                           16, (int)voff, (int)soff, 0, 0);
}

// This lane's index, recomputed where it is used (two vector instructions,
// opaque to the compiler): the walk needs it only for the mask and the last
// tile's clamped addresses, and a lane index kept live across the walk is
// what the compiler spills first (its reload then waits on every load to
// LDS issued before it).
__device__ __forceinline__ int lane_now() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

// Orders the scheduling region it ends (a straight run of n LDS operand
// reads, each feeding one MFMA, n > kReadAhead): kReadAhead reads, then
// alternately one MFMA and one read, then the last kReadAhead MFMAs.
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

// Heads per workgroup: 4, 2 or 1, whichever divides the GQA group size.
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

// Work item p: query tile qt (longest first), then unit u = (row, kv head,
// head group); the units of one tile are consecutive, so their K/V streams
// land on few XCDs and meet in L2.
__global__ __launch_bounds__(256, kWideBlocks == 1 ? 2 : 1) void jeff_bf16_wide_kernel(const JeffArgs a,
                                                                const uint16_t *__restrict__ kp,
                                                                int *__restrict__ flags,
                                                                int rows, int hw) {
  constexpr int NB = kWideBlocks;
  __shared__ __attribute__((aligned(16))) unsigned char lds[2 * kStage];
  __shared__ int s_span[2];
  __shared__ int s_flag;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31, half = lane >> 5;
  const int L = a.L, G = a.heads / a.kv_heads;
  const int ngrp = G / hw;  // head groups per kv head
  const int QT = kWideQueries * (kWideWaves / hw);
  const int nqt = (L + QT - 1) / QT;
  const int units = rows * a.kv_heads * ngrp;
  const int p = blockIdx.x;
  const int qt = nqt - 1 - p / units;
  const int u = p % units;
  const int row = u / (a.kv_heads * ngrp);
  const int kvh = (u / ngrp) % a.kv_heads;
  const int head = kvh * G + (u % ngrp) * hw + wave % hw;
  const int q0w = qt * QT + (wave / hw) * kWideQueries;  // block b: q0w + 32b
  int qv[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) qv[b] = q0w + 32 * b + col;

  const float *maskr = a.mask + (size_t)row * L;
  const uint16_t *Qh =
      static_cast<const uint16_t *>(a.q) + row * a.q_row + (size_t)head * kWideHd * L;
  const uint16_t *Gh =
      static_cast<const uint16_t *>(a.gate) + row * a.q_row + (size_t)head * kWideHd * L;
  const uint16_t *Vh =
      static_cast<const uint16_t *>(a.v) + row * a.kv_row + (size_t)kvh * a.kv_head;
  const uint16_t *Kh = kp + ((size_t)row * a.kv_heads + kvh) * (size_t)L * kWideHd;
  float *Oh = a.out + row * a.q_row + (size_t)head * kWideHd * L;

  // -------- the row's active span (mask != 0), one pass of the workgroup.
  if (tid == 0) {
    s_span[0] = 0x7fffffff;
    s_span[1] = -1;
    s_flag = 0;
  }
  __syncthreads();
  {
    int lo = 0x7fffffff, hi = -1;
    for (int k0 = 0; k0 < L; k0 += 256 * 8) {
      float v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = maskr[min(k0 + tid + 256 * i, L - 1)];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int k = k0 + tid + 256 * i;
        if (k < L && v[i] != 0.0f) {
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
  __syncthreads();
  const int first = s_span[0], last = s_span[1];
  const int start = (a.trim && last >= 0) ? first : 0;
  bool q_live[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) q_live[b] = qv[b] < L && qv[b] >= start;
  const int q_last_wg = min(qt * QT + QT - 1, L - 1);
  int kt_begin = 0, kt_end = 0;
  if (last >= 0 && first <= min(last, q_last_wg)) {
    kt_begin = first / kWideKeys;
    kt_end = min(last, q_last_wg) / kWideKeys + 1;
  }

  // -------- Q: RMSNorm (lib.rs:676-691) and partial RoPE (692-709) in f32,
  // rounded to bf16 B operands: lane (col, half) holds features
  // 16s + 8*half + e of query q0w + 32b + col in qb[b][s]. RoPE partners
  // (i, i + rot/2) sit in the same lane, rot/32 steps apart.
  bf16x8 qb[NB][16];
  const int rh = a.cos_t != nullptr ? a.rot_half : 0;
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const int qc = min(qv[b], L - 1);
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
    const size_t pos = (size_t)min(max(qv[b] - start, 0), L - 1) * (size_t)(rh > 0 ? rh : 1);
    // Steps s < rot/32 hold pairs i = 16s + 8*half + e, step s + rot/32
    // their partners i + rot/2.
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
    if (q_live[b] && rh == 32) {
      rotate(y[0], y[2], 0);
      rotate(y[1], y[3], 1);
    } else if (q_live[b] && rh == 16) {
      rotate(y[0], y[1], 0);
    }
#pragma unroll
    for (int s = 0; s < 16; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) qb[b][s][e] = (__bf16)(q_live[b] ? y[s][e] : 0.0f);
  }

  // -------- staging (tile of keys k0 .. k0+31): chunk c of key k0 + 16B + i
  // to K block B, chunk c of V feature 16B + i to V block B. One 1 KB
  // instruction fills 4 chunks x 16 rows of a block; wavefront w moves K
  // chunks 8w .. 8w+7 of both blocks and V blocks 4w .. 4w+3. A whole tile
  // addresses every row from one uniform base and a fixed lane offset; in
  // the row's last, partial tile keys past L repeat the last key (its keep
  // bit is 0).
  const int si = lane & 15, sc = lane >> 4;  // row, chunk within an instruction
  const uint32_t klane = (uint32_t)(si * kWideHd * 2 + sc * 16);
  const uint32_t vlane = (uint32_t)(si * L * 2 + sc * 16);
  // One (row, kv head)'s prepared K (L x 256) and V (256 x L), bf16 (each
  // under 2 GiB: jeff_bf16_wide_fits).
  const __amdgpu_buffer_rsrc_t rk = buffer_rsrc(Kh, (uint32_t)((size_t)L * kWideHd * 2));
  const __amdgpu_buffer_rsrc_t rv = buffer_rsrc(Vh, (uint32_t)((size_t)L * kWideHd * 2));
  auto stage = [&](int kt, int buf) {
    unsigned char *Kb = lds + buf * kStage;
    unsigned char *Vb = Kb + kKBuf;
    const int k0 = kt * kWideKeys;
    if (k0 + kWideKeys <= L) {
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        const int B = n >> 1, c0 = 8 * wave + 4 * (n & 1);
        load_lds16(rk, klane, (uint32_t)(((k0 + 16 * B) * kWideHd + 8 * c0) * 2),
                   Kb + B * kKBlock + c0 * 256);
      }
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        const int B = 4 * wave + n;
        load_lds16(rv, vlane, (uint32_t)((16 * B * L + k0) * 2), Vb + B * kVBlock);
      }
    } else {
      const int ln = lane_now(), si = ln & 15, sc = ln >> 4;
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        const int B = n >> 1, c0 = 8 * wave + 4 * (n & 1);
        const int key = min(k0 + 16 * B + si, L - 1);
        load_lds16(rk, (uint32_t)((key * kWideHd + 8 * (c0 + sc)) * 2), 0u,
                   Kb + B * kKBlock + c0 * 256);
      }
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        const int B = 4 * wave + n;
        load_lds16(rv, (uint32_t)(((16 * B + si) * L + min(k0 + 8 * sc, L - 8)) * 2), 0u,
                   Vb + B * kVBlock);
      }
    }
  };
  // Operand reads: K step s (features 16s .. 16s+15) of key col, chunk
  // 2s + half; V block j, keys 16hh .. 16hh+15 of feature 32j + col, chunk
  // 2hh + half. Both are one base register plus a constant.
  const int kbase = (col >> 4) * kKBlock + half * 256 + (col & 15) * 16;
  const int vbase = (col >> 4) * kVBlock + half * 256 + (col & 15) * 16;

  auto active_word = [&](float mv, int kt) -> uint32_t {
    const int ln = lane_now();
    const int k = kt * kWideKeys + ln;
    return (uint32_t)__ballot(ln < 32 && k < L && mv != 0.0f);
  };

  f32x16 O[NB][8];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) O[b][j][r] = 0.0f;
  float m[NB], l[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    m[b] = kNoMax;
    l[b] = 0.0f;
  }
  const float c1 = a.c1;
  bool tainted = false;  // wave-uniform

  float mnext = 0.0f;
  if (kt_begin < kt_end) {
    stage(kt_begin, 0);
    mnext = maskr[min(kt_begin * kWideKeys + (lane & 31), L - 1)];
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  uint32_t wact = kt_begin < kt_end ? active_word(mnext, kt_begin) : 0u;
  // Per block: the last tile with a key at or before one of its queries,
  // and whether some / all of its queries are live.
  int kt_blk_end[NB];
  bool blk_live[NB], blk_full[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const int qb0 = q0w + 32 * b;
    kt_blk_end[b] = min(kt_end, min(last, qb0 + 31) / kWideKeys + 1);
    blk_live[b] = qb0 < L && qb0 + 31 >= start;
    blk_full[b] = qb0 >= start && qb0 + 32 <= L;
  }

  int cur = 0;
  for (int kt = kt_begin; kt < kt_end; ++kt) {
    const bool more = kt + 1 < kt_end;
    const int k0 = kt * kWideKeys;
    // Both blocks run whenever one has work: a block past its diagonal or
    // without a live query has an all-zero keep word (probabilities 0).
    bool on = false;
#pragma unroll
    for (int b = 0; b < NB; ++b) on = on || (blk_live[b] && kt < kt_blk_end[b]);
    const bool compute = !tainted && on;
    const unsigned char *Kb = lds + cur * kStage;
    const unsigned char *Vb = Kb + kKBuf;
    f32x16 st[NB];
    if (compute) {
#pragma unroll
      for (int b = 0; b < NB; ++b) st[b] = f32x16{};
#pragma unroll
      for (int s = 0; s < 16; ++s) {
        const bf16x8 ka = *reinterpret_cast<const bf16x8 *>(Kb + kbase + s * 512);
#pragma unroll
        for (int b = 0; b < NB; ++b) st[b] = mfma_32x32x16_bf16(ka, qb[b][s], st[b]);
      }
      // Schedule: kReadAhead operand reads in flight ahead of the MFMA chain
      // (left alone, the scheduler issues two at a time and each MFMA waits
      // on the LDS latency of its operand).
      pipeline_reads<16 * NB>();
    }
    // The next tile's loads are issued behind the S^T MFMAs, which the
    // matrix cores work through meanwhile: issuing the eight loads stalls
    // while the CU's load path is busy with the other wavefronts' tiles, and
    // at the top of the step that stall held up the MFMAs.
    if (more) {
      stage(kt + 1, cur ^ 1);
      mnext = maskr[min((kt + 1) * kWideKeys + (lane_now() & 31), L - 1)];
    }
    if (compute) {
      // Lane (col, half) holds S^T rows 8*(r/4) + 4*half + (r%4): keys of
      // its query q0w + 32b + col.
      bf16x8 pb[NB][2];
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        float e[16];
        float rs = 0.0f;
        const uint32_t keep = q_live[b] ? (wact & range_bits(0, qv[b] - k0)) : 0u;
        const uint32_t kh = keep >> (4 * half);  // bit 8g + r: key 8g + 4*half + r
        const bool full =
            blk_full[b] && wact == 0xffffffffu && k0 + kWideKeys - 1 <= q0w + 32 * b;
        // Score r is kept: the whole tile is (full), or its keep bit. The
        // scores themselves are never rewritten (no second copy of them).
        auto bit = [](uint32_t w, int r) { return ((w >> (8 * (r >> 2) + (r & 3))) & 1u) != 0u; };
        if (full) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            e[r] = fast_exp2(__builtin_fmaf(st[b][r], c1, -m[b]));
            rs += e[r];
          }
        } else {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            e[r] = bit(kh, r) ? fast_exp2(__builtin_fmaf(st[b][r], c1, -m[b])) : 0.0f;
            rs += e[r];
          }
        }
        if (__ballot(q_live[b] && !(rs <= kLazyLimit16)) != 0) {
          // Rare: some term came out large or non-finite; take the max of
          // the kept scores and move the reference. The keep bits are formed
          // again here (from an opaque copy of the word), so that the common
          // path never computes them for a full tile.
          uint32_t kr;
          asm volatile("v_mov_b32 %0, %1" : "=v"(kr) : "v"(full ? 0xffffffffu : kh));
          auto kept = [&](int r) { return bit(kr, r); };
          float mx = -INFINITY;
#pragma unroll
          for (int r = 0; r < 16; ++r) mx = fmaxf(mx, kept(r) ? st[b][r] : -INFINITY);
          const float mxs = pair_max(mx) * c1;
          const float mn = mxs > m[b] + kRescaleSlack ? mxs : m[b];
          rs = 0.0f;
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const float x = st[b][r];
            e[r] = (!kept(r) || (__builtin_isinf(x) && x < 0.0f))
                       ? 0.0f
                       : fast_exp2(__builtin_fmaf(x, c1, -mn));
            rs += e[r];
          }
          if (__ballot(q_live[b] && !__builtin_isfinite(rs)) != 0) {
            tainted = true;
          } else if (__ballot(mn != m[b]) != 0) {
            const float alpha = fast_exp2(m[b] - mn);  // exactly 1 where m stays
            if (__ballot(l[b] != 0.0f) != 0) {  // nothing accumulated yet: O is 0
#pragma unroll
              for (int j = 0; j < 8; ++j) O[b][j] *= alpha;
            }
            l[b] *= alpha;
            m[b] = mn;
          }
        }
        l[b] += rs;
        // P^T B operands: keys 16hh + 8*half + e for query col. Lanes hold
        // keys 8g + 4*half + (0..3) in group g; one v_permlane32_swap per
        // register trades the missing four with lane ^ 32.
        uint32_t g[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) g[i] = pack_bf16x2(e[2 * i], e[2 * i + 1]);
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
          pb[b][hh] = __builtin_bit_cast(
              bf16x8, (__attribute__((ext_vector_type(4))) uint32_t){w[0], w[1], w[2], w[3]});
        }
      }
      if (!tainted) {
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            const bf16x8 va =
                *reinterpret_cast<const bf16x8 *>(Vb + vbase + j * 2 * kVBlock + hh * 512);
#pragma unroll
            for (int b = 0; b < NB; ++b) O[b][j] = mfma_32x32x16_bf16(va, pb[b][hh], O[b][j]);
          }
        pipeline_reads<16 * NB>();
      }
    }
    __builtin_amdgcn_s_waitcnt(0);  // this wave's part of tile kt + 1 is in LDS
    __syncthreads();
    if (more) wact = active_word(mnext, kt + 1);
    cur ^= 1;
  }

  // -------- o / sum (0 when nothing was kept), sigmoid gate, store
  // (lib.rs:731-758). A non-finite output is left to the exact pass.
  bool bad = tainted;
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) bad |= q_live[b] && !__builtin_isfinite(O[b][j][r]);
  if (__ballot(bad) != 0 && lane == 0) s_flag = 1;
  __syncthreads();
  const bool flagged = s_flag != 0;
  // one flag per (row, head, query tile): waves 0 .. hw-1 hold the heads
  if (lane == 0 && wave < hw) flags[((size_t)row * a.heads + head) * nqt + qt] = flagged ? 1 : 0;
  if (flagged) return;
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const int q = qv[b];
    if (q >= L) continue;
    const float lt = pair_sum(l[b]);
    const float inv = lt > 0.0f ? fast_rcp(lt) : 0.0f;
    const bool dropped = a.trim && q < start;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float gv[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int f = 32 * j + 8 * (r >> 2) + 4 * half + (r & 3);
        gv[r] = bf16_to_f32(Gh[(size_t)f * L + q]);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int f = 32 * j + 8 * (r >> 2) + 4 * half + (r & 3);
        Oh[(size_t)f * L + q] = dropped ? 0.0f : O[b][j][r] * inv * fast_sigmoid(gv[r]);
      }
    }
  }
}

hipError_t launch_jeff_bf16_wide(const JeffArgs &a, int rows, const uint16_t *kp, int *flags,
                                 hipStream_t stream) {
  const int hw = wide_heads_per_group(a);
  const int qt = jeff_bf16_wide_query_tile(a);
  const int units = rows * a.kv_heads * (a.heads / a.kv_heads / hw);
  const unsigned grid = (unsigned)(units * ((a.L + qt - 1) / qt));
  hipLaunchKernelGGL(jeff_bf16_wide_kernel, dim3(grid), dim3(256), 0, stream, a, kp, flags, rows,
                     hw);
  return hipGetLastError();
}

}  // namespace tfd
