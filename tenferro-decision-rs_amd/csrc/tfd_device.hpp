// Device helpers shared by the gfx950 attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tfd {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));
typedef unsigned short u16x4 __attribute__((ext_vector_type(4)));

// D(32x32) += A(32x2) * B(2x32) on the f32 matrix cores.
// Lane l supplies A[l%32][l/32] and B[l/32][l%32]; D row for accumulator r is
// acc_row(r, l/32), D column is l%32.
__device__ __forceinline__ f32x16 mfma_32x32x2(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// D(16x16) += A(16x4) * B(4x16). Lane l supplies A[l%16][l/16] and
// B[l/16][l%16]; accumulator r holds D[4*(l/16) + r][l%16].
__device__ __forceinline__ f32x4 mfma_16x16x4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// D(16x16) += A(16x32) * B(32x16) in bf16 with f32 accumulation. Lane l
// supplies A[l%16][8*(l/16) + e] and B[8*(l/16) + e][l%16], e = 0..7;
// accumulator r holds D[4*(l/16) + r][l%16].
__device__ __forceinline__ f32x4 mfma_16x16x32_bf16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// The same product with fp16 operands (same lane layout).
__device__ __forceinline__ f32x4 mfma_16x16x32_f16(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float bf16_to_f32(unsigned short h) {
  return __uint_as_float((uint32_t)h << 16);
}

// Round to nearest even.
__device__ __forceinline__ unsigned short f32_to_bf16(float x) {
  const __bf16 h = (__bf16)x;
  return *reinterpret_cast<const unsigned short *>(&h);
}

__device__ __forceinline__ bool bf16_finite(unsigned short h) { return ((h >> 7) & 0xff) != 0xff; }

__device__ __forceinline__ int acc_row(int r, int half) {
  return 8 * (r >> 2) + 4 * half + (r & 3);
}

// Bits j of a 32-key word with lo <= j <= hi (clamped to the word).
__device__ __forceinline__ uint32_t range_bits(int lo, int hi) {
  lo = lo < 0 ? 0 : lo;
  hi = hi > 31 ? 31 : hi;
  if (lo > hi) return 0u;
  uint32_t upper = hi == 31 ? 0xffffffffu : ((1u << (hi + 1)) - 1u);
  return upper & ~((1u << lo) - 1u);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// 1 / x to 1 ulp (hardware reciprocal).
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

// 1 / (1 + exp(-g)) with the hardware exp2 and reciprocal (a few ulp from
// the libm evaluation the reference uses).
__device__ __forceinline__ float fast_sigmoid(float g) {
  return fast_rcp(1.0f + fast_exp2(-g * 1.4426950408889634f));
}

// max / sum of x over the lane pair (l, l ^ 32), identical in both lanes, with
// one v_permlane32_swap (lanes 32..63 of the first operand trade places with
// lanes 0..31 of the second) instead of an LDS permute.
__device__ __forceinline__ float pair_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// The same over the lane pair (l, l ^ 16), with one v_permlane16_swap (odd
// 16-lane rows of the first operand trade places with even rows of the
// second).
__device__ __forceinline__ float pair16_max(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair16_sum(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Online softmax with a lazily moved reference: exponents are taken against
// a reference m (log2 units) that only moves when a tile's max exceeds it by
// more than kRescaleSlack, so most tiles skip rescaling the accumulators.
// Probabilities stay below 2^kRescaleSlack; O / l is unchanged.
constexpr float kRescaleSlack = 8.0f;
// Initial reference: finite, so exp2(fma(-inf, c1, -m)) is exp2(-inf) = 0.
constexpr float kNoMax = -3.402823466e38f;
// A lane whose 8 terms of a tile, taken against the current reference, sum
// to at most this (2^11 = 8 * 2^kRescaleSlack) needs no new reference.
constexpr float kLazyLimit = 2048.0f;

// Raw buffer access through an SGPR resource: the per-lane byte offset can
// stay fixed for a whole walk, the tile base is a scalar offset, and any byte
// at or past `bytes` reads as 0 (stores there are dropped) by the hardware
// range check.
constexpr int kBufferWord3 = 0x00020000;  // gfx9 raw buffer (no format, no swizzle)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes,
                                           kBufferWord3);
}
// A buffer resource as four scalar words (raw buffer, no swizzle).
typedef unsigned u32x4r __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x4r rsrc_words(const void *base, uint32_t bytes) {
  const uint64_t ad = reinterpret_cast<uint64_t>(base);
  return u32x4r{(uint32_t)ad, (uint32_t)(ad >> 32) & 0xffffu, bytes, (uint32_t)kBufferWord3};
}

// 16 bytes at byte voff + soff of the buffer r into LDS at lds_base + 16*lane
// (M0 = lds_base; lds_base and soff the same for the whole wavefront): one
// 32-bit offset register per lane. Written out rather than through the
// builtin, which the compiler treats as a write to any LDS address: it would
// make the next LDS operand read wait for every such load issued before it.
// Callers order these loads themselves: a wavefront waits for its own loads
// (s_waitcnt vmcnt) before it, or a barrier after it, reads the data, and
// issues them only after its reads of the old contents have completed. M0 is a
// reserved register that the compiler sets right before each of its own
// uses and never keeps a value in across other code (the kernels that use
// this load have no such use; tests/test_kernel_asm.py checks the compiled
// kernels for it), so it needs no clobber.
__device__ __forceinline__ void load_lds16(u32x4r r, uint32_t voff, uint32_t soff,
                                           unsigned char *lds_base) {
  const uint32_t m = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void *)lds_base;
  asm volatile("s_mov_b32 m0, %3\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voff),
               "s"(r), "s"(soff), "s"(m));
}

__device__ __forceinline__ f32x4 buffer_load4(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}
__device__ __forceinline__ float buffer_load1(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}
__device__ __forceinline__ void buffer_store1(float v, __amdgpu_buffer_rsrc_t r, int voff, int soff) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, voff, soff, 0);
}
__device__ __forceinline__ void buffer_store4(f32x4 v, __amdgpu_buffer_rsrc_t r, int voff,
                                              int soff) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned int, v), r, voff, soff, 0);
}
// Non-temporal stores (cache policy nt) for outputs nothing in the kernel
// reads again: they do not leave dirty L2 lines for the end-of-kernel
// write-back.
constexpr int kCacheNT = 2;
__device__ __forceinline__ void buffer_store1_nt(float v, __amdgpu_buffer_rsrc_t r, int voff,
                                                 int soff) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, voff, soff, kCacheNT);
}
__device__ __forceinline__ void buffer_store4_nt(f32x4 v, __amdgpu_buffer_rsrc_t r, int voff,
                                                 int soff) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned int, v), r, voff, soff, kCacheNT);
}

__device__ __forceinline__ float wave_max_f(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

// Exponent e of a power-of-two factor 2^-e for the fp16 Q.K^T operands of
// the bf16 Jeff kernels: max_i |1 + w_i| * 2^-e lies in [0.5, 1) (e clamped
// to [-64, 64]; e = 0 when the max is 0 or not finite). After the centered
// RMSNorm |x_i * scale| <= sqrt(hd), and RoPE keeps each pair's norm, so a
// normalized, rotated q or k times 2^-e stays below sqrt(hd) <= 16 for
// hd <= 256: inside fp16's range, with a relative rounding of 2^-11 instead
// of bf16's 2^-8. Scaling by a power of two is exact; the scores come back
// through c1 * 2^(e_q + e_k). Every lane of the wavefront takes part and
// gets the same e.
__device__ __forceinline__ int norm_weight_exp(const float *__restrict__ w, int hd, int lane) {
  float mx = 0.0f;
  for (int i = lane; i < hd; i += 64) mx = fmaxf(mx, fabsf(1.0f + w[i]));
  mx = wave_max_f(mx);
  if (!(mx > 0.0f) || !__builtin_isfinite(mx)) return 0;
  int e;
  (void)frexpf(mx, &e);
  return __builtin_amdgcn_readfirstlane(e < -64 ? -64 : (e > 64 ? 64 : e));
}

__device__ __forceinline__ unsigned short f32_to_f16_bits(float x) {
  const _Float16 h = (_Float16)x;
  return __builtin_bit_cast(unsigned short, h);
}

__device__ __forceinline__ int wave_min(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o));
  return v;
}

__device__ __forceinline__ int wave_max(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o));
  return v;
}

// Online-softmax step on one 32-key tile held as the S^T accumulators of a
// lane (its query = lane%32, its 16 keys = acc_row(r, lane/32)). Follows the
// reference's masked softmax (cpu-kernels lib.rs:1111-1136): masked or
// non-finite scores contribute 0 and never raise the running max, a +inf
// score makes the row's sum 0. Scores are kept in the log2 domain
// (x = acc * c1 with c1 = scale*log2(e)), so exp(score - max) = exp2(x - m).
// On return s holds the unnormalized probabilities, m/l are updated and
// alpha is the factor the output accumulators must be scaled by.
__device__ __forceinline__ float softmax_tile(f32x16 &s, uint32_t keep, int half, float c1,
                                              float &m, float &l) {
  float mx = -INFINITY;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    bool kept = (keep >> acc_row(r, half)) & 1u;
    float x = kept ? s[r] * c1 : -INFINITY;
    s[r] = x;
    mx = fmaxf(mx, x);
  }
  mx = pair_max(mx);
  const float mn = fmaxf(m, mx);
  const float alpha = (m == mn) ? 1.0f : fast_exp2(m - mn);
  float rs = 0.0f;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    float x = s[r];
    float e = __builtin_isfinite(x) ? fast_exp2(x - mn) : 0.0f;
    s[r] = e;
    rs += e;
  }
  l = l * alpha + rs;
  m = mn;
  return alpha;
}

// Probability of key kk (0..31) of the tile for this lane's query, fetched
// from whichever lane half holds it.
__device__ __forceinline__ float tile_prob(const f32x16 &s, int kk, int col) {
  const int r = ((kk >> 3) << 2) | (kk & 3);
  const int src_half = (kk >> 2) & 1;
  float sel = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) sel = (i == r) ? s[i] : sel;
  return __shfl(sel, col + 32 * src_half);
}

// softmax_tile for the 16x16 layout: a 32-key tile is two S^T blocks,
// s0 (keys 0..15) and s1 (keys 16..31); lane group g = lane/16 holds keys
// 16*b + 4*g + r of its query lane%16.
// With ROUND_BF16 the probabilities are rounded to bf16 (nearest even) before
// they are summed, so that l is the sum of exactly the values a bf16 P.V
// product consumes and O / l stays a convex combination of V.
template <bool ROUND_BF16 = false>
__device__ __forceinline__ float softmax_tile16(f32x4 &s0, f32x4 &s1, uint32_t keep, int grp,
                                                float c1, float &m, float &l) {
  float mx = -INFINITY;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int k = 4 * grp + r;
    const float x0 = ((keep >> k) & 1u) ? s0[r] * c1 : -INFINITY;
    const float x1 = ((keep >> (16 + k)) & 1u) ? s1[r] * c1 : -INFINITY;
    s0[r] = x0;
    s1[r] = x1;
    mx = fmaxf(mx, fmaxf(x0, x1));
  }
  mx = fmaxf(mx, __shfl_xor(mx, 16));
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  const float mn = fmaxf(m, mx);
  const float alpha = (m == mn) ? 1.0f : fast_exp2(m - mn);
  float rs = 0.0f;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float e0 = __builtin_isfinite(s0[r]) ? fast_exp2(s0[r] - mn) : 0.0f;
    float e1 = __builtin_isfinite(s1[r]) ? fast_exp2(s1[r] - mn) : 0.0f;
    if (ROUND_BF16) {
      e0 = bf16_to_f32(f32_to_bf16(e0));
      e1 = bf16_to_f32(f32_to_bf16(e1));
    }
    s0[r] = e0;
    s1[r] = e1;
    rs += e0 + e1;
  }
  l = l * alpha + rs;
  m = mn;
  return alpha;
}

// Probability of key kx (0..31) for this lane's query in the 16x16 layout.
__device__ __forceinline__ float tile_prob16(const f32x4 &s0, const f32x4 &s1, int kx, int col) {
  const int kl = kx & 15, r = kl & 3, g = kl >> 2;
  float sel = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) sel = (i == r) ? ((kx >> 4) ? s1[i] : s0[i]) : sel;
  return __shfl(sel, col + 16 * g);
}

}  // namespace tfd
