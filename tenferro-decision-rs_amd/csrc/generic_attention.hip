// Head dims past the tiled kernels (Laya hd > 128, Jeff hd > 256): one
// wavefront per (batch or row, head, query) in the reference's scalar order,
// so any head dim runs with the reference's results. These shapes do not
// occur in the reference's models (ModernBERT hd 64, Qwen3.5 hd 256); the
// path exists so that the drop-in computes every shape the reference does.
//
// Laya follows the scalar path of cpu-kernels
// laya_attention_block_with_workspace (crates/cpu-kernels/src/lib.rs:
// 1108-1153, RoPE 991-1010): masked keys -inf, max, exp of finite scores,
// o = sum over keys in order of v * (e / sum), skipping p == 0 (a query
// with no kept key divides 0 by 0 and comes out NaN, as there).
// Jeff follows jeff_full_attention_into (lib.rs:653-761): RMSNorm and
// partial RoPE of q (here) and k (jeff_generic_k_prep_kernel, once per key),
// causal and mask != 0, o = 0 unless the sum is positive, times sigmoid(gate).
// Products and sums are unfused and in the reference's order along the head
// dim and the keys; only the max and the sum over keys are reduced across
// the wavefront (a different order, the same values to rounding).
#include "jeff_common.hpp"
#include "tfd_device.hpp"
#include "tfd_internal.hpp"

namespace tfd {

namespace {

__device__ __forceinline__ float wave_maxf(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

__device__ __forceinline__ float wave_sumf(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

template <typename T>
__device__ __forceinline__ float ld(const T *p, size_t i) {
  if constexpr (sizeof(T) == 2)
    return __uint_as_float((uint32_t)reinterpret_cast<const uint16_t *>(p)[i] << 16);
  else
    return p[i];
}

}  // namespace

// ------------------------------------------------------------------ Laya

// grid (L, heads, B), one wavefront; dynamic LDS: the rotated query row
// (hd floats) and the scores of every key (L floats).
__global__ __launch_bounds__(64) void laya_generic_kernel(const LayaArgs a, const uint8_t *keep,
                                                          int mode) {
#pragma clang fp contract(off)
  extern __shared__ float dyn[];
  const int lane = threadIdx.x;
  const int q = blockIdx.x, head = blockIdx.y, b = blockIdx.z;
  const int L = a.L, d = a.d, hd = a.hd, half = a.half;
  float *qr = dyn, *pr = dyn + hd;
  const float *Qrow = a.qkv + (size_t)3 * d * (q + (size_t)L * b) + (size_t)head * hd;
  for (int i = lane; i < hd; i += 64) qr[i] = Qrow[i];
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (a.cos_t != nullptr) {  // lib.rs:991-1010 (pairs i, i + hd/2)
    for (int i = lane; i < half; i += 64) {
      const float c = a.cos_t[(size_t)q * half + i], s = a.sin_t[(size_t)q * half + i];
      const float x = qr[i], y = qr[i + half];
      qr[i] = x * c - y * s;
      qr[i + half] = x * s + y * c;
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const float scale = 1.0f / sqrtf((float)hd);
  const bool vq = mode == kMaskStruct ? a.valid[(size_t)b * L + q] != 0 : true;
  float mx = -INFINITY;
  for (int k = lane; k < L; k += 64) {
    bool kept;
    if (mode == kMaskStruct) {
      const bool vk = a.valid[(size_t)b * L + k] != 0;
      const int dist = q > k ? q - k : k - q;
      kept = vk && (a.window < 0 || dist <= a.window || !vq);
    } else {
      kept = keep[q + (size_t)L * (k + (size_t)L * b)] != 0;
    }
    float s = -INFINITY;
    if (kept) {
      const float *K = a.qkv + (size_t)3 * d * (k + (size_t)L * b) + d + (size_t)head * hd;
      float acc = 0.0f;
      if (a.cos_t != nullptr) {
        const float *ct = a.cos_t + (size_t)k * half, *st = a.sin_t + (size_t)k * half;
        for (int i = 0; i < half; ++i) acc += qr[i] * (K[i] * ct[i] - K[i + half] * st[i]);
        for (int i = 0; i < half; ++i) acc += qr[i + half] * (K[i] * st[i] + K[i + half] * ct[i]);
        for (int i = 2 * half; i < hd; ++i) acc += qr[i] * K[i];
      } else {
        for (int i = 0; i < hd; ++i) acc += qr[i] * K[i];
      }
      s = acc * scale;
      if (s > mx) mx = s;
    }
    pr[k] = s;
  }
  mx = wave_maxf(mx);
  float sum = 0.0f;
  for (int k = lane; k < L; k += 64) {
    const float s = pr[k];
    const float e = __builtin_isfinite(s) ? expf(s - mx) : 0.0f;
    pr[k] = e;
    sum += e;
  }
  sum = wave_sumf(sum);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float *O = a.out + (size_t)d * (q + (size_t)L * b) + (size_t)head * hd;
  for (int i = lane; i < hd; i += 64) {
    float o = 0.0f;
    for (int k = 0; k < L; ++k) {
      const float p = pr[k] / sum;
      if (p == 0.0f) continue;
      o += a.qkv[(size_t)3 * d * (k + (size_t)L * b) + 2 * d + (size_t)head * hd + i] * p;
    }
    O[i] = o;
  }
}

hipError_t launch_laya_generic(const LayaArgs &a, const uint8_t *keep, int heads, int batch,
                               int mode, hipStream_t stream) {
  const size_t lds = sizeof(float) * ((size_t)a.hd + (size_t)a.L);
  hipLaunchKernelGGL(laya_generic_kernel, dim3(a.L, heads, batch), dim3(64), lds, stream, a, keep,
                     mode);
  return hipGetLastError();
}

// ------------------------------------------------------------------ Jeff

// First active key of row `row` (0 when none), by one wavefront.
__device__ __forceinline__ int generic_row_start(const JeffArgs &a, int row) {
  if (!a.trim) return 0;
  const float *m = a.mask + (size_t)row * a.L;
  int lo = 0x7fffffff;
  for (int k = threadIdx.x; k < a.L; k += 64)
    if (m[k] != 0.0f) lo = min(lo, k);
  lo = wave_min(lo);
  return lo == 0x7fffffff ? 0 : lo;
}

// RMSNorm (lib.rs:676-691) and partial RoPE (692-709) of one key row into
// kn[row][kv head][key][hd]. grid (L, kv_heads, rows), one wavefront;
// dynamic LDS: the row (hd floats).
template <typename T>
__global__ __launch_bounds__(64) void jeff_generic_k_prep_kernel(const JeffArgs a, float *kn) {
#pragma clang fp contract(off)
  extern __shared__ float dyn[];
  const int lane = threadIdx.x;
  const int t = blockIdx.x, kvh = blockIdx.y, row = blockIdx.z;
  const int L = a.L, hd = a.hd, rh = a.rot_half;
  const int start = generic_row_start(a, row);
  const T *K = static_cast<const T *>(a.k) + row * a.kv_row + (size_t)kvh * a.kv_head;
  float *kr = dyn;
  float ss = 0.0f;
  for (int i = lane; i < hd; i += 64) {
    const float x = ld(K, t + (size_t)L * i);
    kr[i] = x;
    ss += x * x;
  }
  ss = wave_sumf(ss);
  const float scale = rms_scale(ss, hd, a.eps);
  for (int i = lane; i < hd; i += 64) kr[i] = rms_apply(kr[i], scale, a.k_norm[i]);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (a.cos_t != nullptr && rh > 0 && t >= start) {
    const size_t pos = (size_t)(t - start) * rh;
    for (int i = lane; i < rh; i += 64) {
      const float c = a.cos_t[pos + i], s = a.sin_t[pos + i];
      const float x = kr[i], y = kr[i + rh];
      kr[i] = rope_lo(x, y, c, s);
      kr[i + rh] = rope_hi(x, y, c, s);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  float *dst = kn + (((size_t)row * a.kv_heads + kvh) * L + t) * hd;
  for (int i = lane; i < hd; i += 64) dst[i] = kr[i];
}

// grid (L, heads, rows), one wavefront; dynamic LDS: the query row (hd) and
// the scores of the keys at or before it (L).
template <typename T>
__global__ __launch_bounds__(64) void jeff_generic_kernel(const JeffArgs a, const float *kn) {
#pragma clang fp contract(off)
  extern __shared__ float dyn[];
  const int lane = threadIdx.x;
  const int q = blockIdx.x, head = blockIdx.y, row = blockIdx.z;
  const int L = a.L, hd = a.hd, rh = a.rot_half;
  const int kvh = min(head / a.groups, a.kv_heads - 1);
  const int start = generic_row_start(a, row);
  float *qr = dyn, *pr = dyn + hd;
  const T *Q = static_cast<const T *>(a.q) + row * a.q_row + (size_t)head * hd * L;
  const T *Gt = static_cast<const T *>(a.gate) + row * a.q_row + (size_t)head * hd * L;
  const T *V = static_cast<const T *>(a.v) + row * a.kv_row + (size_t)kvh * a.kv_head;
  float *OUT = a.out + row * a.q_row + (size_t)head * hd * L;
  if (q < start) {  // dropped by the trim (engine.rs:317-329): 0
    for (int i = lane; i < hd; i += 64) OUT[q + (size_t)L * i] = 0.0f;
    return;
  }
  float ss = 0.0f;
  for (int i = lane; i < hd; i += 64) {
    const float x = ld(Q, q + (size_t)L * i);
    qr[i] = x;
    ss += x * x;
  }
  ss = wave_sumf(ss);
  const float scale = rms_scale(ss, hd, a.eps);
  for (int i = lane; i < hd; i += 64) qr[i] = rms_apply(qr[i], scale, a.q_norm[i]);
  if (a.cos_t != nullptr && rh > 0) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const size_t pos = (size_t)(q - start) * rh;
    for (int i = lane; i < rh; i += 64) {
      const float c = a.cos_t[pos + i], s = a.sin_t[pos + i];
      const float x = qr[i], y = qr[i + rh];
      qr[i] = rope_lo(x, y, c, s);
      qr[i + rh] = rope_hi(x, y, c, s);
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const float *maskr = a.mask + (size_t)row * L;
  const float *Kn = kn + ((size_t)row * a.kv_heads + kvh) * (size_t)L * hd;
  const float attn_scale = 1.0f / sqrtf((float)hd);
  float mx = -INFINITY;
  for (int k = lane; k <= q; k += 64) {  // lib.rs:716: key > query or mask == 0 drops it
    float s = -INFINITY;
    if (k >= start && maskr[k] != 0.0f) {
      const float *kr = Kn + (size_t)k * hd;
      float acc = 0.0f;
      for (int i = 0; i < hd; ++i) acc += qr[i] * kr[i];
      s = acc * attn_scale;
      if (s > mx) mx = s;
    }
    pr[k] = s;
  }
  mx = wave_maxf(mx);
  float sum = 0.0f;
  for (int k = lane; k <= q; k += 64) {
    const float s = pr[k];
    const float e = __builtin_isfinite(s) ? expf(s - mx) : 0.0f;
    pr[k] = e;
    sum += e;
  }
  sum = wave_sumf(sum);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  for (int i = lane; i < hd; i += 64) {
    float o = 0.0f;
    if (sum > 0.0f) {  // lib.rs:743-754
      for (int k = 0; k <= q; ++k) {
        const float p = pr[k] / sum;
        if (p == 0.0f) continue;
        o += ld(V, k + (size_t)L * i) * p;
      }
    }
    const float g = ld(Gt, q + (size_t)L * i);
    OUT[q + (size_t)L * i] = o * (1.0f / (1.0f + expf(-g)));
  }
}

hipError_t launch_jeff_generic(const JeffArgs &a, int rows, bool bf16, float *kn,
                               hipStream_t stream, const KernelEvents &ev) {
  const dim3 pgrid(a.L, a.kv_heads, rows), grid(a.L, a.heads, rows);
  const size_t lds = sizeof(float) * ((size_t)a.hd + (size_t)a.L);
  const size_t klds = sizeof(float) * (size_t)a.hd;
  if (bf16) {
    hipExtLaunchKernelGGL((jeff_generic_k_prep_kernel<uint16_t>), pgrid, dim3(64), klds, stream,
                          ev.start, nullptr, 0, a, kn);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipExtLaunchKernelGGL((jeff_generic_kernel<uint16_t>), grid, dim3(64), lds, stream, nullptr,
                          ev.stop, 0, a, kn);
  } else {
    hipExtLaunchKernelGGL((jeff_generic_k_prep_kernel<float>), pgrid, dim3(64), klds, stream,
                          ev.start, nullptr, 0, a, kn);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipExtLaunchKernelGGL((jeff_generic_kernel<float>), grid, dim3(64), lds, stream, nullptr,
                          ev.stop, 0, a, kn);
  }
  return hipGetLastError();
}

}  // namespace tfd
