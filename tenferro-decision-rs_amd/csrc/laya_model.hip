// Elementwise and per-column kernels of the Laya decision-model forward
// (laya-infer model.rs:387-458, 635-645, 773-837, 867-977) around the fused
// attention op and the rocBLAS projections. Activations are feature-first
// column-major (d, columns): one column = one token (or marker) and its d
// contiguous features, so a wavefront owns a column and its loads coalesce.
// These kernels move a few bytes per flop and are bound by HBM / launch
// latency; none of them is on the attention hot path.
#include <math.h>

#include "tfd_device.hpp"
#include "tfd_internal.hpp"

namespace tfd {
namespace {

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// x * (1 + erf(x / sqrt 2)) / 2 (model.rs:312-314) with the device library's
// erff (correctly rounded to within 2 ulp).
__device__ __forceinline__ float gelu_erf(float x) {
  return x * (1.0f + erff(x / 1.41421356237309515f)) / 2.0f;
}

__device__ __forceinline__ float activate(float x, int act) {
  if (act == kActRelu) return fmaxf(x, 0.0f);
  if (act == kActGelu) return gelu_erf(x);
  return x;
}

// One wavefront per output column c: source column map ? map[c] : c of x
// (leading dimension ldx), LayerNorm over its d features (layer_norm_host,
// model.rs:387-422: mean, then the mean of squared deviations, then
// (x - mean) * (1 / sqrt(var + eps)) * w (+ b)), then plus column
// add_col[c / per] of `add` when given (the type embedding, model.rs:916-931).
// NR > 0: the column is held in registers (d <= 64 * NR, one read);
// NR == 0: any d, three passes over the column.
template <int NR>
__global__ __launch_bounds__(256) void norm_columns_kernel(NormArgs a) {
  const int lane = threadIdx.x & 63;
  const long c = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (c >= a.cols) return;
  const long src = a.map ? (long)a.map[c] : c;
  const float *x = a.x + src * (long)a.ldx;
  const int d = a.d;
  float r[NR > 0 ? NR : 1];
  float s = 0.0f;
  if constexpr (NR > 0) {
#pragma unroll
    for (int k = 0; k < NR; ++k) {
      const int i = lane + 64 * k;
      r[k] = i < d ? x[i] : 0.0f;
      s += r[k];
    }
  } else {
    for (int i = lane; i < d; i += 64) s += x[i];
  }
  const float mean = wave_sum(s) / (float)d;
  float v = 0.0f;
  if constexpr (NR > 0) {
#pragma unroll
    for (int k = 0; k < NR; ++k) {
      const float t = r[k] - mean;
      v += lane + 64 * k < d ? t * t : 0.0f;
    }
  } else {
    for (int i = lane; i < d; i += 64) {
      const float t = x[i] - mean;
      v += t * t;
    }
  }
  const float var = wave_sum(v) / (float)d;
  const float inv = 1.0f / sqrtf(var + a.eps);
  float *y = a.y + c * (long)d;
  const float *t = a.add ? a.add + (long)a.add_col[c / a.per] * d : nullptr;
  auto put = [&](int i, float xi) {
    float value = (xi - mean) * inv;
    value = value * a.w[i];
    if (a.b) value = value + a.b[i];
    if (t) value = value + t[i];
    y[i] = value;
  };
  if constexpr (NR > 0) {
#pragma unroll
    for (int k = 0; k < NR; ++k)
      if (lane + 64 * k < d) put(lane + 64 * k, r[k]);
  } else {
    for (int i = lane; i < d; i += 64) put(i, x[i]);
  }
}

// y[o + m*j] = act(y[o + m*j] + b[o]) (b may be null).
__global__ __launch_bounds__(256) void bias_act_kernel(float *__restrict__ y,
                                                       const float *__restrict__ b, int m,
                                                       size_t total, int act) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (size_t)gridDim.x * blockDim.x) {
    float v = y[i];
    if (b) v = v + b[i % (size_t)m];
    y[i] = activate(v, act);
  }
}

// gelu_gate_host (model.rs:635-645): g[i + I*c] = gelu(u[i + 2I*c]) *
// u[I + i + 2I*c], each u plus its bias when the projection has one.
__global__ __launch_bounds__(256) void geglu_kernel(const float *__restrict__ u,
                                                    const float *__restrict__ b, int inter,
                                                    size_t cols, float *__restrict__ g) {
  const size_t total = (size_t)inter * cols;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (size_t)gridDim.x * blockDim.x) {
    const size_t c = i / inter, f = i - c * inter;
    float x = u[2 * inter * c + f], y = u[2 * inter * c + inter + f];
    if (b) {
      x = x + b[f];
      y = y + b[inter + f];
    }
    g[i] = gelu_erf(x) * y;
  }
}

// dst[:, dst_map ? dst_map[j] : j] = src[:, src_map ? src_map[j] : j] for
// j < n, m floats per column: the packed <-> padded column moves around the
// attention op. One wave per column.
__global__ __launch_bounds__(256) void copy_columns_kernel(const float *__restrict__ src,
                                                           const int *__restrict__ src_map,
                                                           float *__restrict__ dst,
                                                           const int *__restrict__ dst_map, int m,
                                                           long n) {
  const int lane = threadIdx.x & 63;
  const long j = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (j >= n) return;
  const float *s = src + (long)(src_map ? src_map[j] : j) * m;
  float *d = dst + (long)(dst_map ? dst_map[j] : j) * m;
  if ((m & 3) == 0) {
    for (int i = 4 * lane; i < m; i += 256)
      *reinterpret_cast<f32x4 *>(d + i) = *reinterpret_cast<const f32x4 *>(s + i);
  } else {
    for (int i = lane; i < m; i += 64) d[i] = s[i];
  }
}

// pool_host (model.rs:773-837) for batch column blockIdx.x on one
// wavefront, markers spread over the lanes (marker j on lane j % 64), and the
// pooled action-head input [h[:, 0, b]; top1; top1 - top2; entropy;
// used / 255] (model.rs:944-952). Masked markers take the logit -1e4
// (model.rs:779-786); the softmax max, sum and entropy are wave reductions,
// and each lane keeps the two largest probabilities it has seen, merged
// across lanes as (max, second largest with repeats), which is the pair the
// reference's sequential scan (model.rs:805-813) ends with.
__device__ __forceinline__ float wave_sum_f(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

__global__ __launch_bounds__(64) void pool_kernel(PoolArgs a) {
  const int b = blockIdx.x, lane = threadIdx.x;
  const int K = a.k;
  const float *raw = a.raw + (size_t)b * K;
  const uint8_t *mm = a.marker_mask + (size_t)b * K;
  float *lo = a.logits + (size_t)b * K;
  float *pooled = a.pooled + (size_t)b * (a.d + 4);
  const float *h0 = a.h + (size_t)(a.h0_col ? a.h0_col[b] : b * a.L) * a.d;
  for (int i = lane; i < a.d; i += 64) pooled[i] = h0[i];

  auto masked = [&](int j) { return mm[j] ? raw[j] : -1.0e4f; };
  float mx = -INFINITY;
  int used = 0;
  for (int j0 = 0; j0 < K; j0 += 64) {
    const int j = j0 + lane;
    const bool in = j < K;
    const float v = in ? masked(j) : -INFINITY;
    if (in) lo[j] = v;
    mx = fmaxf(mx, v);
    used += __popcll(__ballot(in && mm[j] != 0));
  }
  mx = wave_max_f(mx);
  float sum = 0.0f;
  for (int j = lane; j < K; j += 64) sum += expf(masked(j) - mx);
  sum = wave_sum_f(sum);
  float t1 = -INFINITY, t2 = -INFINITY, ent = 0.0f;
  for (int j = lane; j < K; j += 64) {
    const float p = expf(masked(j) - mx) / sum;
    t2 = fmaxf(t2, fminf(t1, p));
    t1 = fmaxf(t1, p);
    ent -= p * logf(fmaxf(p, 1.0e-9f));
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float u1 = __shfl_xor(t1, o), u2 = __shfl_xor(t2, o);
    t2 = fmaxf(fminf(t1, u1), fmaxf(t2, u2));
    t1 = fmaxf(t1, u1);
  }
  ent = wave_sum_f(ent);
  if (lane == 0) {
    const float n = (float)(used < 2 ? 2 : used);
    pooled[a.d] = t1;
    pooled[a.d + 1] = t1 - t2;
    pooled[a.d + 2] = ent / logf(n);
    pooled[a.d + 3] = n / 255.0f;
  }
}

unsigned grid_for(size_t total) {
  size_t blocks = (total + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  return (unsigned)(blocks ? blocks : 1);
}

}  // namespace

hipError_t launch_norm_columns(const NormArgs &a, hipStream_t stream) {
  if (a.cols <= 0) return hipSuccess;
  const dim3 grid((unsigned)((a.cols + 3) / 4));
  if (a.d <= 256)
    hipLaunchKernelGGL(norm_columns_kernel<4>, grid, dim3(256), 0, stream, a);
  else if (a.d <= 1024)
    hipLaunchKernelGGL(norm_columns_kernel<16>, grid, dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL(norm_columns_kernel<0>, grid, dim3(256), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_bias_act(float *y, const float *b, int m, size_t n, int act,
                           hipStream_t stream) {
  const size_t total = (size_t)m * n;
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL(bias_act_kernel, dim3(grid_for(total)), dim3(256), 0, stream, y, b, m, total,
                     act);
  return hipGetLastError();
}

hipError_t launch_geglu(const float *u, const float *b, int inter, size_t cols, float *g,
                        hipStream_t stream) {
  const size_t total = (size_t)inter * cols;
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL(geglu_kernel, dim3(grid_for(total)), dim3(256), 0, stream, u, b, inter, cols,
                     g);
  return hipGetLastError();
}

hipError_t launch_copy_columns(const float *src, const int *src_map, float *dst,
                               const int *dst_map, int m, long n, hipStream_t stream) {
  if (n <= 0 || m <= 0) return hipSuccess;
  hipLaunchKernelGGL(copy_columns_kernel, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, stream, src,
                     src_map, dst, dst_map, m, n);
  return hipGetLastError();
}

hipError_t launch_pool(const PoolArgs &a, int batch, hipStream_t stream) {
  if (batch <= 0) return hipSuccess;
  hipLaunchKernelGGL(pool_kernel, dim3((unsigned)batch), dim3(64), 0, stream, a);
  return hipGetLastError();
}

}  // namespace tfd
