// Per-element arithmetic of the Jeff block shared by its kernels, in the
// reference's operation order (cpu-kernels lib.rs:676-709), evaluated
// without FP contraction as Rust does.
#pragma once

#include <hip/hip_runtime.h>

namespace tfd {

// x * (scale * (1 + w)) with the reference's rounding (no contraction).
__device__ __forceinline__ float rms_apply(float x, float scale, float w) {
#pragma clang fp contract(off)
  return x * (scale * (1.0f + w));
}

__device__ __forceinline__ float rope_lo(float a, float b, float c, float s) {
#pragma clang fp contract(off)
  return a * c - b * s;
}

__device__ __forceinline__ float rope_hi(float a, float b, float c, float s) {
#pragma clang fp contract(off)
  return a * s + b * c;
}

// 1 / sqrt(mean + eps) with mean = sumsq / hd, in the reference's order.
__device__ __forceinline__ float rms_scale(float sumsq, int hd, float eps) {
#pragma clang fp contract(off)
  const float mean = sumsq / (float)hd;
  return 1.0f / sqrtf(mean + eps);
}

}  // namespace tfd
