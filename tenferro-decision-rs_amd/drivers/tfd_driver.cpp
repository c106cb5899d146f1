// tfd_driver -- a C++ host of the C ABI (include/tfd_attention.h), the way a
// non-Python engine binds it: no torch, plain pointers, hipMalloc'd device
// buffers for the device-pointer path.
//
//   tfd_driver abi     ABI version and family ids (no device access)
//   tfd_driver check   closed-form properties of both drop-in ops through host
//                      and device pointers; exit 0 when all hold
//   tfd_driver bench   C2-shaped Laya op (d 768, 12 heads, L 512, B 8, right
//                      padding) on device pointers, HIP events on the context's
//                      stream; one JSON line
//
// The checks need no oracle: with every value row of a head equal, softmax
// weights summing to one give that row back (laya_attention.rs:99-176 through
// lib.rs:843-1156); a query keeping a single key copies that key's value;
// a Jeff query whose only active key at or before it is key 0 gets
// v[0] * sigmoid(gate) (lib.rs:609-763).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "tfd_attention.h"

namespace {

// The reference tests' LCG (laya-infer tests/model.rs:17-31).
struct Lcg {
  uint64_t s;
  explicit Lcg(uint64_t seed) : s(seed) {}
  float uniform() {
    s = s * 6364136223846793005ull + 1442695040888963407ull;
    return (float)((double)(s >> 40) / (double)(1u << 24));
  }
  float sym() { return 2.0f * uniform() - 1.0f; }
};

uint32_t bits(float x) {
  uint32_t b;
  std::memcpy(&b, &x, 4);
  return b;
}

int failures = 0;

// HIP calls of the driver itself (copies, frees, events): a failure is a FAIL.
void hip_ok(hipError_t e) {
  if (e != hipSuccess) {
    std::printf("FAIL HIP: %s\n", hipGetErrorString(e));
    ++failures;
  }
}

void expect(bool ok, const char *what) {
  std::printf("%s %s\n", ok ? "PASS" : "FAIL", what);
  if (!ok) ++failures;
}

bool close(float got, float want, float rel) {
  return std::fabs(got - want) <= rel * std::fmax(1.0f, std::fabs(want));
}

// Runs `call(flags, in_ptrs, out_ptr)` once with host pointers and once with
// device copies of `inputs`; returns both outputs.
template <typename Call>
bool both_paths(const std::vector<std::vector<float>> &inputs, const std::vector<uint8_t> *bytes,
                size_t out_n, Call call, std::vector<float> &host_out,
                std::vector<float> &dev_out) {
  host_out.assign(out_n, 0.0f);
  std::vector<const void *> hp;
  for (const auto &v : inputs) hp.push_back(v.data());
  if (bytes) hp.push_back(bytes->data());
  if (call(TFD_HOST_PTRS, hp, host_out.data()) != TFD_OK) return false;
  std::vector<void *> dbuf;
  for (const auto &v : inputs) {
    void *p = nullptr;
    if (hipMalloc(&p, v.size() * sizeof(float)) != hipSuccess) return false;
    hip_ok(hipMemcpy(p, v.data(), v.size() * sizeof(float), hipMemcpyHostToDevice));
    dbuf.push_back(p);
  }
  if (bytes) {
    void *p = nullptr;
    if (hipMalloc(&p, bytes->size()) != hipSuccess) return false;
    hip_ok(hipMemcpy(p, bytes->data(), bytes->size(), hipMemcpyHostToDevice));
    dbuf.push_back(p);
  }
  float *dout = nullptr;
  if (hipMalloc(&dout, out_n * sizeof(float)) != hipSuccess) return false;
  std::vector<const void *> dp(dbuf.begin(), dbuf.end());
  const int rc = call(TFD_DEVICE_PTRS, dp, dout);
  dev_out.assign(out_n, 0.0f);
  hip_ok(hipMemcpy(dev_out.data(), dout, out_n * sizeof(float), hipMemcpyDeviceToHost));
  for (void *p : dbuf) hip_ok(hipFree(p));
  hip_ok(hipFree(dout));
  return rc == TFD_OK;
}

int check(tfd_ctx *ctx) {
  // ---------------------------------------------------------------- Laya
  const size_t d = 64, H = 4, hd = d / H, L = 32, B = 2;
  const size_t shape[3] = {3 * d, L, B};
  Lcg rng(1);
  std::vector<float> qkv(3 * d * L * B);
  for (size_t t = 0; t < L * B; ++t)
    for (size_t f = 0; f < 3 * d; ++f) {
      float x = rng.sym();
      if (f >= 2 * d) x = 0.25f + 0.01f * (float)(f - 2 * d);  // value rows equal over tokens
      qkv[f + 3 * d * t] = x;
    }
  // keep[q + L*(k + L*b)]: row 1 padded after 20 tokens (every query keeps
  // the valid keys, as build_mask does for full attention).
  std::vector<uint8_t> keep(L * L * B);
  for (size_t b = 0; b < B; ++b)
    for (size_t k = 0; k < L; ++k)
      for (size_t q = 0; q < L; ++q) keep[q + L * (k + L * b)] = (b == 0 || k < 20) ? 1 : 0;
  auto laya = [&](unsigned flags, std::vector<const void *> &in, float *out) {
    return tfd_laya_attention_block_f32(ctx, (const float *)in[0], shape, 3, qkv.size(),
                                        (const uint8_t *)in[1], keep.size(), d, H,
                                        bits(160000.0f), out, d * L * B, flags);
  };
  std::vector<float> ho, dout;
  bool ok = both_paths({qkv}, &keep, d * L * B, laya, ho, dout);
  expect(ok, "laya: both pointer paths return TFD_OK");
  bool mean_ok = ok;
  for (size_t t = 0; t < L * B && ok; ++t)
    for (size_t f = 0; f < d; ++f)
      mean_ok = mean_ok && close(ho[f + d * t], 0.25f + 0.01f * (float)f, 1e-5f);
  expect(mean_ok, "laya: equal value rows come back unchanged (weights sum to one)");
  expect(ok && std::memcmp(ho.data(), dout.data(), ho.size() * 4) == 0,
         "laya: host and device pointer paths agree bitwise");

  // A single kept key per query copies that key's value row.
  for (size_t t = 0; t < L * B; ++t)
    for (size_t f = 2 * d; f < 3 * d; ++f) qkv[f + 3 * d * t] = rng.sym();
  for (size_t b = 0; b < B; ++b)
    for (size_t k = 0; k < L; ++k)
      for (size_t q = 0; q < L; ++q) keep[q + L * (k + L * b)] = k == (q * 7 + 3) % L;
  ok = both_paths({qkv}, &keep, d * L * B, laya, ho, dout);
  bool copy_ok = ok;
  for (size_t b = 0; b < B && ok; ++b)
    for (size_t q = 0; q < L; ++q) {
      const size_t k = (q * 7 + 3) % L;
      for (size_t f = 0; f < d; ++f)
        copy_ok = copy_ok && close(ho[f + d * (q + L * b)], qkv[2 * d + f + 3 * d * (k + L * b)],
                                   1e-6f);
    }
  expect(copy_ok, "laya: a single kept key copies its value row");
  (void)hd;

  // ---------------------------------------------------------------- Jeff
  const size_t JL = 24, JH = 2, jhd = 32, W = JH * jhd;
  const size_t qshape[2] = {JL, W};
  std::vector<float> q(JL * W), k(JL * W), v(JL * W), g(JL * W), qn(jhd), kn(jhd), mask(JL, 0.0f);
  for (auto *vec : {&q, &k, &v, &g})
    for (auto &x : *vec) x = rng.sym();
  for (auto &x : qn) x = 0.1f * rng.sym();
  for (auto &x : kn) x = 0.1f * rng.sym();
  mask[0] = 1.0f;  // only key 0 is active
  auto jeff = [&](unsigned flags, std::vector<const void *> &in, float *out) {
    return tfd_jeff_full_attention_f32(
        ctx, (const float *)in[0], qshape, 2, (const float *)in[1], k.size(), (const float *)in[2],
        v.size(), (const float *)in[3], g.size(), (const float *)in[4], qn.size(),
        (const float *)in[5], kn.size(), (const float *)in[6], mask.size(), JH, jhd, 16,
        bits(10000.0f), bits(1e-6f), out, JL * W, flags);
  };
  ok = both_paths({q, k, v, g, qn, kn, mask}, nullptr, JL * W, jeff, ho, dout);
  expect(ok, "jeff: both pointer paths return TFD_OK");
  bool gate_ok = ok;
  for (size_t t = 0; t < JL && ok; ++t)
    for (size_t f = 0; f < W; ++f) {
      // (L, W) token-contiguous: element t + L*f
      const float want = v[0 + JL * f] / (1.0f + std::exp(-g[t + JL * f]));
      gate_ok = gate_ok && close(ho[t + JL * f], want, 1e-5f);
    }
  expect(gate_ok, "jeff: one active key gives v[0] * sigmoid(gate) for every query");
  expect(ok && std::memcmp(ho.data(), dout.data(), ho.size() * 4) == 0,
         "jeff: host and device pointer paths agree bitwise");

  // ---------------------------------------------------------------- errors
  const size_t bad_shape[3] = {3 * d + 1, L, B};
  const int rc = tfd_laya_attention_block_f32(ctx, qkv.data(), bad_shape, 3, qkv.size(),
                                              keep.data(), keep.size(), d, H, bits(160000.0f),
                                              ho.data(), d * L * B, TFD_HOST_PTRS);
  expect(rc == TFD_EINVAL && std::strstr(tfd_last_error(ctx), "attention block expects") != nullptr,
         "laya: a (3d+1, L, B) input is rejected with the reference's message");
  // cpu-kernels lib.rs:1205-1210: short storage is rejected before any access.
  const int rs = tfd_laya_attention_block_f32(ctx, qkv.data(), shape, 3, qkv.size() - 1,
                                              keep.data(), keep.size(), d, H, bits(160000.0f),
                                              ho.data(), d * L * B, TFD_HOST_PTRS);
  expect(rs == TFD_EINVAL && std::strstr(tfd_last_error(ctx), "qkv length") != nullptr,
         "laya: qkv storage one element short is rejected (\"qkv length\")");
  std::printf("%d failure(s)\n", failures);
  return failures == 0 ? 0 : 1;
}

int bench(tfd_ctx *ctx) {
  const size_t d = 768, H = 12, hd = d / H, L = 512, B = 8;
  const size_t shape[3] = {3 * d, L, B};
  Lcg rng(2);
  std::vector<float> qkv(3 * d * L * B);
  for (auto &x : qkv) x = 0.554f * rng.sym();  // about N(0, 0.32^2): C2's qkv scale
  std::vector<uint8_t> keep(L * L * B);
  size_t pairs = 0;
  for (size_t b = 0; b < B; ++b) {
    const size_t len = 64 + (size_t)(rng.uniform() * 449.0f);
    for (size_t k = 0; k < L; ++k)
      for (size_t q = 0; q < L; ++q) {
        keep[q + L * (k + L * b)] = k < len;
        pairs += k < len;
      }
  }
  float *dq = nullptr, *dout = nullptr;
  uint8_t *dk = nullptr;
  if (hipMalloc(&dq, qkv.size() * 4) != hipSuccess || hipMalloc(&dk, keep.size()) != hipSuccess ||
      hipMalloc(&dout, d * L * B * 4) != hipSuccess) {
    std::fprintf(stderr, "hipMalloc failed\n");
    return 3;
  }
  hip_ok(hipMemcpy(dq, qkv.data(), qkv.size() * 4, hipMemcpyHostToDevice));
  hip_ok(hipMemcpy(dk, keep.data(), keep.size(), hipMemcpyHostToDevice));
  auto call = [&] {
    return tfd_laya_attention_block_f32(ctx, dq, shape, 3, qkv.size(), dk, keep.size(), d, H,
                                        bits(160000.0f), dout, d * L * B,
                                        TFD_DEVICE_PTRS | TFD_ASYNC);
  };
  hipStream_t s = (hipStream_t)tfd_ctx_stream(ctx);
  for (int i = 0; i < 2000; ++i)  // clocks settle and warm up
    if (call() != TFD_OK) {
      std::fprintf(stderr, "%s\n", tfd_last_error(ctx));
      return 1;
    }
  hipEvent_t e0, e1;
  hip_ok(hipEventCreate(&e0));
  hip_ok(hipEventCreate(&e1));
  const int steps = 100;
  hip_ok(hipEventRecord(e0, s));
  for (int i = 0; i < steps; ++i) call();
  hip_ok(hipEventRecord(e1, s));
  hip_ok(hipEventSynchronize(e1));
  float ms = 0.0f;
  hip_ok(hipEventElapsedTime(&ms, e0, e1));
  const double us = 1e3 * ms / steps, flops = 4.0 * (double)hd * (double)pairs * (double)H;
  std::printf("{\"op\": \"tfd_laya_attention_block_f32\", \"shape\": [2304, 512, 8], "
              "\"us_per_call\": %.2f, \"tflops\": %.3f, \"steps\": %d}\n",
              us, flops / (us * 1e-6) / 1e12, steps);
  hip_ok(hipFree(dq));
  hip_ok(hipFree(dk));
  hip_ok(hipFree(dout));
  return 0;
}

}  // namespace

int main(int argc, char **argv) {
  const char *mode = argc > 1 ? argv[1] : "check";
  if (std::strcmp(mode, "abi") == 0) {
    std::printf("abi %d\n%s\n%s\n", tfd_abi_version(), tfd_laya_attention_block_family_id(),
                tfd_jeff_full_attention_family_id());
    return 0;
  }
  tfd_ctx *ctx = nullptr;
  if (tfd_ctx_create(0, &ctx) != TFD_OK) {
    std::fprintf(stderr, "tfd_ctx_create failed\n");
    return 3;
  }
  int devices = 0;
  if (hipGetDeviceCount(&devices) != hipSuccess || devices == 0) {
    // Arguments are still validated without a device; compute calls are not
    // run (there is no CPU fallback).
    const size_t bad_shape[3] = {193, 32, 2};
    float x[4] = {0, 0, 0, 0};
    const int v = tfd_laya_attention_block_f32(ctx, x, bad_shape, 3, 4, nullptr, 0, 64, 4, 0, x,
                                               4, TFD_HOST_PTRS);
    std::printf("no GPU: validation %s (%s); compute checks need a GPU\n",
                v == TFD_EINVAL ? "works" : "FAILED", tfd_last_error(ctx));
    tfd_ctx_destroy(ctx);
    return v == TFD_EINVAL ? 77 : 1;
  }
  int rc = 2;
  if (std::strcmp(mode, "check") == 0)
    rc = check(ctx);
  else if (std::strcmp(mode, "bench") == 0)
    rc = bench(ctx);
  else
    std::fprintf(stderr, "usage: tfd_driver [abi|check|bench]\n");
  tfd_ctx_destroy(ctx);
  return rc;
}
