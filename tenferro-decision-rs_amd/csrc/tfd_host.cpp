// Host side of the C ABI declared in include/tfd_attention.h.
//
// Mirrors the reference extension ops' execute_in_session:
//   Laya: crates/tenferro-ext/src/laya_attention.rs:99-176
//   Jeff: crates/tenferro-ext/src/jeff_attention.rs:103-184
// including their validation order and messages, then runs the gfx950
// kernels on the context's stream. No CPU fallback exists: every failure to
// reach the GPU is reported as TFD_EHIP.
#include "tfd_attention.h"
#include "tfd_laya_model.h"

#include <hip/hip_runtime.h>
#include <rocblas/rocblas.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "tfd_internal.hpp"

namespace {

constexpr const char *kLayaFamily = "tenferro-decision.laya_attention_block.v1";
constexpr const char *kJeffFamily = "tenferro-decision.jeff_full_attention.v1";
constexpr const char *kLayaOp = "tenferro-ext::laya_attention_block";
constexpr const char *kJeffOp = "tenferro-ext::jeff_full_attention";
constexpr float kLog2e = 1.4426950408889634f;
constexpr size_t kRopeCacheEntries = 8;

struct DevBuf {
  void *ptr = nullptr;
  size_t cap = 0;
};

struct RopeEntry {
  int kind = 0;  // 0 = Laya (L, hd/2), 1 = Jeff (L, rot/2)
  size_t length = 0, dim = 0;
  uint32_t bits = 0;
  float *cos_d = nullptr, *sin_d = nullptr;
  size_t bytes = 0;
  uint64_t stamp = 0;
};

}  // namespace

struct tfd_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  bool adopted = false;  // stream given by the caller (may be the null stream)
  bool own_stream = false;
  bool ready = false;
  int cus = 0;  // compute units of the device (launch shape heuristics)
  std::string err;
  DevBuf staging[12];  // uploads of host-pointer operands
  DevBuf bits;        // Laya packed keep words
  DevBuf kp;          // Jeff normalized + rotated keys
  DevBuf layer;       // intermediates of the layer entries (projections, attention output)
  DevBuf model;       // activations and token inputs of the model forward
  std::vector<uint8_t> model_host;  // packed token inputs of the last model forward
  bool model_inflight = false;      // an asynchronous forward may still read model_host
  rocblas_handle blas = nullptr;  // the layer entries' GEMMs, on `stream`
  std::vector<RopeEntry> rope;
  uint64_t clock = 0;
  bool timing = false;
  std::vector<hipEvent_t> events;  // pairs: [2i] before, [2i+1] after launch i
  size_t events_used = 0;
};

namespace {

int fail(tfd_ctx *c, int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  c->err = buf;
  return code;
}

// invalid_argument(op, field, message) of the reference.
int invalid(tfd_ctx *c, const char *op, const char *field, const char *msg) {
  return fail(c, TFD_EINVAL, "%s: invalid argument `%s`: %s", op, field, msg);
}

int hip_fail(tfd_ctx *c, hipError_t e, const char *what) {
  return fail(c, TFD_EHIP, "%s: %s (%s)", what, hipGetErrorString(e), hipGetErrorName(e));
}

#define TFD_HIP(c, expr, what)                \
  do {                                        \
    hipError_t e_ = (expr);                   \
    if (e_ != hipSuccess) return hip_fail((c), e_, (what)); \
  } while (0)

bool mul_ok(size_t a, size_t b, size_t *out) {
  if (a != 0 && b > SIZE_MAX / a) return false;
  *out = a * b;
  return true;
}

int ensure_ready(tfd_ctx *c) {
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count == 0)
    return fail(c, TFD_EHIP, "no HIP device available (%s); tfd has no CPU fallback",
                e == hipSuccess ? "0 devices" : hipGetErrorString(e));
  if (c->device < 0 || c->device >= count)
    return fail(c, TFD_EHIP, "device %d out of range (%d devices)", c->device, count);
  TFD_HIP(c, hipSetDevice(c->device), "hipSetDevice");
  if (!c->ready) {
    if (!c->adopted) {
      TFD_HIP(c, hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking), "hipStreamCreate");
      c->own_stream = true;
    }
    TFD_HIP(c, hipDeviceGetAttribute(&c->cus, hipDeviceAttributeMultiprocessorCount, c->device),
            "hipDeviceGetAttribute");
    c->ready = true;
  }
  return TFD_OK;
}

int reserve(tfd_ctx *c, DevBuf &b, size_t bytes) {
  if (bytes <= b.cap) return TFD_OK;
  if (b.ptr) {
    TFD_HIP(c, hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    TFD_HIP(c, hipFree(b.ptr), "hipFree");
    b.ptr = nullptr;
    b.cap = 0;
  }
  size_t cap = bytes < 256 ? 256 : bytes;
  TFD_HIP(c, hipMalloc(&b.ptr, cap), "hipMalloc");
  b.cap = cap;
  return TFD_OK;
}

// Device operand: the caller's pointer, or an upload of the host buffer into
// staging slot `slot`.
int operand(tfd_ctx *c, unsigned flags, int slot, const void *host_or_dev, size_t bytes,
            const void **dev) {
  if (flags & TFD_DEVICE_PTRS) {
    *dev = host_or_dev;
    return TFD_OK;
  }
  int rc = reserve(c, c->staging[slot], bytes);
  if (rc) return rc;
  if (bytes)
    TFD_HIP(c, hipMemcpyAsync(c->staging[slot].ptr, host_or_dev, bytes, hipMemcpyHostToDevice,
                              c->stream),
            "hipMemcpyAsync H2D");
  *dev = c->staging[slot].ptr;
  return TFD_OK;
}

int output(tfd_ctx *c, unsigned flags, int slot, void *host_or_dev, size_t bytes, void **dev) {
  if (flags & TFD_DEVICE_PTRS) {
    *dev = host_or_dev;
    return TFD_OK;
  }
  int rc = reserve(c, c->staging[slot], bytes);
  if (rc) return rc;
  *dev = c->staging[slot].ptr;
  return TFD_OK;
}

int finish(tfd_ctx *c, unsigned flags, void *host_out, const void *dev_out, size_t bytes) {
  if (!(flags & TFD_DEVICE_PTRS)) {
    if (bytes)
      TFD_HIP(c, hipMemcpyAsync(host_out, dev_out, bytes, hipMemcpyDeviceToHost, c->stream),
              "hipMemcpyAsync D2H");
    TFD_HIP(c, hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    return TFD_OK;
  }
  if (!(flags & TFD_ASYNC)) TFD_HIP(c, hipStreamSynchronize(c->stream), "hipStreamSynchronize");
  return TFD_OK;
}

// RoPE tables. Laya (cpu-kernels lib.rs:874-888): theta = (l as f32) *
// base.powf(-2 i / hd) for i < hd/2. Jeff (lib.rs:692-709): angle = (t as
// f32) * theta.powf(-2 i / rot) for i < rot/2. Both in f32 with the C
// library's powf/cosf/sinf, which is what Rust's f32 methods call on
// linux-gnu.
int rope_table(tfd_ctx *c, int kind, size_t length, size_t dim, float base, uint32_t bits,
               const float **cos_d, const float **sin_d) {
  const size_t half = dim / 2;
  for (auto &e : c->rope) {
    if (e.kind == kind && e.length == length && e.dim == dim && e.bits == bits) {
      e.stamp = ++c->clock;
      *cos_d = e.cos_d;
      *sin_d = e.sin_d;
      return TFD_OK;
    }
  }
  std::vector<float> ct(length * half + 1), st(length * half + 1);
  for (size_t l = 0; l < length; ++l) {
    for (size_t i = 0; i < half; ++i) {
      volatile float expo = -2.0f * (float)i / (float)dim;
      volatile float angle = (float)l * powf(base, expo);
      ct[l * half + i] = cosf(angle);
      st[l * half + i] = sinf(angle);
    }
  }
  RopeEntry ent;
  if (c->rope.size() >= kRopeCacheEntries) {
    size_t victim = 0;
    for (size_t i = 1; i < c->rope.size(); ++i)
      if (c->rope[i].stamp < c->rope[victim].stamp) victim = i;
    TFD_HIP(c, hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    TFD_HIP(c, hipFree(c->rope[victim].cos_d), "hipFree");
    TFD_HIP(c, hipFree(c->rope[victim].sin_d), "hipFree");
    c->rope.erase(c->rope.begin() + victim);
  }
  ent.kind = kind;
  ent.length = length;
  ent.dim = dim;
  ent.bits = bits;
  ent.bytes = 2 * sizeof(float) * ct.size();
  // Allocate and upload both tables; on any failure free what was allocated.
  const char *what = "hipMalloc";
  hipError_t e = hipMalloc((void **)&ent.cos_d, sizeof(float) * ct.size());
  if (e == hipSuccess) e = hipMalloc((void **)&ent.sin_d, sizeof(float) * st.size());
  if (e == hipSuccess) {
    what = "hipMemcpy rope";
    e = hipMemcpy(ent.cos_d, ct.data(), sizeof(float) * ct.size(), hipMemcpyHostToDevice);
  }
  if (e == hipSuccess)
    e = hipMemcpy(ent.sin_d, st.data(), sizeof(float) * st.size(), hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    if (ent.cos_d) (void)hipFree(ent.cos_d);
    if (ent.sin_d) (void)hipFree(ent.sin_d);
    return hip_fail(c, e, what);
  }
  ent.stamp = ++c->clock;
  c->rope.push_back(ent);
  *cos_d = ent.cos_d;
  *sin_d = ent.sin_d;
  return TFD_OK;
}

// The no-allocation entry's RoPE tables: computed on the host exactly as
// rope_table() does, into a static host buffer, and copied into the first
// kNoallocRopeBytes of the device scratch, a region nothing else writes (the
// packed keep words and tile map start after it, also on calls with RoPE
// off); the (length, dim, base) last copied to each device is remembered,
// and an unchanged table is not copied again. One host buffer serves every
// device, so building and copying a table holds a lock (calls on different
// GPUs from different threads would otherwise overwrite each other's table
// before its copy drains). A new table needs a host copy and a stream
// synchronization, which a stream under graph capture cannot take: such a
// call is refused, and one eager call with the same (length, dim, base)
// makes the table resident first.
constexpr size_t kNoallocRopeMax = (size_t)1 << 19;  // floats per table (L * hd / 2)
constexpr size_t kNoallocRopeBytes = 2 * kNoallocRopeMax * sizeof(float);  // 4 MiB
static_assert(kNoallocRopeBytes % 256 == 0 && kNoallocRopeBytes < tfd::kNoallocScratchBytes,
              "the RoPE region leaves room for the keep words");
float g_noalloc_rope_host[2 * kNoallocRopeMax];
std::mutex g_noalloc_rope_lock;
struct NoallocRopeKey {
  bool valid = false;
  size_t length = 0, dim = 0;
  uint32_t bits = 0;
};
NoallocRopeKey g_noalloc_rope_key[64];

int noalloc_rope_table(tfd_ctx *c, size_t length, size_t dim, float base, uint32_t bits,
                       float *dev, const float **cos_d, const float **sin_d) {
  const size_t half = dim / 2, n = length * half;
  *cos_d = dev;
  *sin_d = dev + n;
  std::lock_guard<std::mutex> guard(g_noalloc_rope_lock);
  NoallocRopeKey &key = g_noalloc_rope_key[c->device];
  if (key.valid && key.length == length && key.dim == dim && key.bits == bits) return TFD_OK;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  TFD_HIP(c, hipStreamIsCapturing(c->stream, &cap), "hipStreamIsCapturing");
  if (cap != hipStreamCaptureStatusNone)
    return fail(c, TFD_EUNSUPPORTED,
                "tfd_laya_attention_block_noalloc_f32: the RoPE table for (length %zu, head_dim "
                "%zu) and this base is not resident and cannot be uploaded under stream capture; "
                "make one call with the same length, head_dim and rope_base before capturing",
                length, dim);
  key.valid = false;
  for (size_t l = 0; l < length; ++l) {
    for (size_t i = 0; i < half; ++i) {
      volatile float expo = -2.0f * (float)i / (float)dim;
      volatile float angle = (float)l * powf(base, expo);
      g_noalloc_rope_host[l * half + i] = cosf(angle);
      g_noalloc_rope_host[n + l * half + i] = sinf(angle);
    }
  }
  TFD_HIP(c, hipMemcpyAsync(dev, g_noalloc_rope_host, 2 * n * sizeof(float), hipMemcpyHostToDevice,
                            c->stream),
          "hipMemcpyAsync rope");
  // The host buffer is reused by the next table: let this copy drain first.
  TFD_HIP(c, hipStreamSynchronize(c->stream), "hipStreamSynchronize");
  key.length = length;
  key.dim = dim;
  key.bits = bits;
  key.valid = true;
  return TFD_OK;
}

// Event pair for the next op's attention kernel(s), recorded by their
// dispatches (timing enabled only; both null otherwise).
int timing_events(tfd_ctx *c, tfd::KernelEvents *ev) {
  *ev = tfd::KernelEvents{};
  if (!c->timing) return TFD_OK;
  while (c->events.size() < 2 * (c->events_used + 1)) {
    hipEvent_t e;
    TFD_HIP(c, hipEventCreate(&e), "hipEventCreate");
    c->events.push_back(e);
  }
  ev->start = c->events[2 * c->events_used];
  ev->stop = c->events[2 * c->events_used + 1];
  c->events_used++;
  return TFD_OK;
}

int pad_head_dim(size_t hd, size_t max_hd) {
  if (hd > max_hd) return 0;
  if (hd <= 32) return 32;
  if (hd <= 64) return 64;
  if (hd <= 128) return 128;
  return 256;
}

float bits_to_f32(uint32_t b) {
  float f;
  std::memcpy(&f, &b, sizeof f);
  return f;
}

int check_flags(tfd_ctx *c, const char *op, unsigned flags, unsigned allowed) {
  if (flags & ~allowed) return invalid(c, op, "flags", "unknown flag bits");
  if ((flags & TFD_ASYNC) && !(flags & TFD_DEVICE_PTRS))
    return invalid(c, op, "flags", "TFD_ASYNC requires TFD_DEVICE_PTRS");
  return TFD_OK;
}

// ------------------------------------------------------------------ Laya run

// noalloc: device pointers only, and every workspace (RoPE tables, packed
// keep words, tile map) lives in the static device scratch: nothing is
// allocated and no timing events are created.
int laya_run(tfd_ctx *c, const char *op, const float *qkv, const uint8_t *keep,
             const uint8_t *valid, int64_t window, size_t hidden, size_t heads, size_t length,
             size_t batch, uint32_t rope_bits, float *out, unsigned flags,
             const uint8_t *qneed = nullptr, bool noalloc = false) {
  size_t n = 0, n3 = 0, keep_len = 0, valid_len = 0;
  if (!mul_ok(hidden, length, &n) || !mul_ok(n, batch, &n) || !mul_ok(n, 3, &n3) ||
      !mul_ok(length, length, &keep_len) || !mul_ok(keep_len, batch, &keep_len) ||
      !mul_ok(length, batch, &valid_len))
    return invalid(c, op, "shape", "attention dimensions overflow");
  if (n == 0) return TFD_OK;
  const bool zero_fill = heads == 0 || hidden % heads != 0;
  const size_t hd = zero_fill ? 0 : hidden / heads;
  // hd_pad 0: past the tiled kernels, the one-wavefront-per-query path
  // (its LDS holds a query row and one score per key).
  const int hd_pad = zero_fill ? 32 : pad_head_dim(hd, tfd::kLayaTiledMaxHd);
  if (!hd_pad && hd + length > 16384)
    return fail(c, TFD_EUNSUPPORTED, "%s: head_dim %zu with length %zu exceeds the LDS of the "
                "path for head dims past %d", op, hd, length, tfd::kLayaTiledMaxHd);
  if (length > (size_t)INT32_MAX / 4 || hidden > (size_t)INT32_MAX / 4)
    return fail(c, TFD_EUNSUPPORTED, "%s: length/hidden too large for the kernels", op);
  if (heads > 65535 || batch > 65535 || (length + tfd::kKeyTile - 1) / tfd::kKeyTile > 65535)
    return fail(c, TFD_EUNSUPPORTED, "%s: heads/batch/length exceed the launch grid", op);
  // No-allocation layout: the RoPE region (kNoallocRopeBytes, whether or not
  // this call uses RoPE), then the packed keep words and the tile map.
  const size_t nkt = (length + tfd::kKeyTile - 1) / tfd::kKeyTile;
  if (noalloc) {
    const size_t words = nkt * batch * length, groups = (size_t)tfd::laya_map_row((int)nkt) * batch * ((length + 63) / 64);
    const size_t need = kNoallocRopeBytes + ((sizeof(uint32_t) * words + 255) & ~(size_t)255) + groups;
    if (length * (hd / 2) > kNoallocRopeMax || need > tfd::kNoallocScratchBytes)
      return fail(c, TFD_EUNSUPPORTED,
                  "%s: needs %zu bytes of workspace; this entry has %zu (use "
                  "tfd_laya_attention_block_f32)", op, need, tfd::kNoallocScratchBytes);
  }
  int rc = ensure_ready(c);
  if (rc) return rc;
  unsigned char *scratch = nullptr;
  if (noalloc) {
    // A stream under graph capture records work and cannot synchronize.
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    TFD_HIP(c, hipStreamIsCapturing(c->stream, &cap), "hipStreamIsCapturing");
    if (cap != hipStreamCaptureStatusNone && !(flags & TFD_ASYNC))
      return invalid(c, op, "flags", "a call under stream capture needs TFD_ASYNC");
    hipError_t e = hipSuccess;
    scratch = static_cast<unsigned char *>(tfd::noalloc_scratch(c->device, &e));
    if (!scratch) return hip_fail(c, e, "hipGetSymbolAddress(scratch)");
  }
  void *out_d = nullptr;
  if ((rc = output(c, flags, 0, out, sizeof(float) * n, &out_d))) return rc;
  if (zero_fill) {
    // laya_attention.rs:141 allocates zeros and the kernel returns early
    // (lib.rs:870-872) when heads == 0 or d % heads != 0.
    TFD_HIP(c, tfd::launch_fill_zero(static_cast<float *>(out_d), n, c->stream), "fill launch");
    return finish(c, flags, out, out_d, sizeof(float) * n);
  }
  const void *qkv_d = nullptr, *mask_d = nullptr;
  if ((rc = operand(c, flags, 1, qkv, sizeof(float) * n3, &qkv_d))) return rc;
  if (keep) {
    if ((rc = operand(c, flags, 2, keep, keep_len, &mask_d))) return rc;
  } else {
    if ((rc = operand(c, flags, 2, valid, valid_len, &mask_d))) return rc;
  }
  tfd::LayaArgs a{};
  a.cus = c->cus;
  a.qkv = static_cast<const float *>(qkv_d);
  a.out = static_cast<float *>(out_d);
  a.qneed = keep ? nullptr : qneed;
  a.d = (int)hidden;
  a.hd = (int)hd;
  a.half = (int)(hd / 2);
  a.L = (int)length;
  a.nkt = (int)((length + tfd::kKeyTile - 1) / tfd::kKeyTile);
  a.window = window < 0 ? -1 : (int)(window > (int64_t)length ? (int64_t)length : window);
  const float scale = 1.0f / sqrtf((float)hd);
  a.c1 = scale * kLog2e;
  const float base = bits_to_f32(rope_bits);
  if (base != 0.0f) {
    rc = noalloc ? noalloc_rope_table(c, length, hd, base, rope_bits,
                                      reinterpret_cast<float *>(scratch), &a.cos_t, &a.sin_t)
                 : rope_table(c, 0, length, hd, base, rope_bits, &a.cos_t, &a.sin_t);
    if (rc) return rc;
  }
  int mode = tfd::kMaskStruct;
  if (!hd_pad) {
    if (keep)
      mode = tfd::kMaskBits;
    else
      a.valid = static_cast<const uint8_t *>(mask_d);
    TFD_HIP(c,
            tfd::launch_laya_generic(a, keep ? static_cast<const uint8_t *>(mask_d) : nullptr,
                                     (int)heads, (int)batch, mode, c->stream),
            "laya_generic launch");
    return finish(c, flags, out, out_d, sizeof(float) * n);
  }
  if (keep && tfd::laya_raw_keep(a.L, (int)heads, (int)batch, a.nkt, c->cus)) {
    // A small grid: the attention kernel packs the keep bytes itself (no
    // packing pass, no workspace).
    mode = tfd::kMaskRaw;
    a.keep = static_cast<const uint8_t *>(mask_d);
  } else if (keep) {
    mode = tfd::kMaskBits;
    // Workspace: the packed words, then the per-(tile, 64-query group) map.
    size_t words = 0, groups = 0;
    if (!mul_ok((size_t)a.nkt * batch, length, &words) ||
        !mul_ok((size_t)tfd::laya_map_row(a.nkt) * batch, (length + 63) / 64, &groups) ||
        words > SIZE_MAX / 8)
      return invalid(c, op, "shape", "attention dimensions overflow");
    const size_t map_off = (sizeof(uint32_t) * words + 255) & ~(size_t)255;
    uint8_t *base = nullptr;
    if (noalloc) {
      base = scratch + kNoallocRopeBytes;
    } else {
      if ((rc = reserve(c, c->bits, map_off + groups))) return rc;
      base = static_cast<uint8_t *>(c->bits.ptr);
    }
    a.bits = reinterpret_cast<const uint32_t *>(base);
    a.any = base + map_off;
    TFD_HIP(c,
            tfd::launch_laya_keep_bits(static_cast<const uint8_t *>(mask_d),
                                       reinterpret_cast<uint32_t *>(base), base + map_off, a.L,
                                       (int)batch, a.nkt, c->stream),
            "laya_keep_bits launch");
  } else {
    a.valid = static_cast<const uint8_t *>(mask_d);
    if (tfd::laya_planned(a.L, (int)heads, (int)batch, hd_pad, c->cus)) {
      // A grid that gets the placement plan: the rows' valid-key words, then
      // the tile map of valid + window.
      const size_t words = (size_t)a.nkt * batch;
      const size_t map_off = (sizeof(uint32_t) * words + 255) & ~(size_t)255;
      const size_t groups = (size_t)tfd::laya_map_row(a.nkt) * batch * ((length + 63) / 64);
      uint8_t *base = nullptr;
      if (noalloc) {
        base = scratch + kNoallocRopeBytes;
      } else {
        if ((rc = reserve(c, c->bits, map_off + groups))) return rc;
        base = static_cast<uint8_t *>(c->bits.ptr);
      }
      a.bits = reinterpret_cast<const uint32_t *>(base);
      a.any = base + map_off;
      TFD_HIP(c,
              tfd::launch_laya_valid_prep(a.valid, reinterpret_cast<uint32_t *>(base),
                                          base + map_off, a.L, (int)batch, a.nkt, a.window,
                                          c->stream),
              "laya_valid_prep launch");
    }
  }
  tfd::KernelEvents ev;
  if (!noalloc && (rc = timing_events(c, &ev))) return rc;
  TFD_HIP(c, tfd::launch_laya_attention(a, (int)heads, (int)batch, hd_pad, mode, c->stream, ev),
          "laya_attention launch");
  return finish(c, flags, out, out_d, sizeof(float) * n);
}

// ------------------------------------------------------------------ Jeff run

// kv_copies > 1: K and V hold kv_heads * kv_copies heads, each group of
// kv_copies consecutive heads identical copies (GQA weights expanded as
// jeff-infer checkpoint.rs:307-319 does); only the first head of each group
// is read.
int jeff_run(tfd_ctx *c, const char *op, bool bf16, size_t rows, size_t length, size_t heads,
             size_t kv_heads, size_t head_dim, size_t rotary_dim, const void *q, const void *k,
             const void *v, const void *gate, const float *q_norm, const float *k_norm,
             const float *mask, uint32_t theta_bits, uint32_t eps_bits, float *out,
             unsigned flags, size_t kv_copies = 1) {
  size_t width = 0, kv_width = 0, qn = 0, kvn = 0, mn = 0, kv_stored = 0;
  if (!mul_ok(heads, head_dim, &width) || !mul_ok(kv_heads, kv_copies, &kv_stored) ||
      !mul_ok(kv_stored, head_dim, &kv_width) ||
      !mul_ok(width, length, &qn) || !mul_ok(qn, rows, &qn) || !mul_ok(kv_width, length, &kvn) ||
      !mul_ok(kvn, rows, &kvn) || !mul_ok(rows, length, &mn))
    return invalid(c, op, "shape", "attention dimensions overflow");
  // cpu-kernels lib.rs:643-645: nothing to do for an empty problem.
  if (qn == 0 || head_dim == 0) return TFD_OK;
  // hd_pad 0: past the tiled kernels, the one-wavefront-per-query path.
  const int hd_pad = pad_head_dim(head_dim, tfd::kJeffTiledMaxHd);
  if (!hd_pad && head_dim + length > 16384)
    return fail(c, TFD_EUNSUPPORTED, "%s: head_dim %zu with length %zu exceeds the LDS of the "
                "path for head dims past %d", op, head_dim, length, tfd::kJeffTiledMaxHd);
  if (length > (size_t)INT32_MAX / 4 || width > (size_t)INT32_MAX / 4)
    return fail(c, TFD_EUNSUPPORTED, "%s: length/width too large for the kernels", op);
  if (heads > 65535 || rows > 65535)
    return fail(c, TFD_EUNSUPPORTED, "%s: heads/rows exceed the launch grid", op);
  int rc = ensure_ready(c);
  if (rc) return rc;
  const size_t es = bf16 ? 2 : 4;
  const void *q_d, *k_d, *v_d, *g_d, *qn_d, *kn_d, *m_d;
  void *out_d;
  if ((rc = operand(c, flags, 1, q, es * qn, &q_d))) return rc;
  if ((rc = operand(c, flags, 2, k, es * kvn, &k_d))) return rc;
  if ((rc = operand(c, flags, 3, v, es * kvn, &v_d))) return rc;
  if ((rc = operand(c, flags, 4, gate, es * qn, &g_d))) return rc;
  if ((rc = operand(c, flags, 5, q_norm, sizeof(float) * head_dim, &qn_d))) return rc;
  if ((rc = operand(c, flags, 6, k_norm, sizeof(float) * head_dim, &kn_d))) return rc;
  if ((rc = operand(c, flags, 7, mask, sizeof(float) * mn, &m_d))) return rc;
  if ((rc = output(c, flags, 0, out, sizeof(float) * qn, &out_d))) return rc;
  tfd::JeffArgs a{};
  a.q = q_d;
  a.k = k_d;
  a.v = v_d;
  a.gate = g_d;
  a.q_norm = static_cast<const float *>(qn_d);
  a.k_norm = static_cast<const float *>(kn_d);
  a.mask = static_cast<const float *>(m_d);
  a.out = static_cast<float *>(out_d);
  a.L = (int)length;
  a.heads = (int)heads;
  a.kv_heads = (int)kv_heads;
  a.hd = (int)head_dim;
  a.rot_half = (int)(rotary_dim / 2);
  a.groups = (int)(heads / kv_heads);
  a.gdiv = tfd::FastDiv::make((uint32_t)a.groups);
  a.kvdiv = tfd::FastDiv::make((uint32_t)kv_heads);
  a.hdiv = tfd::FastDiv::make((uint32_t)heads);
  a.heads_per_group = (a.groups % 4 == 0) ? 4 : (a.groups % 2 == 0) ? 2 : 1;
  a.trim = (flags & TFD_TRIM_LEADING) ? 1 : 0;
  a.cus = c->cus;
  a.eps = bits_to_f32(eps_bits);
  a.c1 = (1.0f / sqrtf((float)head_dim)) * kLog2e;
  a.q_row = qn / rows;
  a.kv_row = kvn / rows;
  a.kv_head = kv_copies * head_dim * length;
  if (a.rot_half > 0) {
    if ((rc = rope_table(c, 1, length, rotary_dim, bits_to_f32(theta_bits), theta_bits, &a.cos_t,
                         &a.sin_t)))
      return rc;
  }
  if (!hd_pad) {
    if ((rc = reserve(c, c->kp, tfd::jeff_generic_kn_bytes(a, (int)rows)))) return rc;
    tfd::KernelEvents ev;
    if ((rc = timing_events(c, &ev))) return rc;
    TFD_HIP(c,
            tfd::launch_jeff_generic(a, (int)rows, bf16, static_cast<float *>(c->kp.ptr),
                                     c->stream, ev),
            "jeff_generic launch");
    return finish(c, flags, out, out_d, sizeof(float) * qn);
  }
  if ((rc = reserve(c, c->kp, tfd::jeff_kp_bytes(a, (int)rows, hd_pad, bf16)))) return rc;
  tfd::KernelEvents ev;
  if ((rc = timing_events(c, &ev))) return rc;
  hipError_t e =
      bf16 ? tfd::launch_jeff_attention_bf16(a, (int)rows, hd_pad, c->kp.ptr, c->stream, ev)
           : tfd::launch_jeff_attention_f32(a, (int)rows, hd_pad, c->kp.ptr, c->stream, ev);
  if (e == hipErrorNotSupported)
    return fail(c, TFD_EUNSUPPORTED, "%s: this variant is not available", op);
  if (e != hipSuccess) return hip_fail(c, e, "jeff_attention launch");
  return finish(c, flags, out, out_d, sizeof(float) * qn);
}

int jeff_rows_common(tfd_ctx *c, bool bf16, size_t rows, size_t length, size_t heads,
                     size_t kv_heads, size_t head_dim, size_t rotary_dim, const void *q,
                     const void *k, const void *v, const void *gate, const float *q_norm,
                     const float *k_norm, const float *mask, uint32_t theta_bits,
                     uint32_t eps_bits, float *out, unsigned flags) {
  const char *op = bf16 ? "tfd_jeff_full_attention_rows_bf16" : "tfd_jeff_full_attention_rows_f32";
  if (!c) return TFD_EINVAL;
  c->err.clear();
  int rc = check_flags(c, op, flags, TFD_DEVICE_PTRS | TFD_ASYNC | TFD_TRIM_LEADING);
  if (rc) return rc;
  if (kv_heads == 0 || heads % kv_heads != 0)
    return invalid(c, op, "kv_heads", "heads must be a multiple of kv_heads");
  if (rotary_dim > head_dim)
    return invalid(c, op, "rotary_dim", "rotary_dim must not exceed head_dim");
  if (rows && length && heads && head_dim &&
      (!q || !k || !v || !gate || !q_norm || !k_norm || !mask || !out))
    return invalid(c, op, "inputs", "null buffer");
  return jeff_run(c, op, bf16, rows, length, heads, kv_heads, head_dim, rotary_dim, q, k, v, gate,
                  q_norm, k_norm, mask, theta_bits, eps_bits, out, flags);
}

// ------------------------------------------------------------------ layers

int blas_fail(tfd_ctx *c, rocblas_status st, const char *what) {
  return fail(c, TFD_EHIP, "%s: rocBLAS status %d (%s)", what, (int)st,
              rocblas_status_to_string(st));
}

int blas_ready(tfd_ctx *c) {
  if (!c->blas) {
    const rocblas_status st = rocblas_create_handle(&c->blas);
    if (st != rocblas_status_success) {
      c->blas = nullptr;
      return blas_fail(c, st, "rocblas_create_handle");
    }
  }
  const rocblas_status st = rocblas_set_stream(c->blas, c->stream);
  if (st != rocblas_status_success) return blas_fail(c, st, "rocblas_set_stream");
  return TFD_OK;
}

// C_b = op(A_b) op(B_b) for b < batch, column-major f32 (strides in
// elements, 0 repeats an operand), on the context's stream.
int gemm(tfd_ctx *c, bool ta, bool tb, size_t m, size_t n, size_t k, const float *A, size_t lda,
         size_t sa, const float *B, size_t ldb, size_t sb, float *C, size_t ldc, size_t sc,
         size_t batch, float beta = 0.0f) {
  if (m > INT32_MAX || n > INT32_MAX || k > INT32_MAX || lda > INT32_MAX || ldb > INT32_MAX ||
      ldc > INT32_MAX || batch > INT32_MAX)
    return fail(c, TFD_EUNSUPPORTED, "linear: dimensions exceed the GEMM interface");
  const float one = 1.0f;
  const rocblas_status st = rocblas_sgemm_strided_batched(
      c->blas, ta ? rocblas_operation_transpose : rocblas_operation_none,
      tb ? rocblas_operation_transpose : rocblas_operation_none, (rocblas_int)m, (rocblas_int)n,
      (rocblas_int)k, &one, A, (rocblas_int)lda, (rocblas_stride)sa, B, (rocblas_int)ldb,
      (rocblas_stride)sb, &beta, C, (rocblas_int)ldc, (rocblas_stride)sc, (rocblas_int)batch);
  if (st != rocblas_status_success) return blas_fail(c, st, "rocblas_sgemm_strided_batched");
  return TFD_OK;
}

// attention_block_tenferro (laya-infer model.rs:1304-1347) on device
// pointers: qkv = W_in^T x (+ b_in), the fused op under a keep tensor or a
// structured (valid, window) mask, out = W_out^T attended (+ b_out); with
// `accumulate` the projection adds into out (a residual stream). Uses the
// context's layer workspace.
int laya_layer_dev(tfd_ctx *c, const char *op, const float *x, size_t hidden, size_t heads,
                   size_t length, size_t batch, const uint8_t *keep, const uint8_t *valid,
                   int64_t window, const float *w_in, const float *b_in, const float *w_out,
                   const float *b_out, uint32_t rope_bits, float *out, bool accumulate) {
  const size_t tokens = length * batch, n = hidden * tokens;
  int rc = 0;
  // Workspace: qkv (3d, L, B), then the attention output (d, L, B).
  if ((rc = reserve(c, c->layer, sizeof(float) * 4 * n))) return rc;
  float *qkv = static_cast<float *>(c->layer.ptr), *att = qkv + 3 * n;
  // qkv = W_in^T x (+ b_in): linear_feature_first (model.rs:1179-1216).
  if ((rc = gemm(c, true, false, 3 * hidden, tokens, hidden, w_in, hidden, 0, x, hidden, 0, qkv,
                 3 * hidden, 0, 1)))
    return rc;
  if (b_in)
    TFD_HIP(c, tfd::launch_add_row_bias(qkv, b_in, (int)(3 * hidden), tokens, c->stream),
            "bias launch");
  if ((rc = laya_run(c, op, qkv, keep, valid, window, hidden, heads, length, batch, rope_bits, att,
                     TFD_DEVICE_PTRS | TFD_ASYNC)))
    return rc;
  if ((rc = gemm(c, true, false, hidden, tokens, hidden, w_out, hidden, 0, att, hidden, 0, out,
                 hidden, 0, 1, accumulate ? 1.0f : 0.0f)))
    return rc;
  if (b_out)
    TFD_HIP(c, tfd::launch_add_row_bias(out, b_out, (int)hidden, tokens, c->stream),
            "bias launch");
  return TFD_OK;
}

// attention_block_tenferro (laya-infer model.rs:1304-1347) on the f32 path.
int laya_layer(tfd_ctx *c, const float *x, size_t hidden, size_t heads, size_t length,
               size_t batch, const uint8_t *keep, const float *w_in, const float *b_in,
               const float *w_out, const float *b_out, uint32_t rope_bits, float *out,
               unsigned flags) {
  const char *op = "tfd_laya_attention_layer_f32";
  size_t n = 0, tokens = 0, keep_len = 0, wi = 0, wo = 0;
  if (!mul_ok(length, batch, &tokens) || !mul_ok(hidden, tokens, &n) ||
      !mul_ok(length, length, &keep_len) || !mul_ok(keep_len, batch, &keep_len) ||
      !mul_ok(hidden, hidden, &wo) || !mul_ok(wo, 3, &wi) || n > SIZE_MAX / 16)
    return invalid(c, op, "shape", "attention dimensions overflow");
  if (n == 0) return TFD_OK;
  if (!x || !keep || !w_in || !w_out || !out) return invalid(c, op, "inputs", "null buffer");
  int rc = ensure_ready(c);
  if (rc) return rc;
  if ((rc = blas_ready(c))) return rc;
  const void *x_d = nullptr, *k_d = nullptr, *wi_d = nullptr, *wo_d = nullptr, *bi_d = nullptr,
             *bo_d = nullptr;
  void *out_d = nullptr;
  if ((rc = operand(c, flags, 1, x, sizeof(float) * n, &x_d))) return rc;
  if ((rc = operand(c, flags, 2, keep, keep_len, &k_d))) return rc;
  if ((rc = operand(c, flags, 3, w_in, sizeof(float) * wi, &wi_d))) return rc;
  if ((rc = operand(c, flags, 4, w_out, sizeof(float) * wo, &wo_d))) return rc;
  if (b_in && (rc = operand(c, flags, 5, b_in, sizeof(float) * 3 * hidden, &bi_d))) return rc;
  if (b_out && (rc = operand(c, flags, 6, b_out, sizeof(float) * hidden, &bo_d))) return rc;
  if ((rc = output(c, flags, 0, out, sizeof(float) * n, &out_d))) return rc;
  if ((rc = laya_layer_dev(c, op, static_cast<const float *>(x_d), hidden, heads, length, batch,
                           static_cast<const uint8_t *>(k_d), nullptr, -1,
                           static_cast<const float *>(wi_d), static_cast<const float *>(bi_d),
                           static_cast<const float *>(wo_d), static_cast<const float *>(bo_d),
                           rope_bits, static_cast<float *>(out_d), false)))
    return rc;
  return finish(c, flags, out, out_d, sizeof(float) * n);
}

// full_attention_tenferro (jeff-infer model.rs:686-780) on the f32 path,
// over rows.
int jeff_layer(tfd_ctx *c, size_t rows, size_t length, size_t hidden, size_t heads,
               size_t kv_heads, size_t head_dim, size_t rotary_dim, const float *x,
               const float *w_q, const float *w_gate, const float *w_k, const float *w_v,
               const float *w_o, const float *q_norm, const float *k_norm, const float *mask,
               uint32_t theta_bits, uint32_t eps_bits, float *out, unsigned flags) {
  const char *op = "tfd_jeff_full_attention_layer_rows_f32";
  if (kv_heads == 0 || heads % kv_heads != 0)
    return invalid(c, op, "kv_heads", "heads must be a multiple of kv_heads");
  if (rotary_dim > head_dim)
    return invalid(c, op, "rotary_dim", "rotary_dim must not exceed head_dim");
  size_t W = 0, KW = 0, xn = 0, qn = 0, kvn = 0, mn = 0, wq = 0, wk = 0;
  if (!mul_ok(heads, head_dim, &W) || !mul_ok(kv_heads, head_dim, &KW) ||
      !mul_ok(length, hidden, &xn) || !mul_ok(xn, rows, &xn) || !mul_ok(length, W, &qn) ||
      !mul_ok(qn, rows, &qn) || !mul_ok(length, KW, &kvn) || !mul_ok(kvn, rows, &kvn) ||
      !mul_ok(rows, length, &mn) || !mul_ok(hidden, W, &wq) || !mul_ok(hidden, KW, &wk) ||
      qn > SIZE_MAX / 32)
    return invalid(c, op, "shape", "attention dimensions overflow");
  if (xn == 0) return TFD_OK;
  if (!x || !w_q || !w_gate || !w_k || !w_v || !w_o || !q_norm || !k_norm || !mask || !out)
    return invalid(c, op, "inputs", "null buffer");
  int rc = ensure_ready(c);
  if (rc) return rc;
  if ((rc = blas_ready(c))) return rc;
  const void *x_d = nullptr, *wq_d = nullptr, *wg_d = nullptr, *wk_d = nullptr, *wv_d = nullptr,
             *wo_d = nullptr, *qn_d = nullptr, *kn_d = nullptr, *m_d = nullptr;
  void *out_d = nullptr;
  if ((rc = operand(c, flags, 1, x, sizeof(float) * xn, &x_d))) return rc;
  if ((rc = operand(c, flags, 2, w_q, sizeof(float) * wq, &wq_d))) return rc;
  if ((rc = operand(c, flags, 3, w_gate, sizeof(float) * wq, &wg_d))) return rc;
  if ((rc = operand(c, flags, 4, w_k, sizeof(float) * wk, &wk_d))) return rc;
  if ((rc = operand(c, flags, 5, w_v, sizeof(float) * wk, &wv_d))) return rc;
  if ((rc = operand(c, flags, 6, w_o, sizeof(float) * wq, &wo_d))) return rc;
  if ((rc = operand(c, flags, 7, q_norm, sizeof(float) * head_dim, &qn_d))) return rc;
  if ((rc = operand(c, flags, 8, k_norm, sizeof(float) * head_dim, &kn_d))) return rc;
  if ((rc = operand(c, flags, 9, mask, sizeof(float) * mn, &m_d))) return rc;
  if ((rc = output(c, flags, 0, out, sizeof(float) * xn, &out_d))) return rc;
  // Workspace: q, gate, merged (rows x (L, W)), then k, v (rows x (L, KW)).
  if ((rc = reserve(c, c->layer, sizeof(float) * (3 * qn + 2 * kvn)))) return rc;
  float *q = static_cast<float *>(c->layer.ptr), *g = q + qn, *merged = g + qn, *k = merged + qn,
        *v = k + kvn;
  const float *xf = static_cast<const float *>(x_d);
  // y_r = x_r W for every row r, (L, hidden) x (hidden, out): linear_tenferro
  // (model.rs:289-317).
  auto proj = [&](const void *w, size_t out_dim, float *y) {
    return gemm(c, false, false, length, out_dim, hidden, xf, length, length * hidden,
                static_cast<const float *>(w), hidden, 0, y, length, length * out_dim, rows);
  };
  if ((rc = proj(wq_d, W, q)) || (rc = proj(wg_d, W, g)) || (rc = proj(wk_d, KW, k)) ||
      (rc = proj(wv_d, KW, v)))
    return rc;
  if ((rc = jeff_run(c, op, false, rows, length, heads, kv_heads, head_dim, rotary_dim, q, k, v, g,
                     static_cast<const float *>(qn_d), static_cast<const float *>(kn_d),
                     static_cast<const float *>(m_d), theta_bits, eps_bits, merged,
                     (flags & TFD_TRIM_LEADING) | TFD_DEVICE_PTRS | TFD_ASYNC)))
    return rc;
  if ((rc = gemm(c, false, false, length, hidden, W, merged, length, length * W,
                 static_cast<const float *>(wo_d), W, 0, static_cast<float *>(out_d), length,
                 length * hidden, rows)))
    return rc;
  return finish(c, flags, out, out_d, sizeof(float) * xn);
}

// ------------------------------------------------------------ model forward

// LayerNorm columns (see tfd::NormArgs) on the context's stream.
int norm_cols(tfd_ctx *c, const float *x, const int *map, long cols, size_t d, const float *w,
              const float *b, float eps, float *y, const float *add = nullptr,
              const int *add_col = nullptr, size_t per = 1) {
  tfd::NormArgs a{};
  a.x = x;
  a.map = map;
  a.w = w;
  a.b = b;
  a.add = add;
  a.add_col = add_col;
  a.y = y;
  a.cols = cols;
  a.ldx = (int)d;
  a.d = (int)d;
  a.per = (int)per;
  a.eps = eps;
  TFD_HIP(c, tfd::launch_norm_columns(a, c->stream), "norm launch");
  return TFD_OK;
}

// y (out, cols) = W^T x for a column-major (in, out) weight, then + bias and
// the activation (linear_host, model.rs:424-457, with the elementwise maps
// the forward applies to its result). `accumulate`: y += W^T x instead.
int linear_cols(tfd_ctx *c, const float *w, const float *b, size_t in, size_t out,
                const float *x, size_t cols, float *y, int act, bool accumulate = false) {
  int rc = gemm(c, true, false, out, cols, in, w, in, 0, x, in, 0, y, out, 0, 1,
                accumulate ? 1.0f : 0.0f);
  if (rc) return rc;
  if (b || act != tfd::kActNone)
    TFD_HIP(c, tfd::launch_bias_act(y, b, (int)out, cols, act, c->stream), "bias launch");
  return TFD_OK;
}

int missing(tfd_ctx *c, const char *op, const std::string &field) {
  return invalid(c, op, field.c_str(), "missing weights");
}

// LayaWeights::validate (model.rs:187-295) on the shapes the struct carries;
// the element counts are fixed by those shapes.
int validate_model(tfd_ctx *c, const char *op, const tfd_laya_model *m) {
  const size_t d = m->hidden;
  if (d == 0) return invalid(c, op, "encoder.hidden_size", "must be positive");
  if (!m->tok_embeddings || m->vocab == 0)
    return invalid(c, op, "laya.tok_embeddings", "shape must be (hidden, vocab)");
  if (!m->embed_norm_w) return missing(c, op, "laya.embed_norm");
  if (!m->final_norm_w) return missing(c, op, "laya.final_norm");
  if (m->n_layers && !m->layers) return missing(c, op, "laya.layers");
  for (size_t i = 0; i < m->n_layers; ++i) {
    const tfd_laya_encoder_layer &l = m->layers[i];
    const std::string f = "laya.layers[" + std::to_string(i) + "]";
    if (m->heads == 0 || d % m->heads != 0)
      return invalid(c, op, (f + ".num_heads").c_str(), "must divide hidden_size");
    if ((d / m->heads) % 2 != 0)
      return invalid(c, op, (f + ".num_heads").c_str(),
                     "the attention head dimension must be even for RoPE");
    if (!l.wqkv) return missing(c, op, f + ".wqkv");
    if (!l.wo) return missing(c, op, f + ".wo");
    if (!l.mlp_norm_w) return missing(c, op, f + ".mlp_norm");
    if (!l.wi) return missing(c, op, f + ".wi");
    if (!l.wo_mlp) return missing(c, op, f + ".wo_mlp");
    const float base = bits_to_f32(l.rope_base_bits);
    if (!(std::isfinite(base) && base > 0.0f))
      return invalid(c, op, (f + ".rope_base").c_str(), "must be a positive finite number");
  }
  if (m->n_layers && m->intermediate == 0) return missing(c, op, "laya.layers[0].wi");
  if (!m->type_emb) return invalid(c, op, "laya.type_emb", "shape must be (hidden, 3)");
  if (!m->scorer_norm_w) return missing(c, op, "laya.scorer_norm");
  if (!m->scorer1_w) return missing(c, op, "laya.scorer1");
  if (!m->scorer2_w) return missing(c, op, "laya.scorer2");
  if (m->n_head_layers && !m->head) return missing(c, op, "laya.head");
  for (size_t i = 0; i < m->n_head_layers; ++i) {
    const tfd_laya_head_layer &h = m->head[i];
    const std::string f = "laya.head[" + std::to_string(i) + "]";
    if (h.heads == 0 || d % h.heads != 0)
      return invalid(c, op, (f + ".num_heads").c_str(), "must divide hidden_size");
    if (!h.norm1_w) return missing(c, op, f + ".norm1");
    if (!h.in_proj_w) return missing(c, op, f + ".in_proj");
    if (!h.out_proj_w) return missing(c, op, f + ".out_proj");
    if (!h.norm2_w) return missing(c, op, f + ".norm2");
    if (!h.linear1_w || h.ff == 0)
      return invalid(c, op, (f + ".linear1").c_str(), "shape must be (hidden, ff)");
    if (!h.linear2_w) return missing(c, op, f + ".linear2");
  }
  if (!m->act1_w || m->action_hidden == 0) return missing(c, op, "laya.act1");
  if (!m->act2_w || m->actions == 0) return missing(c, op, "laya.act2");
  return TFD_OK;
}

// forward_reference (laya-infer model.rs:867-977): encoder (646-713), typed
// head (916-935), head layers (715-747), marker scorer (937-941), pooling
// (773-837) and the action head (943-966), all on the context's stream.
int laya_forward(tfd_ctx *c, const tfd_laya_model *m, const int64_t *ids, const uint8_t *mask,
                 size_t L, size_t B, const int64_t *marker_pos, const uint8_t *marker_mask,
                 size_t K, const int64_t *qtype, float *logits, float *action, unsigned flags) {
  const char *op = "tfd_laya_forward_f32";
  if (!m) return invalid(c, op, "model", "null model");
  // The reference's checks, in its order (model.rs:877-911, 661-669, 920-927).
  if (B == 0) return invalid(c, op, "laya.qtype", "the batch must be non-empty");
  if (L == 0) return invalid(c, op, "laya.ids", "ids must be a non-empty (L, B) batch");
  if (!ids || !mask || !qtype || (K && (!marker_pos || !marker_mask)) || !logits || !action)
    return invalid(c, op, "inputs", "null buffer");
  int rc = validate_model(c, op, m);
  if (rc) return rc;
  if (K < 2) return invalid(c, op, "laya.marker_pos", "at least two marker slots are required");
  const size_t d = m->hidden, I = m->intermediate, AH = m->action_hidden, A = m->actions;
  size_t T = 0, KB = 0, xs = 0;
  if (!mul_ok(L, B, &T) || !mul_ok(K, B, &KB) || !mul_ok(d, T, &xs) || T > (size_t)INT32_MAX ||
      KB > (size_t)INT32_MAX || d > (size_t)INT32_MAX / 4 || xs > SIZE_MAX / 64)
    return invalid(c, op, "shape", "dimensions overflow");
  for (size_t t = 0; t < T; ++t)
    if (ids[t] < 0 || (uint64_t)ids[t] >= m->vocab)
      return invalid(c, op, "laya.ids", "token id is outside the vocabulary");
  for (size_t b = 0; b < B; ++b)
    if (qtype[b] < 0 || qtype[b] > 2)
      return invalid(c, op, "laya.qtype", "qtype must be 0 (choice), 1 (score) or 2 (noul)");
  // gather_markers_host reads token max(pos, 0) of its own row.
  for (size_t j = 0; j < KB; ++j)
    if (marker_pos[j] >= (int64_t)L)
      return invalid(c, op, "laya.marker_pos", "marker position outside the sequence");
  size_t ff_max = 0;
  for (size_t i = 0; i < m->n_head_layers; ++i) ff_max = std::max(ff_max, m->head[i].ff);
  const size_t wide = std::max(2 * I, ff_max);
  if (wide > SIZE_MAX / 64 / (T ? T : 1)) return invalid(c, op, "shape", "dimensions overflow");
  const float eps = bits_to_f32(m->eps_bits);
  if ((rc = ensure_ready(c))) return rc;
  if ((rc = blas_ready(c))) return rc;

  // The columns the outputs read: every valid token (keys, and queries whose
  // states reach the head), token 0 of every prompt (pooled, model.rs:944-948)
  // and every marker position (gather_markers_host, 749-771), even where
  // padded. All per-token work runs on these packed columns only; other
  // padded tokens never reach a valid token (they are masked as keys) or an
  // output, so skipping them changes no result.
  if (c->model_inflight) {
    TFD_HIP(c, hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    c->model_inflight = false;
  }
  std::vector<int32_t> pidx(T, -1);
  for (size_t t = 0; t < T; ++t)
    if (mask[t]) pidx[t] = 0;
  for (size_t b = 0; b < B; ++b) pidx[L * b] = 0;
  for (size_t j = 0; j < KB; ++j)
    pidx[(size_t)(marker_pos[j] < 0 ? 0 : marker_pos[j]) + L * (j / K)] = 0;
  size_t Tc = 0;
  for (size_t t = 0; t < T; ++t)
    if (pidx[t] == 0) pidx[t] = (int32_t)Tc++;
  // Packed host inputs: ids, padded column, qtype per packed column (Tc
  // i32 each); packed marker columns (KB i32); packed token 0 (B i32);
  // valid (T u8); marker mask (KB u8).
  auto up = [](size_t bytes) { return (bytes + 255) & ~(size_t)255; };
  const size_t o_cols = up(4 * Tc), o_qt = o_cols + up(4 * Tc), o_mk = o_qt + up(4 * Tc),
               o_h0 = o_mk + up(4 * KB), o_valid = o_h0 + up(4 * B), o_mm = o_valid + up(T),
               o_need = o_mm + up(KB), host_bytes = o_need + up(T);
  c->model_host.assign(host_bytes, 0);
  uint8_t *hb = c->model_host.data();
  int32_t *h_ids = reinterpret_cast<int32_t *>(hb), *h_cols = reinterpret_cast<int32_t *>(hb + o_cols),
          *h_qt = reinterpret_cast<int32_t *>(hb + o_qt), *h_mk = reinterpret_cast<int32_t *>(hb + o_mk),
          *h_h0 = reinterpret_cast<int32_t *>(hb + o_h0);
  for (size_t t = 0; t < T; ++t) {
    hb[o_valid + t] = mask[t] ? 1 : 0;
    hb[o_need + t] = pidx[t] >= 0 ? 1 : 0;
    if (pidx[t] >= 0) {
      h_ids[pidx[t]] = (int32_t)ids[t];
      h_cols[pidx[t]] = (int32_t)t;
      h_qt[pidx[t]] = (int32_t)qtype[t / L];
    }
  }
  for (size_t j = 0; j < KB; ++j) {
    h_mk[j] = pidx[(size_t)(marker_pos[j] < 0 ? 0 : marker_pos[j]) + L * (j / K)];
    hb[o_mm + j] = marker_mask[j] ? 1 : 0;
  }
  for (size_t b = 0; b < B; ++b) h_h0[b] = pidx[L * b];

  // Device workspace: the packed inputs, then float activations (packed
  // unless named _f, the padded layout of the attention op).
  const size_t xp = d * Tc;
  const size_t nf = 2 * xp + wide * Tc + I * Tc + 3 * xp + xp + 3 * xs + xs + 2 * d * KB + KB +
                    (d + 4) * B + AH * B + A * B + KB + 16 * 64;
  if ((rc = reserve(c, c->model, up(host_bytes) + sizeof(float) * nf + 1024))) return rc;
  uint8_t *db = static_cast<uint8_t *>(c->model.ptr);
  TFD_HIP(c, hipMemcpyAsync(db, hb, host_bytes, hipMemcpyHostToDevice, c->stream),
          "hipMemcpyAsync");
  const int *d_ids = reinterpret_cast<const int *>(db);
  const int *d_cols = reinterpret_cast<const int *>(db + o_cols);
  const int *d_qt = reinterpret_cast<const int *>(db + o_qt);
  const int *d_mk = reinterpret_cast<const int *>(db + o_mk);
  const int *d_h0 = reinterpret_cast<const int *>(db + o_h0);
  const uint8_t *d_valid = db + o_valid, *d_mm = db + o_mm, *d_need = db + o_need;
  float *fp = reinterpret_cast<float *>(db + up(host_bytes));
  auto take = [&](size_t n) {
    float *p = fp;
    fp += (n + 63) & ~(size_t)63;
    return p;
  };
  float *x = take(xp), *a = take(xp), *u = take(wide * Tc), *g = take(I * Tc),
        *qkv_p = take(3 * xp), *att_p = take(xp), *qkv_f = take(3 * xs), *att_f = take(xs),
        *s0 = take(d * KB), *s1 = take(d * KB), *raw = take(KB), *pooled = take((d + 4) * B),
        *a1 = take(AH * B);
  const bool dev_out = (flags & TFD_DEVICE_PTRS) != 0;
  float *act_d = dev_out ? action : take(A * B), *log_d = dev_out ? logits : take(KB);
  // Padded columns of the attention input that no packed column fills stay 0.
  TFD_HIP(c, tfd::launch_fill_zero(qkv_f, 3 * xs, c->stream), "fill launch");

  // attention_block_host (model.rs:612-633) on the packed columns, its
  // result added into `res` (the residual stream): qkv projected for the
  // packed columns, moved into the padded (3d, L, B) layout, the fused op
  // under the structured mask (build_mask, 467-490; 64-query groups with no
  // packed column are skipped), its packed columns projected by W_out.
  auto attention = [&](const float *in, size_t heads, int64_t window, const float *w_in,
                       const float *b_in, const float *w_out, const float *b_out,
                       uint32_t rope_bits, float *res) {
    int r = linear_cols(c, w_in, b_in, d, 3 * d, in, Tc, qkv_p, tfd::kActNone);
    if (r) return r;
    TFD_HIP(c, tfd::launch_copy_columns(qkv_p, nullptr, qkv_f, d_cols, (int)(3 * d), (long)Tc,
                                        c->stream),
            "copy launch");
    if ((r = laya_run(c, op, qkv_f, nullptr, d_valid, window, d, heads, L, B, rope_bits, att_f,
                      TFD_DEVICE_PTRS | TFD_ASYNC, d_need)))
      return r;
    TFD_HIP(c, tfd::launch_copy_columns(att_f, d_cols, att_p, nullptr, (int)d, (long)Tc, c->stream),
            "copy launch");
    return linear_cols(c, w_out, b_out, d, d, att_p, Tc, res, tfd::kActNone, true);
  };

  // Encoder: x = LN(tok_embeddings[:, ids]) (model.rs:671-686).
  if ((rc = norm_cols(c, m->tok_embeddings, d_ids, (long)Tc, d, m->embed_norm_w, m->embed_norm_b,
                      eps, x)))
    return rc;
  for (size_t i = 0; i < m->n_layers; ++i) {
    const tfd_laya_encoder_layer &l = m->layers[i];
    const float *ain = x;
    if (l.attn_norm_w) {
      if ((rc = norm_cols(c, x, nullptr, (long)Tc, d, l.attn_norm_w, l.attn_norm_b, eps, a)))
        return rc;
      ain = a;
    }
    // z = x + attention_block(attn_input) (model.rs:693-704)
    if ((rc = attention(ain, m->heads, l.sliding ? (int64_t)m->window : -1, l.wqkv, l.bqkv, l.wo,
                        l.bo, l.rope_base_bits, x)))
      return rc;
    // z += Wo_mlp^T geglu(Wi^T LN(z)) (model.rs:706-710)
    if ((rc = norm_cols(c, x, nullptr, (long)Tc, d, l.mlp_norm_w, l.mlp_norm_b, eps, a))) return rc;
    if ((rc = gemm(c, true, false, 2 * I, Tc, d, l.wi, d, 0, a, d, 0, u, 2 * I, 0, 1))) return rc;
    TFD_HIP(c, tfd::launch_geglu(u, l.bi, (int)I, Tc, g, c->stream), "geglu launch");
    if ((rc = linear_cols(c, l.wo_mlp, l.bo_mlp, I, d, g, Tc, x, tfd::kActNone, true))) return rc;
  }
  // h = final_norm(x) + type_emb[:, qtype[b]] (model.rs:706-712, 916-931)
  float *h = a, *n = x;
  if ((rc = norm_cols(c, x, nullptr, (long)Tc, d, m->final_norm_w, m->final_norm_b, eps, h,
                      m->type_emb, d_qt, 1)))
    return rc;
  // Head layers, full attention without RoPE (model.rs:715-747, 932-935).
  for (size_t i = 0; i < m->n_head_layers; ++i) {
    const tfd_laya_head_layer &hl = m->head[i];
    if ((rc = norm_cols(c, h, nullptr, (long)Tc, d, hl.norm1_w, hl.norm1_b, eps, n))) return rc;
    if ((rc = attention(n, hl.heads, -1, hl.in_proj_w, hl.in_proj_b, hl.out_proj_w, hl.out_proj_b,
                        0u, h)))
      return rc;
    if ((rc = norm_cols(c, h, nullptr, (long)Tc, d, hl.norm2_w, hl.norm2_b, eps, n))) return rc;
    if ((rc = linear_cols(c, hl.linear1_w, hl.linear1_b, d, hl.ff, n, Tc, u, tfd::kActRelu)))
      return rc;
    if ((rc = linear_cols(c, hl.linear2_w, hl.linear2_b, hl.ff, d, u, Tc, h, tfd::kActNone, true)))
      return rc;
  }
  // Marker scorer: LN of the gathered columns, linear + GELU, linear to one
  // logit per marker (model.rs:937-941).
  if ((rc = norm_cols(c, h, d_mk, (long)KB, d, m->scorer_norm_w, m->scorer_norm_b, eps, s0)))
    return rc;
  if ((rc = linear_cols(c, m->scorer1_w, m->scorer1_b, d, d, s0, KB, s1, tfd::kActGelu))) return rc;
  if ((rc = linear_cols(c, m->scorer2_w, m->scorer2_b, d, 1, s1, KB, raw, tfd::kActNone))) return rc;
  tfd::PoolArgs pa{};
  pa.raw = raw;
  pa.marker_mask = d_mm;
  pa.h = h;
  pa.h0_col = d_h0;
  pa.logits = log_d;
  pa.pooled = pooled;
  pa.k = (int)K;
  pa.d = (int)d;
  pa.L = (int)L;
  TFD_HIP(c, tfd::launch_pool(pa, (int)B, c->stream), "pool launch");
  // Action head (model.rs:954-966).
  if ((rc = linear_cols(c, m->act1_w, m->act1_b, d + 4, AH, pooled, B, a1, tfd::kActGelu)))
    return rc;
  if ((rc = linear_cols(c, m->act2_w, m->act2_b, AH, A, a1, B, act_d, tfd::kActNone))) return rc;
  if (dev_out) {
    if (flags & TFD_ASYNC) {
      c->model_inflight = true;
      return TFD_OK;
    }
    TFD_HIP(c, hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    return TFD_OK;
  }
  TFD_HIP(c, hipMemcpyAsync(logits, log_d, sizeof(float) * KB, hipMemcpyDeviceToHost, c->stream),
          "hipMemcpyAsync");
  TFD_HIP(c, hipMemcpyAsync(action, act_d, sizeof(float) * A * B, hipMemcpyDeviceToHost, c->stream),
          "hipMemcpyAsync");
  TFD_HIP(c, hipStreamSynchronize(c->stream), "hipStreamSynchronize");
  return TFD_OK;
}

}  // namespace

// ---------------------------------------------------------------- C ABI

extern "C" {

int tfd_abi_version(void) { return TFD_ABI_VERSION; }

const char *tfd_laya_attention_block_family_id(void) { return kLayaFamily; }
const char *tfd_jeff_full_attention_family_id(void) { return kJeffFamily; }

int tfd_ctx_create(int device, tfd_ctx **out) {
  if (!out) return TFD_EINVAL;
  *out = new (std::nothrow) tfd_ctx();
  if (!*out) return TFD_EHIP;
  (*out)->device = device;
  return TFD_OK;
}

int tfd_ctx_create_on_stream(int device, void *stream, tfd_ctx **out) {
  int rc = tfd_ctx_create(device, out);
  if (rc) return rc;
  (*out)->stream = static_cast<hipStream_t>(stream);
  (*out)->adopted = true;
  return TFD_OK;
}

void tfd_ctx_destroy(tfd_ctx *c) {
  if (!c) return;
  if (c->ready) {
    (void)hipSetDevice(c->device);
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    for (auto &b : c->staging)
      if (b.ptr) (void)hipFree(b.ptr);
    if (c->bits.ptr) (void)hipFree(c->bits.ptr);
    if (c->kp.ptr) (void)hipFree(c->kp.ptr);
    if (c->layer.ptr) (void)hipFree(c->layer.ptr);
    if (c->model.ptr) (void)hipFree(c->model.ptr);
    if (c->blas) (void)rocblas_destroy_handle(c->blas);
    for (auto &e : c->rope) {
      (void)hipFree(e.cos_d);
      (void)hipFree(e.sin_d);
    }
    for (auto &e : c->events) (void)hipEventDestroy(e);
    if (c->own_stream) (void)hipStreamDestroy(c->stream);
  }
  delete c;
}

const char *tfd_last_error(const tfd_ctx *c) { return c ? c->err.c_str() : "null context"; }

int tfd_ctx_synchronize(tfd_ctx *c) {
  if (!c) return TFD_EINVAL;
  if (!c->ready) return TFD_OK;
  TFD_HIP(c, hipSetDevice(c->device), "hipSetDevice");
  TFD_HIP(c, hipStreamSynchronize(c->stream), "hipStreamSynchronize");
  return TFD_OK;
}

void *tfd_ctx_stream(tfd_ctx *c) {
  if (!c) return nullptr;
  if (!c->ready && ensure_ready(c) != TFD_OK) return nullptr;
  return c->stream;
}

size_t tfd_ctx_retained_bytes(const tfd_ctx *c) {
  if (!c) return 0;
  size_t total = sizeof(tfd_ctx) + c->bits.cap + c->kp.cap + c->layer.cap + c->model.cap +
                 c->model_host.capacity();
  for (const auto &b : c->staging) total += b.cap;
  for (const auto &e : c->rope) total += e.bytes;
  return total;
}

int tfd_ctx_set_timing(tfd_ctx *c, int enabled) {
  if (!c) return TFD_EINVAL;
  c->timing = enabled != 0;
  return TFD_OK;
}

int tfd_ctx_take_kernel_time(tfd_ctx *c, double *total_ms, uint64_t *launches) {
  if (!c) return TFD_EINVAL;
  double total = 0.0;
  const uint64_t n = c->events_used;
  if (n) {
    TFD_HIP(c, hipSetDevice(c->device), "hipSetDevice");
    TFD_HIP(c, hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    for (size_t i = 0; i < n; ++i) {
      float ms = 0.0f;
      TFD_HIP(c, hipEventElapsedTime(&ms, c->events[2 * i], c->events[2 * i + 1]),
              "hipEventElapsedTime");
      total += ms;
    }
  }
  c->events_used = 0;
  if (total_ms) *total_ms = total;
  if (launches) *launches = n;
  return TFD_OK;
}

}  // extern "C"

namespace {

// execute_laya_attention_block_in_session's checks (laya_attention.rs:99-176)
// and the run, shared by the drop-in and its no-allocation variant.
int laya_block(tfd_ctx *c, const char *op, const float *qkv, const size_t *qkv_shape,
               size_t qkv_rank, size_t qkv_len, const uint8_t *keep, size_t keep_len,
               size_t hidden, size_t heads, uint32_t rope_base_bits, float *out, size_t out_len,
               unsigned flags, bool noalloc) {
  if (!c) return TFD_EINVAL;
  c->err.clear();
  int rc = check_flags(c, op, flags, TFD_DEVICE_PTRS | TFD_ASYNC);
  if (rc) return rc;
  if (noalloc && !(flags & TFD_DEVICE_PTRS))
    return invalid(c, op, "flags", "this entry takes device pointers only (TFD_DEVICE_PTRS)");
  // laya_attention.rs:111-114 (and infer_output_meta 80-83)
  if (qkv_shape == nullptr || qkv_rank != 3 || hidden > SIZE_MAX / 3 ||
      qkv_shape[0] != 3 * hidden)
    return invalid(c, op, "shape", "attention block expects (3d, L, B)");
  const size_t length = qkv_shape[1], batch = qkv_shape[2];
  size_t expect = 0;
  // cpu-kernels lib.rs:855-864: a slice shorter (or longer) than the shape
  // says is rejected before any access ("qkv length").
  if (!mul_ok(qkv_shape[0], length, &expect) || !mul_ok(expect, batch, &expect) ||
      qkv_len != expect)
    return invalid(c, op, "qkv", "qkv length");
  // laya_attention.rs:138-140
  if (!mul_ok(length, length, &expect) || !mul_ok(expect, batch, &expect) || keep_len != expect)
    return invalid(c, op, "keep", "keep must be (L, L, B)");
  if (!mul_ok(hidden, length, &expect) || !mul_ok(expect, batch, &expect) || out_len != expect)
    return invalid(c, op, "out", "out must be (d, L, B)");
  if (expect != 0 && (!qkv || !out || (keep_len && !keep)))
    return invalid(c, op, "inputs", "null buffer");
  return laya_run(c, op, qkv, keep, nullptr, -1, hidden, heads, length, batch, rope_base_bits,
                  out, flags, nullptr, noalloc);
}

}  // namespace

extern "C" {

int tfd_laya_attention_block_f32(tfd_ctx *c, const float *qkv, const size_t *qkv_shape,
                                 size_t qkv_rank, size_t qkv_len, const uint8_t *keep,
                                 size_t keep_len, size_t hidden, size_t heads,
                                 uint32_t rope_base_bits, float *out, size_t out_len,
                                 unsigned flags) {
  return laya_block(c, kLayaOp, qkv, qkv_shape, qkv_rank, qkv_len, keep, keep_len, hidden, heads,
                    rope_base_bits, out, out_len, flags, false);
}

int tfd_laya_attention_block_noalloc_f32(tfd_ctx *c, const float *qkv, const size_t *qkv_shape,
                                         size_t qkv_rank, size_t qkv_len, const uint8_t *keep,
                                         size_t keep_len, size_t hidden, size_t heads,
                                         uint32_t rope_base_bits, float *out, size_t out_len,
                                         unsigned flags) {
  return laya_block(c, "tfd_laya_attention_block_noalloc_f32", qkv, qkv_shape, qkv_rank, qkv_len,
                    keep, keep_len, hidden, heads, rope_base_bits, out, out_len, flags, true);
}

int tfd_laya_attention_structured_f32(tfd_ctx *c, const float *qkv, size_t hidden, size_t heads,
                                      size_t length, size_t batch, const uint8_t *valid,
                                      int64_t window, uint32_t rope_base_bits, float *out,
                                      unsigned flags) {
  const char *op = "tfd_laya_attention_structured_f32";
  if (!c) return TFD_EINVAL;
  c->err.clear();
  int rc = check_flags(c, op, flags, TFD_DEVICE_PTRS | TFD_ASYNC);
  if (rc) return rc;
  if (hidden && length && batch && (!qkv || !valid || !out))
    return invalid(c, op, "inputs", "null buffer");
  return laya_run(c, op, qkv, nullptr, valid, window, hidden, heads, length, batch,
                  rope_base_bits, out, flags);
}

int tfd_jeff_full_attention_f32(tfd_ctx *c, const float *q, const size_t *q_shape,
                                size_t q_rank, const float *k, size_t k_len, const float *v,
                                size_t v_len, const float *gate, size_t gate_len,
                                const float *q_norm, size_t q_norm_len, const float *k_norm,
                                size_t k_norm_len, const float *mask, size_t mask_len,
                                size_t heads, size_t head_dim, size_t rotary_dim,
                                uint32_t theta_bits, uint32_t eps_bits, float *out,
                                size_t out_len, unsigned flags) {
  if (!c) return TFD_EINVAL;
  c->err.clear();
  const size_t kv_groups = (flags & TFD_KV_HEADS_MASK) >> 16;  // 0: every head distinct
  flags &= ~TFD_KV_HEADS_MASK;
  int rc = check_flags(c, kJeffOp, flags, TFD_DEVICE_PTRS | TFD_ASYNC);
  if (rc) return rc;
  // jeff_attention.rs:116-125
  if (q_shape == nullptr || q_rank != 2)
    return invalid(c, kJeffOp, "shape", "full attention expects (length, width)");
  const size_t length = q_shape[0], width = q_shape[1];
  size_t hw = 0;
  if (!mul_ok(heads, head_dim, &hw) || width != hw)
    return invalid(c, kJeffOp, "shape", "width must equal heads * head_dim");
  // jeff_attention.rs:159-164
  if (q_norm_len != head_dim || k_norm_len != head_dim || mask_len != length)
    return invalid(c, kJeffOp, "shape", "q_norm/k_norm must be (head_dim) and mask (length)");
  size_t n = 0;
  if (!mul_ok(length, width, &n))
    return invalid(c, kJeffOp, "shape", "attention dimensions overflow");
  // The reference only debug-asserts these (cpu-kernels lib.rs:635-642).
  if (k_len != n || v_len != n || gate_len != n)
    return invalid(c, kJeffOp, "shape", "k/v/gate must be (length, width)");
  if (out_len != n) return invalid(c, kJeffOp, "out", "out must be (length, width)");
  if (rotary_dim > head_dim)
    return invalid(c, kJeffOp, "rotary_dim", "rotary_dim must not exceed head_dim");
  if (n != 0 && (!q || !k || !v || !gate || !q_norm || !k_norm || !mask || !out))
    return invalid(c, kJeffOp, "inputs", "null buffer");
  if (kv_groups != 0 && heads % kv_groups != 0)
    return invalid(c, kJeffOp, "flags", "TFD_KV_HEADS(kv_heads): kv_heads must divide heads");
  const size_t kvh = kv_groups ? kv_groups : heads;
  return jeff_run(c, kJeffOp, false, 1, length, heads, kvh, head_dim, rotary_dim, q, k, v, gate,
                  q_norm, k_norm, mask, theta_bits, eps_bits, out, flags, heads / kvh);
}

int tfd_jeff_full_attention_rows_f32(tfd_ctx *c, size_t rows, size_t length, size_t heads,
                                     size_t kv_heads, size_t head_dim, size_t rotary_dim,
                                     const float *q, const float *k, const float *v,
                                     const float *gate, const float *q_norm,
                                     const float *k_norm, const float *mask,
                                     uint32_t theta_bits, uint32_t eps_bits, float *out,
                                     unsigned flags) {
  return jeff_rows_common(c, false, rows, length, heads, kv_heads, head_dim, rotary_dim, q, k, v,
                          gate, q_norm, k_norm, mask, theta_bits, eps_bits, out, flags);
}

int tfd_jeff_full_attention_rows_bf16(tfd_ctx *c, size_t rows, size_t length, size_t heads,
                                      size_t kv_heads, size_t head_dim, size_t rotary_dim,
                                      const uint16_t *q, const uint16_t *k, const uint16_t *v,
                                      const uint16_t *gate, const float *q_norm,
                                      const float *k_norm, const float *mask,
                                      uint32_t theta_bits, uint32_t eps_bits, float *out,
                                      unsigned flags) {
  return jeff_rows_common(c, true, rows, length, heads, kv_heads, head_dim, rotary_dim, q, k, v,
                          gate, q_norm, k_norm, mask, theta_bits, eps_bits, out, flags);
}

int tfd_laya_attention_layer_f32(tfd_ctx *c, const float *x, size_t hidden, size_t heads,
                                 size_t length, size_t batch, const uint8_t *keep,
                                 const float *w_in, const float *b_in, const float *w_out,
                                 const float *b_out, uint32_t rope_base_bits, float *out,
                                 unsigned flags) {
  if (!c) return TFD_EINVAL;
  c->err.clear();
  int rc = check_flags(c, "tfd_laya_attention_layer_f32", flags, TFD_DEVICE_PTRS | TFD_ASYNC);
  if (rc) return rc;
  return laya_layer(c, x, hidden, heads, length, batch, keep, w_in, b_in, w_out, b_out,
                    rope_base_bits, out, flags);
}

int tfd_jeff_full_attention_layer_rows_f32(tfd_ctx *c, size_t rows, size_t length,
                                           size_t hidden, size_t heads, size_t kv_heads,
                                           size_t head_dim, size_t rotary_dim, const float *x,
                                           const float *w_q, const float *w_gate,
                                           const float *w_k, const float *w_v, const float *w_o,
                                           const float *q_norm, const float *k_norm,
                                           const float *mask, uint32_t theta_bits,
                                           uint32_t eps_bits, float *out, unsigned flags) {
  if (!c) return TFD_EINVAL;
  c->err.clear();
  int rc = check_flags(c, "tfd_jeff_full_attention_layer_rows_f32", flags,
                       TFD_DEVICE_PTRS | TFD_ASYNC | TFD_TRIM_LEADING);
  if (rc) return rc;
  return jeff_layer(c, rows, length, hidden, heads, kv_heads, head_dim, rotary_dim, x, w_q,
                    w_gate, w_k, w_v, w_o, q_norm, k_norm, mask, theta_bits, eps_bits, out, flags);
}

int tfd_laya_forward_f32(tfd_ctx *c, const tfd_laya_model *model, const int64_t *ids,
                         const uint8_t *mask, size_t length, size_t batch,
                         const int64_t *marker_pos, const uint8_t *marker_mask, size_t k_count,
                         const int64_t *qtype, float *logits, float *action, unsigned flags) {
  if (!c) return TFD_EINVAL;
  c->err.clear();
  int rc = check_flags(c, "tfd_laya_forward_f32", flags, TFD_DEVICE_PTRS | TFD_ASYNC);
  if (rc) return rc;
  return laya_forward(c, model, ids, mask, length, batch, marker_pos, marker_mask, k_count, qtype,
                      logits, action, flags);
}

}  // extern "C"
