// Internal declarations shared by the host code (tfd_host.cpp) and the gfx950
// kernels (laya_attention.hip, jeff_attention.hip). Not part of the C ABI.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace tfd {

// Keys per tile of the Laya and Jeff bf16 kernels.
constexpr int kKeyTile = 32;
constexpr int kWavesPerGroup = 4;     // 256 threads per workgroup
constexpr int kLayaWaveQueries = 16;  // Laya waves use the 16x16x4 MFMA
constexpr int kLayaGroupQueries = kLayaWaveQueries * kWavesPerGroup;
constexpr int kJeffWaveQueries = 16;  // Jeff waves use the 16x16x4 MFMA
constexpr int kJeffF32Waves = 8;      // Jeff f32 workgroup: 512 threads, one per CU
constexpr int kJeffKeyTile = 16;      // keys per Jeff f32 tile

// Bytes per 64-query group in the Laya tile map: nkt flags rounded up to
// whole 64-byte scalar loads.
__host__ __device__ constexpr int laya_map_row(int nkt) { return (nkt + 63) & ~63; }

// Laya workgroups per CU (launch bounds): four at padded head dims up to 64,
// two at 128.
__host__ __device__ constexpr int laya_groups_per_cu(int hd_pad) { return hd_pad <= 64 ? 4 : 2; }

// Teams of four waves per Laya workgroup when the grid has at most one
// workgroup per CU: as many as the teams' double-buffered K/V tiles fit in a
// CU's LDS (four at padded head dims up to 64, two at 128).
__host__ __device__ constexpr int laya_teams(int hd_pad) { return hd_pad <= 64 ? 4 : 2; }

// Whether a Laya grid of nqb x H x B workgroups gets the XCD-aware layout:
// the whole grid fits in one dispatch round (workgroup p then runs on XCD
// p % 8 and CU slot p % cus) and each of the 8 XCDs can take an equal share
// of every batch row, three (or S) workgroups per CU from different rows.
__host__ __device__ constexpr bool laya_xcd_layout(int nqb, int H, int B, int groups_per_cu,
                                                    int cus) {
  return cus > 0 && nqb * H * B <= groups_per_cu * cus && (H * nqb) % 8 == 0 && 32 % B == 0 &&
         ((H * nqb) / 8) % (32 / B) == 0;
}

// Most (batch row, 64-query group) spans a Laya placement plan tabulates in
// LDS.
constexpr int kLayaPlanMax = 1024;

enum LayaMaskMode : int {
  kMaskBits = 0,    // general (L, L, B) keep tensor, pre-packed into 32-key words
  kMaskStruct = 1,  // valid (L, B) + window (build_mask semantics)
  kMaskRaw = 2,     // the (L, L, B) keep bytes themselves, packed by the attention kernel
};

// Division by a divisor fixed for a launch: floor(n / d) = umulhi(n, m) with
// m = ceil(2^32 / d), exact whenever n * d <= 2^32 (m * d = 2^32 + e with
// e < d, so n * m / 2^32 = n / d + n * e / (d * 2^32) stays below the next
// integer; Granlund and Montgomery, "Division by invariant integers using
// multiplication", 1994). m = 0 stands for d = 1. A run-time divisor
// otherwise costs a ~25-instruction sequence, which the kernels' prologues
// run on the scalar unit that a CU's waves share.
struct FastDiv {
  uint32_t d = 1, m = 0;
  static FastDiv make(uint32_t dv) {
    FastDiv f;
    f.d = dv;
    f.m = dv <= 1 ? 0u : (uint32_t)((((uint64_t)1 << 32) + dv - 1) / dv);
    return f;
  }
  __device__ __forceinline__ uint32_t div(uint32_t n) const {
    return m == 0 ? n : __umulhi(n, m);
  }
};

struct LayaArgs {
  const float *qkv;      // (3d, L, B)
  const uint32_t *bits;  // kMaskBits: word (b*nkt + kt)*L + q, bit j = key 32*kt + j kept;
                         // kMaskStruct (optional): word b*nkt + kt, bit j = key 32*kt + j valid
  const uint8_t *any;    // byte (b*ceil(L/64) + q/64)*laya_map_row(nkt) + kt: tile kt kept by
                         // any query of that 64-query group (kMaskBits; optional in
                         // kMaskStruct, where it only feeds the placement plan)
  const uint8_t *valid;  // kMaskStruct: (L, B)
  const uint8_t *qneed;  // kMaskStruct, or null: (L, B), a 64-query group with no
                         // non-zero entry is skipped (its output left unwritten)
  const uint8_t *keep;   // kMaskRaw: byte b*L*L + key*L + query, kept when non-zero
  const float *cos_t;    // (L, half) or nullptr (no RoPE)
  const float *sin_t;
  float *out;            // (d, L, B)
  int d, hd, half, L, nkt, window;
  int cus;               // compute units of the device (grid shapes)
  float c1;              // (1/sqrt(hd)) * log2(e)
  // Set by the launcher for the one-round 64-query grid (TEAMS == 1):
  // layout 0 = grid order, 1 = laya_xcd_layout, 2 = that layout with the
  // placement plan; division by ceil(L/64) and by the plan's items per
  // batch row and XCD (heads * ceil(L/64) / 8).
  int layout;
  FastDiv ngdiv, mdiv;
};

struct JeffArgs {
  const void *q, *k, *v, *gate;  // f32 or bf16 per kernel
  const float *q_norm, *k_norm;  // (hd)
  const float *mask;             // rows x (L)
  const float *cos_t, *sin_t;    // (L, rot_half) by RoPE position, or nullptr
  float *out;
  int L, heads, kv_heads, hd, rot_half, groups;
  int heads_per_group;           // query heads sharing one workgroup (1, 2 or 4)
  int trim;                      // TFD_TRIM_LEADING semantics
  int cus;                       // compute units of the device (grid shapes)
  float c1;                      // (1/sqrt(hd)) * log2(e)
  float eps;
  size_t q_row, kv_row;          // elements per row: L*heads*hd and L*kv_heads*hd (times
                                 // the copies of an expanded K/V, see kv_head)
  size_t kv_head;                // elements between consecutive kv heads of K/V: L*hd, or
                                 // L*hd*G when each of G expanded copies is skipped
  FastDiv gdiv, kvdiv, hdiv;     // by groups, kv_heads, heads (exact for n <= rows * heads)
};

// Timing of an op's attention kernel(s): `start` is recorded when the first
// of them begins executing and `stop` when the last one ends (the dispatch
// packets' own timestamps, hipExtLaunchKernel), so the pair measures the
// kernels and not the queue around them. Both null: untimed.
struct KernelEvents {
  hipEvent_t start = nullptr, stop = nullptr;
};

// Kernel launchers (return the launch status). hd_pad selects the
// compile-time padded head dim (32, 64, 128 or 256).
hipError_t launch_fill_zero(float *out, size_t n, hipStream_t stream);
// c[o + m*j] += b[o] for o < m, j < n: a column-major (m, n) matrix plus a
// per-row bias (the linears of the layer entries).
hipError_t launch_add_row_bias(float *c, const float *b, int m, size_t n, hipStream_t stream);
hipError_t launch_laya_keep_bits(const uint8_t *keep, uint32_t *bits, uint8_t *any, int L, int B,
                                 int nkt, hipStream_t stream);
// The structured mask's valid-key words (LayaArgs::bits, kMaskStruct) and,
// when `any` is given, its tile map (valid (L, B) + window; window < 0: none)
// in laya_keep_bits_kernel's `any` layout.
hipError_t launch_laya_valid_prep(const uint8_t *valid, uint32_t *words, uint8_t *any, int L,
                                  int B, int nkt, int window, hipStream_t stream);
// Whether a grid of (L, heads, batch) at padded head dim hd_pad gets the
// placement plan from a tile map (one dispatch round, laya_xcd_layout).
// Whether a Laya grid takes the teams variant of the attention kernel (at
// most one 64-query workgroup per CU, more than one key tile), and whether
// that variant packs the keep bytes itself (kMaskRaw: whole rows of 16-byte
// pieces, L % 4 == 0) instead of a packing pass.
inline bool laya_teams_grid(int L, int heads, int batch, int nkt, int cus) {
  const long groups = (long)((L + kLayaGroupQueries - 1) / kLayaGroupQueries) * heads * batch;
  return cus > 0 && nkt > 1 && groups <= cus;
}
inline bool laya_raw_keep(int L, int heads, int batch, int nkt, int cus) {
  return laya_teams_grid(L, heads, batch, nkt, cus) && L % 4 == 0 &&
         (size_t)L * (size_t)L < ((size_t)1 << 31);
}
inline bool laya_planned(int L, int heads, int batch, int hd_pad, int cus) {
  const int nqb = (L + kLayaGroupQueries - 1) / kLayaGroupQueries;
  return laya_xcd_layout(nqb, heads, batch, laya_groups_per_cu(hd_pad), cus) &&
         nqb * batch <= kLayaPlanMax;
}
hipError_t launch_laya_attention(const LayaArgs &a, int heads, int batch, int hd_pad, int mode,
                                 hipStream_t stream, const KernelEvents &ev);
// Jeff launchers run a K prep kernel into `kp` (workspace of
// jeff_kp_bytes()) and then the attention kernel.
size_t jeff_kp_bytes(const JeffArgs &a, int rows, int hd_pad, bool bf16);
hipError_t launch_jeff_attention_f32(const JeffArgs &a, int rows, int hd_pad, void *kp,
                                     hipStream_t stream, const KernelEvents &ev);
hipError_t launch_jeff_attention_bf16(const JeffArgs &a, int rows, int hd_pad, void *kp,
                                      hipStream_t stream, const KernelEvents &ev);
// The bf16 kernel at head dim 256 on the 32x32x16 matrix cores (used by
// launch_jeff_attention_bf16 when it fits): one flag per (row, head, query
// tile of jeff_bf16_wide_query_tile) marks tiles left to the exact pass.
// kbits: the rows' active key bits, written by the K prep.
bool jeff_bf16_wide_fits(const JeffArgs &a);
int jeff_bf16_wide_query_tile(const JeffArgs &a);
size_t jeff_bf16_wide_flag_count(const JeffArgs &a, int rows);
size_t jeff_bf16_flags_offset(const JeffArgs &a, int rows);
hipError_t launch_jeff_bf16_wide(const JeffArgs &a, int rows, const uint16_t *kp,
                                 const uint32_t *kbits, int *flags, hipStream_t stream);

// Head dims past the tiled kernels (Laya hd > 128, Jeff hd > 256): one
// wavefront per query in the reference's scalar order. Laya reads `keep`
// (kMaskBits) or a.valid + a.window (kMaskStruct) directly; Jeff prepares
// the keys into `kn` (jeff_generic_kn_bytes) first.
constexpr int kLayaTiledMaxHd = 128;
constexpr int kJeffTiledMaxHd = 256;
hipError_t launch_laya_generic(const LayaArgs &a, const uint8_t *keep, int heads, int batch,
                               int mode, hipStream_t stream);
inline size_t jeff_generic_kn_bytes(const JeffArgs &a, int rows) {
  return (size_t)rows * a.kv_heads * a.L * a.hd * sizeof(float);
}
hipError_t launch_jeff_generic(const JeffArgs &a, int rows, bool bf16, float *kn,
                               hipStream_t stream, const KernelEvents &ev);

// ------------------------------------------------ no-allocation entry

// Bytes of the static device scratch of tfd_laya_attention_block_noalloc_f32
// (RoPE tables, packed keep words and tile map of one call).
constexpr size_t kNoallocScratchBytes = (size_t)16 << 20;
// The scratch array's address on `device`, which must be current: looked up
// once per device (hipGetSymbolAddress) and kept; null with *err set on
// failure. Device code only ever sees this address, never the array's name.
void *noalloc_scratch(int device, hipError_t *err);

// ------------------------------------------------ Laya decision-model forward

enum Activation : int { kActNone = 0, kActRelu = 1, kActGelu = 2 };

// LayerNorm of `cols` feature columns (d features each): output column c
// reads column map ? map[c] : c of x (column stride ldx); y is (d, cols).
// add/add_col/per: optional y[:, c] += add[:, add_col[c / per]].
struct NormArgs {
  const float *x;
  const int *map;
  const float *w, *b;
  const float *add;
  const int *add_col;
  float *y;
  long cols;
  int ldx, d, per;
  float eps;
};

// Marker pooling: raw (K, B) logits, marker_mask (K, B) bytes, h the head
// output with token 0 of prompt b in column h0_col[b] (or b*L when null);
// writes the masked logits (K, B) and pooled (d + 4, B).
struct PoolArgs {
  const float *raw;
  const uint8_t *marker_mask;
  const float *h;
  const int *h0_col;
  float *logits, *pooled;
  int k, d, L;
};

hipError_t launch_norm_columns(const NormArgs &a, hipStream_t stream);
// y[o + m*j] = act(y[o + m*j] + b[o]) for o < m, j < n (b may be null).
hipError_t launch_bias_act(float *y, const float *b, int m, size_t n, int act,
                           hipStream_t stream);
// g (I, cols) = gelu(u[:I] + b[:I]) * (u[I:] + b[I:]) per column of u (2I, cols).
hipError_t launch_geglu(const float *u, const float *b, int inter, size_t cols, float *g,
                        hipStream_t stream);
hipError_t launch_pool(const PoolArgs &a, int batch, hipStream_t stream);
// dst[:, dst_map ? dst_map[j] : j] = src[:, src_map ? src_map[j] : j], j < n,
// m floats per column.
hipError_t launch_copy_columns(const float *src, const int *src_map, float *dst,
                               const int *dst_map, int m, long n, hipStream_t stream);

}  // namespace tfd
