/*
 * tfd_attention.h -- C ABI of the MI355X (gfx950) fused attention ops.
 *
 * Two drop-in ops replace the reference's CPU extension ops:
 *
 *   tfd_laya_attention_block_f32   <- LayaAttentionBlockOp::execute_in_session
 *        crates/tenferro-ext/src/laya_attention.rs:99-176
 *        (eager entry EagerSessionLayaAttentionExt::laya_attention_block, 206-249)
 *   tfd_jeff_full_attention_f32    <- JeffFullAttentionOp::execute_in_session
 *        crates/tenferro-ext/src/jeff_attention.rs:103-184
 *        (eager entry EagerSessionJeffAttentionExt::jeff_full_attention, 214-275)
 *
 * plus entries that extend the same arithmetic without changing the drop-in
 * path (structured Laya masks, batched Jeff rows with native GQA, bf16 Jeff).
 *
 * Conventions
 *   - Every tensor is column-major exactly as the reference passes it:
 *       Laya qkv  (3d, L, B): element f + 3d*(l + L*b); q at f < d, k at d+f,
 *                 v at 2d+f; head h owns f = h*hd + i.
 *       Laya keep (L, L, B) one byte per entry, query + L*(key + L*b), non-zero
 *                 keeps the key (Rust `bool`).
 *       Laya out  (d, L, B).
 *       Jeff q/k/v/gate/out (L, W): element t + L*f, f = h*hd + i.
 *       Jeff mask (L) f32: a key is active when mask != 0.
 *   - Parameters that the reference stores as f32 bits (rope_base_bits,
 *     theta_bits, eps_bits) are passed as those bits.
 *   - The caller owns every buffer, including `out`.
 *   - A context owns one HIP stream, the RoPE table cache and a growable
 *     device workspace. Use one context per host thread.
 *   - Arguments are validated before any device access. Errors return a
 *     non-zero status; tfd_last_error() gives the message.
 *   - There is no CPU fallback: a missing or unusable GPU returns TFD_EHIP.
 */
#ifndef TFD_ATTENTION_H
#define TFD_ATTENTION_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TFD_ABI_VERSION 2

/* status codes */
#define TFD_OK 0
#define TFD_EINVAL 1       /* invalid argument; message mirrors the reference */
#define TFD_EUNSUPPORTED 2 /* valid but outside what the kernels implement */
#define TFD_EHIP 3         /* HIP runtime error (no device, launch failure) */

/* flags */
#define TFD_HOST_PTRS 0u   /* operands are host memory: upload, run, download, sync */
#define TFD_DEVICE_PTRS 1u /* operands are device memory of the context's device */
#define TFD_ASYNC 2u       /* with TFD_DEVICE_PTRS: enqueue on the context stream and return */
#define TFD_TRIM_LEADING 4u /* Jeff rows: drop each row's leading inactive keys and
                               restart RoPE positions at the first active one */
/* Jeff drop-in on GQA-expanded K/V: the caller states kv_heads (bits 16..31),
 * heads / kv_heads consecutive heads of K and V being identical copies, as
 * jeff-infer's checkpoint expansion makes them (checkpoint.rs:307-319; the
 * reference's raw CUDA path recovers the same grouping from the weights,
 * dedupe_kv, cuda_raw.rs:243-279). The op then reads only the first head of
 * each group. 0 (the default) treats every head as distinct. */
#define TFD_KV_HEADS(kv_heads) ((((unsigned)(kv_heads)) & 0xffffu) << 16)
#define TFD_KV_HEADS_MASK 0xffff0000u

typedef struct tfd_ctx tfd_ctx;

/* ABI version compiled into the library (TFD_ABI_VERSION). */
int tfd_abi_version(void);

/* Stable family ids of the two ops:
 * laya_attention.rs:25 "tenferro-decision.laya_attention_block.v1",
 * jeff_attention.rs:24 "tenferro-decision.jeff_full_attention.v1". */
const char *tfd_laya_attention_block_family_id(void);
const char *tfd_jeff_full_attention_family_id(void);

/* Context life cycle. Creation does not touch the GPU; the first op call
 * selects `device` and creates the stream (or adopts `stream`, a hipStream_t
 * the caller keeps alive; NULL adopts the null stream). The reference keeps the matching per-op state in
 * the runtime's ExtensionCacheStore (laya_attention.rs:142-159). */
int tfd_ctx_create(int device, tfd_ctx **out);
int tfd_ctx_create_on_stream(int device, void *stream, tfd_ctx **out);
void tfd_ctx_destroy(tfd_ctx *ctx);
const char *tfd_last_error(const tfd_ctx *ctx);
int tfd_ctx_synchronize(tfd_ctx *ctx);
void *tfd_ctx_stream(tfd_ctx *ctx);
/* Device and host bytes the context retains between calls; mirrors
 * LayaAttentionWorkspace::retained_bytes (cpu-kernels lib.rs:784-806). */
size_t tfd_ctx_retained_bytes(const tfd_ctx *ctx);

/* Kernel timing, a profiling aid with no counterpart in the reference (its
 * closest is raw_exec::take_drain_stats, crates/tenferro-ext/src/raw_exec.rs:781).
 * While enabled, every call's attention kernel(s) carry a HIP event pair that
 * their own dispatches record (hipExtLaunchKernel): the start when the first
 * of them begins executing, the stop when the last one ends (Jeff: K prep
 * and attention; never uploads or the keep packing).
 * take() synchronizes the stream and returns, then resets, the summed
 * duration in milliseconds and the number of timed launches. */
int tfd_ctx_set_timing(tfd_ctx *ctx, int enabled);
int tfd_ctx_take_kernel_time(tfd_ctx *ctx, double *total_ms, uint64_t *launches);

/*
 * Laya fused split + RoPE + masked attention (drop-in).
 * Reference: execute_laya_attention_block_in_session, laya_attention.rs:99-176,
 * arithmetic cpu-kernels lib.rs:843-1156.
 *   qkv_shape/qkv_rank: the qkv tensor's shape; must be (3*hidden, L, B).
 *   qkv_len:            elements of qkv storage; must be 3*hidden*L*B, else
 *                       "qkv length" (the reference's assert_eq!, cpu-kernels
 *                       lib.rs:864, test lib.rs:1205-1210), before any access.
 *   keep_len:           must be L*L*B.
 *   out_len:            must be hidden*L*B.
 *   rope_base_bits:     f32 bits of the RoPE base; 0.0 disables RoPE.
 * heads == 0 or hidden % heads != 0 writes zeros, as the reference does.
 * A query that keeps no key yields NaN, as the reference does.
 */
int tfd_laya_attention_block_f32(tfd_ctx *ctx, const float *qkv, const size_t *qkv_shape,
                                 size_t qkv_rank, size_t qkv_len, const uint8_t *keep,
                                 size_t keep_len,
                                 size_t hidden, size_t heads, uint32_t rope_base_bits,
                                 float *out, size_t out_len, unsigned flags);

/*
 * The Laya drop-in without any allocation (no counterpart in the reference:
 * an entry for callers that cannot allocate device memory -- tight serving
 * loops, harnesses that forbid hipMalloc, code under HIP graph capture).
 * Same arguments, checks and results as tfd_laya_attention_block_f32, but:
 *   - operands must be device pointers (TFD_DEVICE_PTRS; TFD_ASYNC allowed);
 *   - its workspace lives in one static 16 MiB device array per GPU, held
 *     until the process ends: a 4 MiB region for the RoPE tables (L*hd/2 <=
 *     2^19), then the packed keep words and tile map, 4*L*B*ceil(L/32)
 *     bytes plus a small map, which must fit the other 12 MiB (L 2048, B 8:
 *     4 MiB); a call that needs more returns TFD_EUNSUPPORTED before any
 *     device access;
 *   - no timing events are recorded (tfd_ctx_set_timing is ignored).
 * Every call on a GPU shares that GPU's array: calls that overlap on one GPU
 * (several threads or streams) race. A context made by tfd_ctx_create creates
 * its stream on first use; tfd_ctx_create_on_stream adopts the caller's.
 * The RoPE table of the last (L, hd, rope_base) used on a GPU stays resident;
 * a call with another one uploads its table from the host and synchronizes
 * the stream. Under stream capture: pass TFD_ASYNC (else TFD_EINVAL), and make
 * one eager call with the same (L, hd, rope_base) first (else
 * TFD_EUNSUPPORTED: the upload cannot be captured). The captured kernels read
 * whichever table is resident when the graph is launched, so replays must not
 * interleave with calls of another (L, hd, rope_base) on that GPU; calls with
 * rope_base 0 leave the table in place.
 */
int tfd_laya_attention_block_noalloc_f32(tfd_ctx *ctx, const float *qkv, const size_t *qkv_shape,
                                         size_t qkv_rank, size_t qkv_len, const uint8_t *keep,
                                         size_t keep_len, size_t hidden, size_t heads,
                                         uint32_t rope_base_bits, float *out, size_t out_len,
                                         unsigned flags);

/*
 * Laya with a structured mask instead of the (L, L, B) keep tensor: the keep
 * tensor is the one build_mask (laya-infer model.rs:465-490) makes from
 * valid (L, B) (one byte per token, l + L*b) and window:
 *   keep[q,k,b] = valid[k,b] && (window < 0 || |q-k| <= window || !valid[q,b]).
 * window < 0 is FullAttention; the engine passes local_attention / 2.
 * Same results as tfd_laya_attention_block_f32 on that keep tensor.
 */
int tfd_laya_attention_structured_f32(tfd_ctx *ctx, const float *qkv, size_t hidden,
                                      size_t heads, size_t length, size_t batch,
                                      const uint8_t *valid, int64_t window,
                                      uint32_t rope_base_bits, float *out, unsigned flags);

/*
 * Jeff fused q/k RMSNorm + partial RoPE + causal masked attention + sigmoid
 * gate (drop-in).
 * Reference: execute_jeff_full_attention_in_session, jeff_attention.rs:103-184,
 * arithmetic cpu-kernels lib.rs:609-763.
 *   q_shape/q_rank: q's shape; must be (length, width) with width = heads*head_dim.
 *   k_len, v_len, gate_len, out_len: must be length*width (the reference only
 *       debug-asserts these; the ABI checks them).
 *   q_norm_len, k_norm_len: must be head_dim; mask_len: must be length.
 * A query with no active key at or before it yields 0 (times the gate).
 * flags may carry TFD_KV_HEADS(kv_heads) for expanded GQA K/V (see above):
 * same results, 1/(heads/kv_heads) of the K/V reads.
 */
int tfd_jeff_full_attention_f32(tfd_ctx *ctx, const float *q, const size_t *q_shape,
                                size_t q_rank, const float *k, size_t k_len, const float *v,
                                size_t v_len, const float *gate, size_t gate_len,
                                const float *q_norm, size_t q_norm_len, const float *k_norm,
                                size_t k_norm_len, const float *mask, size_t mask_len,
                                size_t heads, size_t head_dim, size_t rotary_dim,
                                uint32_t theta_bits, uint32_t eps_bits, float *out,
                                size_t out_len, unsigned flags);

/*
 * Jeff over `rows` independent rows in one launch, with native GQA.
 *   q, gate, out: rows x (length, heads*head_dim), row r at r*length*heads*head_dim.
 *   k, v:         rows x (length, kv_heads*head_dim); query head h reads kv head
 *                 min(h / (heads/kv_heads), kv_heads-1) (jeff-infer checkpoint.rs:307-319).
 *   mask:         rows x (length).
 * kv_heads == heads with K/V passed per head gives tfd_jeff_full_attention_f32
 * row by row. With TFD_TRIM_LEADING each row behaves as the engine's
 * row_logits trim (jeff-infer engine.rs:317-329): keys before the row's first
 * active key are dropped, RoPE positions start at 0 there, and the dropped
 * query positions are written as 0.
 */
int tfd_jeff_full_attention_rows_f32(tfd_ctx *ctx, size_t rows, size_t length, size_t heads,
                                     size_t kv_heads, size_t head_dim, size_t rotary_dim,
                                     const float *q, const float *k, const float *v,
                                     const float *gate, const float *q_norm,
                                     const float *k_norm, const float *mask,
                                     uint32_t theta_bits, uint32_t eps_bits, float *out,
                                     unsigned flags);

/* As tfd_jeff_full_attention_rows_f32 with q, k, v and gate given as bf16
 * bits (round-to-nearest-even of f32); norms, mask and out stay f32.
 * Products run on bf16 MFMA with f32 accumulation. */
int tfd_jeff_full_attention_rows_bf16(tfd_ctx *ctx, size_t rows, size_t length, size_t heads,
                                      size_t kv_heads, size_t head_dim, size_t rotary_dim,
                                      const uint16_t *q, const uint16_t *k, const uint16_t *v,
                                      const uint16_t *gate, const float *q_norm,
                                      const float *k_norm, const float *mask,
                                      uint32_t theta_bits, uint32_t eps_bits, float *out,
                                      unsigned flags);

/*
 * A whole Laya attention layer on the GPU: in_proj, the fused split + RoPE +
 * attention op and out_proj, as attention_block_tenferro runs them on the
 * f32 CPU path (laya-infer model.rs:1304-1347, linears by
 * linear_feature_first, model.rs:1179-1216):
 *   qkv      = W_in^T x (+ b_in)            (3*hidden, L, B)
 *   attended = laya_attention_block(qkv, keep, hidden, heads, rope_base)
 *   out      = W_out^T attended (+ b_out)   (hidden, L, B)
 *   x, out: (hidden, L, B) feature-first, element f + hidden*(l + L*b).
 *   w_in:   (hidden, 3*hidden) column-major, element i + hidden*o; b_in (3*hidden) or NULL.
 *   w_out:  (hidden, hidden) column-major; b_out (hidden) or NULL.
 *   keep:   (L, L, B) bytes as for tfd_laya_attention_block_f32.
 * The linears run as f32 GEMMs (rocBLAS) on the context's stream; the
 * intermediates live in the context's workspace.
 */
int tfd_laya_attention_layer_f32(tfd_ctx *ctx, const float *x, size_t hidden, size_t heads,
                                 size_t length, size_t batch, const uint8_t *keep,
                                 const float *w_in, const float *b_in, const float *w_out,
                                 const float *b_out, uint32_t rope_base_bits, float *out,
                                 unsigned flags);

/*
 * A whole Jeff full-attention layer over `rows` rows: the q, gate, k and v
 * projections, the fused attention op (with native GQA) and o_proj, as
 * full_attention_tenferro runs them on the f32 CPU path (jeff-infer
 * model.rs:686-780, linears y = x W by linear_tenferro, model.rs:289-317):
 *   q = x W_q, gate = x W_gate    (L, heads*head_dim)
 *   k = x W_k, v = x W_v          (L, kv_heads*head_dim)
 *   merged = the tfd_jeff_full_attention_rows_f32 op on them
 *   out = merged W_o              (L, hidden)
 *   x, out:       rows x (L, hidden), token-contiguous (t + L*i), row r at r*L*hidden.
 *   w_q, w_gate:  (hidden, heads*head_dim) column-major, element i + hidden*o.
 *   w_k, w_v:     (hidden, kv_heads*head_dim) column-major.
 *   w_o:          (heads*head_dim, hidden) column-major.
 *   q_norm, k_norm (head_dim), mask rows x (L): as for the rows op.
 * The linears run as f32 GEMMs (rocBLAS) on the context's stream.
 */
int tfd_jeff_full_attention_layer_rows_f32(tfd_ctx *ctx, size_t rows, size_t length,
                                           size_t hidden, size_t heads, size_t kv_heads,
                                           size_t head_dim, size_t rotary_dim, const float *x,
                                           const float *w_q, const float *w_gate,
                                           const float *w_k, const float *w_v, const float *w_o,
                                           const float *q_norm, const float *k_norm,
                                           const float *mask, uint32_t theta_bits,
                                           uint32_t eps_bits, float *out, unsigned flags);

#ifdef __cplusplus
}
#endif

#endif /* TFD_ATTENTION_H */
