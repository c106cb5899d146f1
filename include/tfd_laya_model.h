/*
 * tfd_laya_model.h -- C ABI of the Laya decision-model forward on the GPU.
 *
 *   tfd_laya_forward_f32  <- laya_infer::model::forward_reference
 *        crates/laya-infer/src/model.rs:867-977 (encoder 646-713, head layer
 *        715-747, markers 749-771, pooling 773-837), the forward that
 *        crates/laya-infer/tests/native_fixture.rs:75-139 checks against
 *        fixtures/laya-tiny/reference.json.
 *
 * Every linear runs as an f32 GEMM (rocBLAS), every attention block through
 * the fused split + RoPE + attention op of tfd_attention.h (structured
 * masks, build_mask semantics, model.rs:467-490), LayerNorm / GeGLU /
 * activations / pooling in small HIP kernels, all on the context's stream.
 *
 * Layout: activations are feature-first (d, L, B) as in the reference. A
 * linear's weight is (in, out) column-major, element i + in*o (the
 * safetensors (out, in) row-major bytes unchanged, checkpoint.rs:9-18), its
 * bias (out) or NULL. LayerNorm weights (d), bias (d) or NULL.
 *
 * All weight pointers are DEVICE memory of the context's device (the model
 * stays resident). The token inputs (ids, mask, marker_pos, marker_mask,
 * qtype) are HOST arrays, validated on the host as the reference does.
 * logits and action are host memory, or device memory with TFD_DEVICE_PTRS
 * (TFD_ASYNC then enqueues without synchronizing).
 */
#ifndef TFD_LAYA_MODEL_H
#define TFD_LAYA_MODEL_H

#include "tfd_attention.h"

#ifdef __cplusplus
extern "C" {
#endif

/* One ModernBERT encoder layer (EncoderLayerWeights, model.rs:66-89). */
typedef struct tfd_laya_encoder_layer {
  int sliding;                 /* 0: FullAttention, 1: SlidingAttention */
  uint32_t rope_base_bits;     /* f32 bits of the layer's RoPE base */
  const float *attn_norm_w;    /* (d) or NULL: identity (the first layer) */
  const float *attn_norm_b;    /* (d) or NULL */
  const float *wqkv, *bqkv;    /* (d, 3d), (3d) or NULL */
  const float *wo, *bo;        /* (d, d), (d) or NULL */
  const float *mlp_norm_w, *mlp_norm_b;
  const float *wi, *bi;        /* (d, 2*intermediate), (2*intermediate) or NULL */
  const float *wo_mlp, *bo_mlp;/* (intermediate, d), (d) or NULL */
} tfd_laya_encoder_layer;

/* One decision-head transformer layer (HeadLayerWeights, model.rs:102-121). */
typedef struct tfd_laya_head_layer {
  size_t heads;                /* max(1, d / 64) in the reference (checkpoint.rs:284-291) */
  size_t ff;                   /* linear1 width (4d) */
  const float *norm1_w, *norm1_b;
  const float *in_proj_w, *in_proj_b;   /* (d, 3d), (3d) */
  const float *out_proj_w, *out_proj_b; /* (d, d), (d) */
  const float *norm2_w, *norm2_b;
  const float *linear1_w, *linear1_b;   /* (d, ff), (ff) */
  const float *linear2_w, *linear2_b;   /* (ff, d), (d) */
} tfd_laya_head_layer;

/* The whole model (LayaWeights + the config fields the forward reads). */
typedef struct tfd_laya_model {
  size_t hidden, heads, intermediate, vocab;
  size_t window;               /* local_attention / 2 (build_mask, model.rs:474) */
  uint32_t eps_bits;           /* f32 bits of norm_eps */
  size_t n_layers, n_head_layers;
  size_t action_hidden, actions;
  const float *tok_embeddings; /* (d, vocab) */
  const float *embed_norm_w, *embed_norm_b;
  const tfd_laya_encoder_layer *layers;   /* host array of n_layers */
  const float *final_norm_w, *final_norm_b;
  const tfd_laya_head_layer *head;        /* host array of n_head_layers */
  const float *type_emb;       /* (d, 3) */
  const float *scorer_norm_w, *scorer_norm_b;
  const float *scorer1_w, *scorer1_b;     /* (d, d), (d) */
  const float *scorer2_w, *scorer2_b;     /* (d, 1), (1) */
  const float *act1_w, *act1_b;           /* (d + 4, action_hidden), (action_hidden) */
  const float *act2_w, *act2_b;           /* (action_hidden, actions), (actions) */
} tfd_laya_model;

/*
 * forward_reference (model.rs:867-977) over a batch of `batch` prompts of
 * `length` tokens with `k_count` marker slots each:
 *   ids (L, B) int64, mask (L, B) bytes (non-zero = valid token),
 *   marker_pos (K, B) int64 (negative positions read token 0 and must be
 *   masked), marker_mask (K, B) bytes, qtype (B) int64 in {0, 1, 2}.
 * Outputs: logits (K, B) masked marker logits (-1e4 where masked), action
 * (actions, B).
 * Errors (TFD_EINVAL) follow the reference's fields and messages:
 * `laya.qtype` (empty batch, qtype outside 0..2), `laya.ids` (empty
 * sequence, token outside the vocabulary), `laya.marker_pos` (fewer than two
 * marker slots), and the weight-shape fields of LayaWeights::validate.
 */
int tfd_laya_forward_f32(tfd_ctx *ctx, const tfd_laya_model *model, const int64_t *ids,
                         const uint8_t *mask, size_t length, size_t batch,
                         const int64_t *marker_pos, const uint8_t *marker_mask, size_t k_count,
                         const int64_t *qtype, float *logits, float *action, unsigned flags);

#ifdef __cplusplus
}
#endif

#endif /* TFD_LAYA_MODEL_H */
