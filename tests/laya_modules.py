"""The Laya decision model assembled from library modules, on the CPU: an
implementation independent of the oracle's step-by-step restatement.

* encoder: ``transformers``' ModernBertModel (eager attention) with the
  checkpoint's encoder weights -- the published ModernBERT the Laya encoder
  is (laya-infer model.rs:646-713: embeddings + LayerNorm, pre-norm layers
  with the identity first attn_norm, RoPE global/local, GeGLU MLP with the
  erf GELU on the first half, final LayerNorm);
* decision-head layers: ``torch.nn.TransformerEncoderLayer`` with
  ``norm_first=True``, ReLU and the key padding mask (model.rs:715-747);
* scorer and action head: ``nn.LayerNorm`` / ``nn.Linear`` / ``nn.GELU()``
  (exact erf) (model.rs:937-966); pooling with ``torch.softmax`` /
  ``torch.topk`` (model.rs:773-837).

Only the outputs of valid tokens are comparable: ModernBertModel restricts a
padded query to its window in sliding layers where build_mask lets it see
every valid key (model.rs:467-490); no valid token ever reads a padded one.
"""
import numpy as np
import torch
from torch import nn


def _t(x, shape, dtype):
    return torch.from_numpy(np.asarray(x, np.float64).reshape(shape)).to(dtype)


def encoder_module(enc, w, dtype=torch.float64):
    from transformers import ModernBertConfig, ModernBertModel
    from transformers.utils import logging as hf_logging

    hf_logging.set_verbosity_error()
    cfg = ModernBertConfig(
        vocab_size=enc.vocab_size, hidden_size=enc.hidden_size,
        intermediate_size=enc.intermediate_size, num_hidden_layers=enc.num_hidden_layers,
        num_attention_heads=enc.num_attention_heads, norm_eps=enc.norm_eps,
        norm_bias=enc.norm_bias, attention_bias=enc.attention_bias, mlp_bias=enc.mlp_bias,
        local_attention=enc.local_attention,
        global_attn_every_n_layers=enc.global_attn_every_n_layers,
        global_rope_theta=enc.global_rope_theta, local_rope_theta=enc.local_rope_theta,
        max_position_embeddings=enc.max_position_embeddings, hidden_activation="gelu",
        embedding_dropout=0.0, attention_dropout=0.0, mlp_dropout=0.0, pad_token_id=0,
        bos_token_id=None, eos_token_id=None, cls_token_id=None, sep_token_id=None,
        attn_implementation="eager")
    m = ModernBertModel(cfg).eval().to(dtype)
    d, inter = enc.hidden_size, enc.intermediate_size
    sd = {"embeddings.tok_embeddings.weight": _t(w["tok_embeddings"], (-1, d), dtype),
          "embeddings.norm.weight": _t(w["embed_norm.w"], (d,), dtype),
          "final_norm.weight": _t(w["final_norm.w"], (d,), dtype)}
    for i in range(enc.num_hidden_layers):
        p = f"layers.{i}."
        if w[p + "attn_norm.w"] is not None:
            sd[p + "attn_norm.weight"] = _t(w[p + "attn_norm.w"], (d,), dtype)
        sd[p + "attn.Wqkv.weight"] = _t(w[p + "wqkv.w"], (3 * d, d), dtype)
        sd[p + "attn.Wo.weight"] = _t(w[p + "wo.w"], (d, d), dtype)
        sd[p + "mlp_norm.weight"] = _t(w[p + "mlp_norm.w"], (d,), dtype)
        sd[p + "mlp.Wi.weight"] = _t(w[p + "wi.w"], (2 * inter, d), dtype)
        sd[p + "mlp.Wo.weight"] = _t(w[p + "wo_mlp.w"], (d, inter), dtype)
    missing, unexpected = m.load_state_dict(sd, strict=False)
    assert not unexpected and not [k for k in missing if "weight" in k], (missing, unexpected)
    return m


def encode(enc, w, ids, mask, B, dtype=torch.float64):
    """(B, L, d) final_norm outputs of ModernBertModel."""
    m = encoder_module(enc, w, dtype)
    L = len(ids) // B
    ids_t = torch.from_numpy(np.asarray(ids, np.int64).reshape(B, L))
    am = torch.from_numpy(np.asarray(mask, bool).reshape(B, L).astype(np.int64))
    with torch.no_grad():
        return m(input_ids=ids_t, attention_mask=am).last_hidden_state


def forward(ckpt, ids, mask, marker_pos, marker_mask, qtype, dtype=torch.float64):
    """(logits (B, K), action (B, actions)) of the module assembly."""
    enc, w = ckpt.encoder, ckpt.weights
    d, eps = enc.hidden_size, enc.norm_eps
    B = len(qtype)
    L, K = len(ids) // B, len(marker_pos) // B
    e = encode(enc, w, ids, mask, B, dtype)
    temb = _t(w["type_emb"], (3, d), dtype)
    h = e + temb[torch.from_numpy(np.asarray(qtype, np.int64))][:, None, :]
    pad = torch.from_numpy(~np.asarray(mask, bool).reshape(B, L))
    # A padded query whose window holds no valid key comes out of
    # ModernBertModel as NaN, which the head's masked keys would still carry
    # into valid tokens (0 * NaN); no valid token depends on a padded one, so
    # those states are zeroed here.
    h = torch.where(pad[:, :, None], torch.zeros_like(h), h)
    with torch.no_grad():
        for i in range(ckpt.agent.head_layers):
            p = f"head.{i}."
            layer = nn.TransformerEncoderLayer(d, ckpt.head_heads, 4 * d, dropout=0.0,
                                               activation="relu", layer_norm_eps=eps,
                                               batch_first=True, norm_first=True).to(dtype)
            layer.train()  # the slow path, exactly the documented math (dropout 0)
            sa = layer.self_attn
            sa.in_proj_weight.copy_(_t(w[p + "in_proj.w"], (3 * d, d), dtype))
            sa.in_proj_bias.copy_(_t(w[p + "in_proj.b"], (3 * d,), dtype))
            sa.out_proj.weight.copy_(_t(w[p + "out_proj.w"], (d, d), dtype))
            sa.out_proj.bias.copy_(_t(w[p + "out_proj.b"], (d,), dtype))
            for name, part, shape in (("linear1", "linear1", (4 * d, d)),
                                      ("linear2", "linear2", (d, 4 * d))):
                getattr(layer, name).weight.copy_(_t(w[p + part + ".w"], shape, dtype))
                getattr(layer, name).bias.copy_(_t(w[p + part + ".b"], (shape[0],), dtype))
            for name in ("norm1", "norm2"):
                getattr(layer, name).weight.copy_(_t(w[p + name + ".w"], (d,), dtype))
                getattr(layer, name).bias.copy_(_t(w[p + name + ".b"], (d,), dtype))
            h = layer(h, src_key_padding_mask=pad)
        pos = torch.from_numpy(np.maximum(np.asarray(marker_pos, np.int64).reshape(B, K), 0))
        markers = h[torch.arange(B)[:, None], pos]                       # (B, K, d)
        norm = nn.LayerNorm(d, eps=eps).to(dtype)
        norm.weight.copy_(_t(w["scorer_norm.w"], (d,), dtype))
        norm.bias.copy_(_t(w["scorer_norm.b"], (d,), dtype))

        def lin(key, n_in, n_out):
            layer = nn.Linear(n_in, n_out).to(dtype)
            layer.weight.copy_(_t(w[key + ".w"], (n_out, n_in), dtype))
            layer.bias.copy_(_t(w[key + ".b"], (n_out,), dtype))
            return layer

        gelu = nn.GELU()
        raw = lin("scorer2", d, 1)(gelu(lin("scorer1", d, d)(norm(markers))))[..., 0]  # (B, K)
        mm = torch.from_numpy(np.asarray(marker_mask, bool).reshape(B, K))
        logits = torch.where(mm, raw, torch.full_like(raw, -1.0e4))
        probs = torch.softmax(logits, dim=1)
        top = torch.topk(probs, 2, dim=1).values
        used = mm.sum(dim=1).clamp(min=2).to(dtype)
        ent = -(probs * torch.log(probs.clamp(min=1e-9))).sum(dim=1) / torch.log(used)
        feats = torch.stack([top[:, 0], top[:, 0] - top[:, 1], ent, used / 255.0], dim=1)
        pooled = torch.cat([h[:, 0, :], feats], dim=1)
        ah = len(w["act1.b"])
        action = lin("act2", ah, ckpt.agent.action_count())(gelu(lin("act1", d + 4, ah)(pooled)))
    return logits.numpy(), action.numpy()
