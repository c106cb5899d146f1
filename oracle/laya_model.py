"""TEST INFRASTRUCTURE ONLY -- CPU restatements of the Laya decision-model
forward, the checker of ``tfd_laya_forward_f32``.

* ``forward(...)``: float32 numpy, step by step as ``forward_reference``
  (crates/laya-infer/src/model.rs:867-977) and its host helpers
  (``layer_norm_host`` 387-422, ``linear_host`` 424-457, ``gelu_gate_host``
  635-645, ``encoder_host`` 646-713, ``head_layer_host`` 715-747,
  ``gather_markers_host`` 749-771, ``pool_host`` 773-837), with every
  attention block through the C restatement (``oracle.laya_attention_layer``
  under ``oracle.laya_build_mask``).
* ``forward(..., f64=True)``: the same steps in float64 with the float64
  brute-force attention (``oracle.brute.laya_attention_layer_host``).

The exact GELU takes erf from Python's ``math.erf`` (float64, correctly
rounded to a few ulp); the reference evaluates the MLX single-precision erf
polynomial, which agrees with it to within a few f32 ulp.

Pinned by the reference's own golden vector: ``fixtures/laya-tiny``'s
``reference.json`` logits and action (the Julia ``DecisionModel`` outputs,
native_fixture.rs:75-139, tolerance 1e-5), held under tests/golden/laya_tiny.

``weights`` is a dict of host-layout float32 arrays keyed as
``tenferro_ext.laya_model.build_weights`` writes them.
"""
from __future__ import annotations

import math

import numpy as np

from . import brute, laya_attention_layer, laya_build_mask

_erf = np.vectorize(math.erf, otypes=[np.float64])


def _dt(f64):
    return np.float64 if f64 else np.float32


def gelu(x, f64=False):
    """exact_gelu (model.rs:312-314): x * (1 + erf(x / sqrt 2)) / 2."""
    t = _dt(f64)
    x = np.asarray(x, t)
    e = _erf((x / t(math.sqrt(2.0))).astype(np.float64)).astype(t)
    return (x * (t(1.0) + e) / t(2.0)).astype(t)


def layer_norm(w, b, x, d, eps, f64=False):
    """layer_norm_host (model.rs:387-422) over the columns of a flat (d, N)."""
    t = _dt(f64)
    X = np.asarray(x, t).reshape(-1, d)                 # (N, d): one row per column
    mean = (X.sum(axis=1, dtype=t) / t(d)).astype(t)
    c = X - mean[:, None]
    var = ((c * c).sum(axis=1, dtype=t) / t(d)).astype(t)
    inv = (t(1.0) / np.sqrt(var + t(eps))).astype(t)
    y = (c * inv[:, None]) * np.asarray(w, t)[None, :]
    if b is not None:
        y = y + np.asarray(b, t)[None, :]
    return y.astype(t).reshape(-1)


def linear(w, b, n_in, n_out, x, f64=False):
    """linear_host (model.rs:424-457): y (out, N) = W^T x (+ b) for the
    column-major (in, out) weight."""
    t = _dt(f64)
    W = np.asarray(w, t).reshape(n_out, n_in)           # row o = column o of (in, out)
    X = np.asarray(x, t).reshape(-1, n_in)              # (N, in)
    y = X @ W.T
    if b is not None:
        y = y + np.asarray(b, t)[None, :]
    return y.astype(t).reshape(-1)


def _attn(d, L, B, f64):
    def attn(x, keep, wi, bi, wo, bo, heads, base):
        if f64:
            return brute.laya_attention_layer_host(x, keep, wi, bi, wo, bo, d, heads, L, B, base)
        return laya_attention_layer(x, keep, wi, bi, wo, bo, d, heads, L, B, base)
    return attn


def _act(plant, f64):
    t = _dt(f64)

    def act(x):
        if plant == "tanh_gelu":
            x = np.asarray(x, np.float64)
            return (0.5 * x * (1 + np.tanh(math.sqrt(2 / math.pi) * (x + 0.044715 * x ** 3)))).astype(t)
        return gelu(x, f64)
    return act


def encoder(enc, w, ids, mask, B, *, f64=False, plant=None):
    """encoder_host (model.rs:646-713): final_norm of the last layer's output,
    flat (d, L, B)."""
    t = _dt(f64)
    d, inter, eps = enc.hidden_size, enc.intermediate_size, enc.norm_eps
    L = len(ids) // B
    valid = np.asarray(mask, np.uint8).reshape(-1)
    attn, act = _attn(d, L, B, f64), _act(plant, f64)
    # encoder_host (646-713)
    tok = np.asarray(w["tok_embeddings"], t).reshape(-1, d)
    x = tok[np.asarray(ids, np.int64)].reshape(-1)
    if plant != "no_embed_norm":
        x = layer_norm(w["embed_norm.w"], w["embed_norm.b"], x, d, eps, f64)
    window = enc.local_attention // 2
    for i, kind in enumerate(enc.layer_types):
        p = f"layers.{i}."
        a = x if w[p + "attn_norm.w"] is None else layer_norm(
            w[p + "attn_norm.w"], w[p + "attn_norm.b"], x, d, eps, f64)
        sliding = kind == "sliding_attention" and plant != "global_only"
        keep = laya_build_mask(valid, L, B, window if sliding else -1)
        base = 0.0 if plant == "no_rope" else enc.rope_base(kind)
        z = (x + attn(a, keep, w[p + "wqkv.w"], w[p + "wqkv.b"], w[p + "wo.w"], w[p + "wo.b"],
                      enc.num_attention_heads, base)).astype(t)
        if plant != "no_mlp":
            hn = layer_norm(w[p + "mlp_norm.w"], w[p + "mlp_norm.b"], z, d, eps, f64)
            u = linear(w[p + "wi.w"], w[p + "wi.b"], d, 2 * inter, hn, f64).reshape(-1, 2 * inter)
            first, second = (u[:, inter:], u[:, :inter]) if plant == "swap_geglu" else \
                (u[:, :inter], u[:, inter:])
            g = (act(first) * second).astype(t).reshape(-1)
            z = (z + linear(w[p + "wo_mlp.w"], w[p + "wo_mlp.b"], inter, d, g, f64)).astype(t)
        x = z
    return layer_norm(w["final_norm.w"], w["final_norm.b"], x, d, eps, f64)


def forward(enc, agent_actions, w, head_heads, ids, mask, marker_pos, marker_mask, qtype, *,
            f64=False, plant=None):
    """forward_reference (model.rs:867-977). ``enc`` is the EncoderConfig,
    ``ids``/``mask`` flat (L, B), ``marker_pos``/``marker_mask`` flat (K, B),
    ``qtype`` (B). Returns (masked logits (K, B), action (actions, B)).

    ``plant`` names one deliberate mistake for the tests that check what the
    golden vector catches: "no_embed_norm", "tanh_gelu", "no_mlp",
    "swap_geglu", "no_head_layer", "qtype0", "no_rope", "global_only"."""
    t = _dt(f64)
    d = enc.hidden_size
    eps = enc.norm_eps
    B = len(qtype)
    L = len(ids) // B
    K = len(marker_pos) // B
    valid = np.asarray(mask, np.uint8).reshape(-1)
    attn, act = _attn(d, L, B, f64), _act(plant, f64)
    e = encoder(enc, w, ids, mask, B, f64=f64, plant=plant)

    # typed head (916-931)
    temb = np.asarray(w["type_emb"], t).reshape(3, d)
    qt = np.zeros(B, np.int64) if plant == "qtype0" else np.asarray(qtype, np.int64)
    h = (e.reshape(B, L, d) + temb[qt][:, None, :]).astype(t).reshape(-1)
    head_keep = laya_build_mask(valid, L, B, -1)
    n_head = 0 if plant == "no_head_layer" else sum(1 for k in w if k.endswith(".norm1.w"))
    for i in range(n_head):
        p = f"head.{i}."
        n = layer_norm(w[p + "norm1.w"], w[p + "norm1.b"], h, d, eps, f64)
        z = (h + attn(n, head_keep, w[p + "in_proj.w"], w[p + "in_proj.b"], w[p + "out_proj.w"],
                      w[p + "out_proj.b"], head_heads, 0.0)).astype(t)
        hn = layer_norm(w[p + "norm2.w"], w[p + "norm2.b"], z, d, eps, f64)
        ff = len(w[p + "linear1.b"])
        r = np.maximum(linear(w[p + "linear1.w"], w[p + "linear1.b"], d, ff, hn, f64), t(0.0))
        h = (z + linear(w[p + "linear2.w"], w[p + "linear2.b"], ff, d, r, f64)).astype(t)

    # markers and scorer (937-941)
    H = h.reshape(B, L, d)
    pos = np.maximum(np.asarray(marker_pos, np.int64).reshape(B, K), 0)
    markers = H[np.arange(B)[:, None], pos].reshape(-1)
    s0 = layer_norm(w["scorer_norm.w"], w["scorer_norm.b"], markers, d, eps, f64)
    s1 = act(linear(w["scorer1.w"], w["scorer1.b"], d, d, s0, f64))
    raw = linear(w["scorer2.w"], w["scorer2.b"], d, 1, s1, f64)

    # pool_host (773-837)
    mm = np.asarray(marker_mask, bool).reshape(B, K)
    logits = np.where(mm, raw.reshape(B, K), t(-1.0e4)).astype(t)
    feats = np.zeros((B, 4), t)
    for b in range(B):
        row = logits[b]
        ex = np.exp(row - row.max()).astype(t)
        probs = (ex / ex.sum(dtype=t)).astype(t)
        srt = np.sort(probs)[::-1]
        top1, top2 = srt[0], (srt[1] if K > 1 else t(-np.inf))
        ent = -(probs * np.log(np.maximum(probs, t(1e-9)))).sum(dtype=t)
        used = t(max(int(mm[b].sum()), 2))
        feats[b] = [top1, top1 - top2, ent / np.log(used), used / t(255.0)]
    pooled = np.concatenate([H[:, 0, :], feats], axis=1).astype(t).reshape(-1)

    # action head (943-966)
    ah = len(w["act1.b"])
    a1 = act(linear(w["act1.w"], w["act1.b"], d + 4, ah, pooled, f64))
    action = linear(w["act2.w"], w["act2.b"], ah, agent_actions, a1, f64)
    return logits.reshape(-1), action
