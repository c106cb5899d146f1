"""TEST INFRASTRUCTURE ONLY -- float64 brute-force restatements of the
reference's host oracles, used to pin the C oracle on small inputs.

These follow different reference functions than ``tfd_oracle.c`` does:

* ``laya_attention_host`` follows the host forward's split/RoPE/attention
  (crates/laya-infer/src/model.rs: ``rope_host`` 492-519, ``attention_host``
  521-581): per query, masked softmax over all keys in float64.
* ``jeff_full_attention_host`` follows ``full_attention_host``
  (crates/jeff-infer/src/model.rs:404-473) with ``rms_heads`` (477-501) and
  the partial RoPE, in float64.

RoPE angles are evaluated in float64 here (the reference's host oracle uses
f32 ``exp2``), so agreement with the f32 restatement is a tolerance, not a
bit pattern.
"""
from __future__ import annotations

import numpy as np


def _rotate(x, pos, base, rot):
    """Rotate pairs (i, i + rot/2), i < rot/2, of the last axis by pos * base^(-2i/rot)."""
    half = rot // 2
    if half == 0 or base == 0.0:
        return x.copy()
    i = np.arange(half, dtype=np.float64)
    ang = np.asarray(pos, dtype=np.float64)[:, None] * np.power(float(base), -2.0 * i / rot)[None, :]
    c, s = np.cos(ang), np.sin(ang)
    y = x.copy()
    a, b = x[..., :half], x[..., half:2 * half]
    y[..., :half] = a * c - b * s
    y[..., half:2 * half] = a * s + b * c
    return y


def laya_attention_host(qkv, keep, d, heads, length, batch, rope_base):
    """(d, L, B) float64 output of split + RoPE + masked attention.
    A query that keeps no key yields NaN (0/0), as in attention_host."""
    hd = d // heads
    x = np.asarray(qkv, np.float64).reshape(batch, length, 3 * d)
    kp = np.asarray(keep).reshape(batch, length, length).astype(bool)  # [b, key, query]
    out = np.zeros((batch, length, d))
    pos = np.arange(length)
    for b in range(batch):
        for h in range(heads):
            f = slice(h * hd, (h + 1) * hd)
            q = x[b, :, f]
            k = x[b, :, d + h * hd:d + (h + 1) * hd]
            v = x[b, :, 2 * d + h * hd:2 * d + (h + 1) * hd]
            if rope_base != 0.0:
                q = _rotate(q, pos, rope_base, hd)
                k = _rotate(k, pos, rope_base, hd)
            s = (q @ k.T) / np.sqrt(hd)  # [query, key]
            allowed = kp[b].T  # [query, key]
            s = np.where(allowed, s, -np.inf)
            with np.errstate(invalid="ignore", divide="ignore"):
                m = np.max(s, axis=1, keepdims=True)
                e = np.where(allowed, np.exp(s - m), 0.0)
                p = e / e.sum(axis=1, keepdims=True)
            vv = np.where(np.isfinite(v), v, 0.0)
            o = p @ vv
            o[~allowed.any(axis=1)] = np.nan
            out[b, :, f] = o
    return out.reshape(-1)


def jeff_full_attention_host(q, k, v, gate, q_norm, k_norm, mask, length, heads, head_dim,
                             rotary_dim, theta, eps, zero_empty=True):
    """Flat (L, W) float64 output. ``zero_empty`` applies the op's rule that a
    query with no kept key gives 0 (cpu-kernels lib.rs:743); the host oracle
    itself would give NaN there."""
    W = heads * head_dim
    shape = (W, length)  # column-major (L, W): element t + L*f
    Q, K, V, G = (np.asarray(a, np.float64).reshape(shape) for a in (q, k, v, gate))
    qn, kn = np.asarray(q_norm, np.float64), np.asarray(k_norm, np.float64)
    mk = np.asarray(mask, np.float64)
    pos = np.arange(length)
    out = np.zeros(shape)
    for h in range(heads):
        f = slice(h * head_dim, (h + 1) * head_dim)
        qh, kh, vh, gh = Q[f].T, K[f].T, V[f].T, G[f].T  # [t, i]
        qh = qh / np.sqrt(np.mean(qh * qh, axis=1, keepdims=True) + eps) * (1.0 + qn)
        kh = kh / np.sqrt(np.mean(kh * kh, axis=1, keepdims=True) + eps) * (1.0 + kn)
        qh = _rotate(qh, pos, theta, rotary_dim)
        kh = _rotate(kh, pos, theta, rotary_dim)
        s = qh @ kh.T / np.sqrt(head_dim)
        allowed = (pos[None, :] <= pos[:, None]) & (mk[None, :] != 0.0)
        s = np.where(allowed, s, -np.inf)
        with np.errstate(invalid="ignore", divide="ignore"):
            m = np.max(s, axis=1, keepdims=True)
            e = np.where(allowed, np.exp(s - m), 0.0)
            p = e / e.sum(axis=1, keepdims=True)
        o = p @ vh
        empty = ~allowed.any(axis=1)
        o[empty] = 0.0 if zero_empty else np.nan
        out[f] = (o / (1.0 + np.exp(-gh))).T
    return out.reshape(-1)


def laya_attention_layer_host(x, keep, w_in, b_in, w_out, b_out, hidden, heads, length, batch,
                              rope_base):
    """The Laya layer (laya-infer model.rs:1304-1347) in float64: linears as
    float64 matrix products around laya_attention_host."""
    d = hidden
    X = np.asarray(x, np.float64).reshape(-1, d).T
    qkv = np.asarray(w_in, np.float64).reshape(-1, d) @ X
    if b_in is not None:
        qkv = qkv + np.asarray(b_in, np.float64)[:, None]
    att = laya_attention_host(qkv.T.reshape(-1), keep, d, heads, length, batch, rope_base)
    y = np.asarray(w_out, np.float64).reshape(-1, d) @ att.reshape(-1, d).T
    if b_out is not None:
        y = y + np.asarray(b_out, np.float64)[:, None]
    return y.T.reshape(-1)


def jeff_layer_host(x, w_q, w_gate, w_k_expanded, w_v_expanded, w_o, q_norm, k_norm, mask,
                    length, hidden, heads, head_dim, rotary_dim, theta, eps):
    """One row of the Jeff layer (jeff-infer model.rs:686-780) in float64,
    with K/V projections already expanded to every query head."""
    W = heads * head_dim
    X = np.asarray(x, np.float64).reshape(hidden, length).T                  # (L, hidden)
    proj = lambda w: (X @ np.asarray(w, np.float64).reshape(-1, hidden).T).T.reshape(-1)
    merged = jeff_full_attention_host(proj(w_q), proj(w_k_expanded), proj(w_v_expanded),
                                      proj(w_gate), q_norm, k_norm, mask, length, heads,
                                      head_dim, rotary_dim, theta, eps)
    M = merged.reshape(W, length).T                                            # (L, W)
    return (M @ np.asarray(w_o, np.float64).reshape(hidden, W).T).T.reshape(-1)
