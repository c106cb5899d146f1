"""TEST INFRASTRUCTURE ONLY -- CPU oracle for the fused attention path.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg may
import this package, and only as the checker or the timed CPU baseline; the
product (``tenferro_ext`` / ``libtfd_attention.so``) never calls into it.

Two independent restatements live here:

* ``libtfd_oracle.so`` (``tfd_oracle.c``): a plain-C restatement of the
  reference's CPU kernels (crates/cpu-kernels/src/lib.rs:609-1156), including
  the Laya tile/GEMM/scalar policy, RoPE tables from the C library's f32
  ``powf``/``cosf``/``sinf``, the NaN and zero-row semantics, and the rayon
  decomposition on a pthread pool. This is the parity oracle and the CPU
  baseline ("port").
* ``brute``: float64 numpy restatements of the reference's *host* oracles,
  ``attention_host`` (crates/laya-infer/src/model.rs:521-581) and
  ``full_attention_host`` (crates/jeff-infer/src/model.rs:404-473), used to
  pin the C restatement on small inputs.

What pins each part: the reference's known-answer tests and golden vectors
(tests/test_golden.py, tests/test_oracle.py; the model forward of
``laya_model`` against the laya-tiny fixture's outputs and an assembly of
library modules, tests/test_laya_model.py), float64 brute force at the
reference tests' shapes, closed forms of the Jeff norm convention
(tests/test_jeff_closed_forms.py) and planted mistakes that each of these
checks must catch. No function here is left without such a check.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "libtfd_oracle.so")

_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P, S, F, I = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_float, ctypes.c_int
        L.oracle_set_threads.argtypes = [I]
        L.oracle_set_threads.restype = None
        L.oracle_get_threads.restype = I
        L.oracle_rope_table.argtypes = [S, S, F, P, P]
        L.oracle_rope_table.restype = None
        L.oracle_laya_attention_block.argtypes = [P, S, P, S, S, S, S, S, F, P, S, I]
        L.oracle_laya_attention_block.restype = I
        L.oracle_laya_build_mask.argtypes = [P, S, S, ctypes.c_long, P]
        L.oracle_laya_build_mask.restype = None
        L.oracle_jeff_full_attention.argtypes = [P, P, P, P, P, P, P, S, S, S, S, F, F, P]
        L.oracle_jeff_full_attention.restype = I
        L.oracle_expand_kv.argtypes = [P, S, S, S, S, P]
        L.oracle_expand_kv.restype = None
        _lib = L
    return _lib


def _f32(x):
    return np.ascontiguousarray(x, dtype=np.float32).reshape(-1)


def _u8(x):
    return np.ascontiguousarray(x, dtype=np.uint8).reshape(-1)


def set_threads(n: int) -> None:
    lib().oracle_set_threads(int(n))


def get_threads() -> int:
    return lib().oracle_get_threads()


def rope_table(length: int, dim: int, base: float):
    """(cos, sin) of shape (length, dim//2), cpu-kernels lib.rs:874-888."""
    half = dim // 2
    c = np.zeros(length * half + 1, np.float32)
    s = np.zeros(length * half + 1, np.float32)
    lib().oracle_rope_table(length, dim, base, c.ctypes.data, s.ctypes.data)
    return c[:-1].reshape(length, half), s[:-1].reshape(length, half)


def laya_attention_block(qkv, keep, d, heads, length, batch, rope_base, *, scalar_only=False,
                         out=None):
    """laya_attention_block_into (lib.rs:809-840) on flat column-major buffers.
    Returns the flat (d, L, B) output; raises ValueError on a storage mismatch
    (the reference panics with "qkv length"/"output length"/"mask length")."""
    qkv = _f32(qkv)
    keep = _u8(keep)
    if out is None:
        out = np.zeros(d * length * batch, np.float32)  # laya_attention.rs:141
    rc = lib().oracle_laya_attention_block(qkv.ctypes.data, qkv.size, keep.ctypes.data, keep.size,
                                           d, heads, length, batch, rope_base, out.ctypes.data,
                                           out.size, 1 if scalar_only else 0)
    if rc != 0:
        raise ValueError({-1: "qkv length", -2: "output length", -3: "mask length"}[rc])
    return out


def laya_build_mask(valid, length, batch, window):
    """build_mask (laya-infer model.rs:465-490); window < 0 = FullAttention."""
    valid = _u8(valid)
    keep = np.zeros(length * length * batch, np.uint8)
    lib().oracle_laya_build_mask(valid.ctypes.data, length, batch, int(window), keep.ctypes.data)
    return keep


def jeff_full_attention(q, k, v, gate, q_norm, k_norm, mask, length, heads, head_dim, rotary_dim,
                        theta, eps):
    """jeff_full_attention_into (lib.rs:618-763); returns flat (L, W)."""
    q, k, v, gate, q_norm, k_norm, mask = map(_f32, (q, k, v, gate, q_norm, k_norm, mask))
    out = np.zeros(length * heads * head_dim, np.float32)
    lib().oracle_jeff_full_attention(q.ctypes.data, k.ctypes.data, v.ctypes.data,
                                     gate.ctypes.data, q_norm.ctypes.data, k_norm.ctypes.data,
                                     mask.ctypes.data, length, heads, head_dim, rotary_dim, theta,
                                     eps, out.ctypes.data)
    return out


def expand_kv(src, length, heads, kv_heads, head_dim):
    """GQA expansion of a (L, kv_heads*hd) tensor (jeff checkpoint.rs:307-319)."""
    src = _f32(src)
    dst = np.zeros(length * heads * head_dim, np.float32)
    lib().oracle_expand_kv(src.ctypes.data, length, heads, kv_heads, head_dim, dst.ctypes.data)
    return dst


def jeff_rows(q, k, v, gate, q_norm, k_norm, mask, rows, length, heads, kv_heads, head_dim,
              rotary_dim, theta, eps, *, trim_leading=False):
    """Row-by-row Jeff with GQA expansion; with trim_leading, each row is first
    trimmed to its first active key as JeffEngine::row_logits does
    (jeff engine.rs:317-329) and dropped positions are 0."""
    W, KW = heads * head_dim, kv_heads * head_dim
    q, k, v, gate, mask = map(_f32, (q, k, v, gate, mask))
    out = np.zeros(rows * length * W, np.float32)
    for r in range(rows):
        qr = q[r * length * W:(r + 1) * length * W].reshape(W, length)
        gr = gate[r * length * W:(r + 1) * length * W].reshape(W, length)
        kr = k[r * length * KW:(r + 1) * length * KW].reshape(KW, length)
        vr = v[r * length * KW:(r + 1) * length * KW].reshape(KW, length)
        mr = mask[r * length:(r + 1) * length]
        start = 0
        if trim_leading:
            nz = np.nonzero(mr != 0.0)[0]
            start = int(nz[0]) if nz.size else 0
        n = length - start
        if n == 0:
            continue
        ke = expand_kv(kr[:, start:], n, heads, kv_heads, head_dim)
        ve = expand_kv(vr[:, start:], n, heads, kv_heads, head_dim)
        o = jeff_full_attention(qr[:, start:], ke, ve, gr[:, start:], q_norm, k_norm, mr[start:],
                                n, heads, head_dim, rotary_dim, theta, eps)
        full = np.zeros((W, length), np.float32)
        full[:, start:] = o.reshape(W, n)
        out[r * length * W:(r + 1) * length * W] = full.reshape(-1)
    return out


# ------------------------------------------------------------------ layers
#
# The layer entries' linears restated as float32 GEMMs (numpy, i.e. a library
# sgemm with f32 accumulation, like the reference's matrixmultiply / portable
# gemm on the CPU path); the attention op between them is the C restatement.


def _cols(flat, rows_of_matrix):
    """A column-major (m, n) buffer as an (m, n) numpy view."""
    return np.asarray(flat, np.float32).reshape(-1, rows_of_matrix).T


def laya_attention_layer(x, keep, w_in, b_in, w_out, b_out, hidden, heads, length, batch,
                         rope_base):
    """attention_block_tenferro (laya-infer model.rs:1304-1347), f32 CPU path:
    qkv = W_in^T x (+ b_in) by linear_feature_first (model.rs:1179-1216), the
    Laya op, out = W_out^T attended (+ b_out). Flat (hidden, L, B) in and out."""
    d, n = hidden, length * batch
    X = _cols(x, d)                                  # (d, N)
    qkv = _cols(w_in, d).T @ X                       # (3d, N)
    if b_in is not None:
        qkv = qkv + np.asarray(b_in, np.float32)[:, None]
    att = laya_attention_block(np.ascontiguousarray(qkv.T).reshape(-1), keep, d, heads, length,
                               batch, rope_base)
    y = _cols(w_out, d).T @ _cols(att, d)            # (d, N)
    if b_out is not None:
        y = y + np.asarray(b_out, np.float32)[:, None]
    return np.ascontiguousarray(y.T, np.float32).reshape(-1)


def jeff_layer_rows(x, w_q, w_gate, w_k, w_v, w_o, q_norm, k_norm, mask, rows, length, hidden,
                    heads, kv_heads, head_dim, rotary_dim, theta, eps, *, trim_leading=False):
    """full_attention_tenferro (jeff-infer model.rs:686-780), f32 CPU path,
    row by row: y = x W by linear_tenferro (model.rs:289-317) for q, gate, k
    and v, the Jeff op (GQA), out = merged W_o. Flat rows x (L, hidden)."""
    W, KW = heads * head_dim, kv_heads * head_dim
    x = np.asarray(x, np.float32)
    Wq, Wg = _cols(w_q, hidden), _cols(w_gate, hidden)
    Wk, Wv, Wo = _cols(w_k, hidden), _cols(w_v, hidden), _cols(w_o, W)
    flat = lambda m: np.ascontiguousarray(m.T, np.float32).reshape(-1)
    q, g, k, v = [], [], [], []
    for r in range(rows):
        Xr = _cols(x[r * length * hidden:(r + 1) * length * hidden], length)  # (L, hidden)
        q.append(flat(Xr @ Wq))
        g.append(flat(Xr @ Wg))
        k.append(flat(Xr @ Wk))
        v.append(flat(Xr @ Wv))
    merged = jeff_rows(np.concatenate(q), np.concatenate(k), np.concatenate(v), np.concatenate(g),
                       q_norm, k_norm, mask, rows, length, heads, kv_heads, head_dim, rotary_dim,
                       theta, eps, trim_leading=trim_leading)
    out = []
    for r in range(rows):
        Mr = _cols(merged[r * length * W:(r + 1) * length * W], length)       # (L, W)
        out.append(flat(Mr @ Wo))
    return np.concatenate(out)
