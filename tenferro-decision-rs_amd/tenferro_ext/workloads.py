"""Seeded synthetic inputs for the five benchmark configurations.

Uniforms come from the LCG of the reference's tests
(crates/laya-infer/tests/model.rs:17-31): s = s*6364136223846793005 +
1442695040888963407 (mod 2^64), u = (s >> 40) / 2^24. Normals are Box-Muller
pairs (z0 = r cos(2 pi u2), z1 = r sin(2 pi u2), r = sqrt(-2 ln u1)); a pair
whose u1 is 0 uses u1 = 2^-25. The seed is the configuration number. The
sequence is produced with LCG jump-ahead so full-size inputs take
milliseconds, with exactly the values a sequential loop would give.

Configurations (BASELINE.json "configs"):
  C1 Laya-tiny: qkv (192, 32, 1) ~ N(0,1), 4 heads x 16, RoPE 160000, all keep.
  C2 ModernBERT-base global: qkv (2304, 512, 8) ~ N(0, s^2), s = 0.02*sqrt(768)
     (a 768-wide projection of unit activations with N(0, 0.02^2) weights),
     RoPE 160000, right padding with valid lengths U{64..512}, full attention.
  C3 ModernBERT local: qkv (2304, 2048, 4) ~ N(0,1), RoPE 10000, all valid,
     window +-64 (local_attention 128).
  C4 Jeff full attention: 16 rows x L 256, 8 q heads / 2 kv heads x 256,
     rot 64, theta 1e7, eps 1e-6; q, gate ~ N(0, s^2) at width 2048 and
     k, v ~ N(0, s^2) at width 512 with s = 0.02*sqrt(1024) (projections of
     unit activations by N(0, 0.02^2) weights), q_norm/k_norm ~ N(0, 0.02^2);
     left padding with valid lengths U{32..256}; causal.
  C5 as C4 at 2 rows x L 8192, all active, inputs rounded to bf16.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, Optional

import numpy as np

_A = 6364136223846793005
_C = 1442695040888963407
_M = (1 << 64) - 1
_BLOCK = 8192


class Lcg:
    """The reference tests' LCG (laya-infer tests/model.rs:17-31)."""

    def __init__(self, seed: int):
        self.state = seed & _M

    def uniform(self, n: int) -> np.ndarray:
        """n uniforms in [0, 1) as float64, advancing the state by n."""
        out = np.empty(n, np.float64)
        if n == 0:
            return out
        first = np.empty(min(n, _BLOCK), np.uint64)
        s = self.state
        for i in range(first.size):
            s = (s * _A + _C) & _M
            first[i] = s
        # Jump ahead by _BLOCK: s' = A^B s + C (A^B - 1)/(A - 1).
        ab, cb = 1, 0
        for _ in range(_BLOCK):
            ab, cb = (ab * _A) & _M, (cb * _A + _C) & _M
        ab_u, cb_u = np.uint64(ab), np.uint64(cb)
        states = first
        done = 0
        with np.errstate(over="ignore"):
            while done < n:
                take = min(states.size, n - done)
                out[done:done + take] = (states[:take] >> np.uint64(40)).astype(np.float64) / float(1 << 24)
                done += take
                last = int(states[take - 1])
                if done < n:
                    states = states * ab_u + cb_u
        # Final state = the n-th draw.
        self.state = last
        return out

    def normal(self, n: int) -> np.ndarray:
        m = n + (n & 1)
        u = self.uniform(m).reshape(-1, 2)
        u1 = np.where(u[:, 0] > 0.0, u[:, 0], 2.0 ** -25)
        r = np.sqrt(-2.0 * np.log(u1))
        t = 2.0 * np.pi * u[:, 1]
        z = np.empty(m, np.float64)
        z[0::2] = r * np.cos(t)
        z[1::2] = r * np.sin(t)
        return z[:n]

    def integers(self, lo: int, hi: int, n: int) -> np.ndarray:
        """n integers uniform in [lo, hi]."""
        u = self.uniform(n)
        return lo + np.minimum((u * (hi - lo + 1)).astype(np.int64), hi - lo)


@dataclass
class LayaWorkload:
    name: str
    hidden: int
    heads: int
    length: int
    batch: int
    rope_base: float
    qkv: np.ndarray            # flat (3d, L, B) column-major, f32
    valid: np.ndarray          # flat (L, B) u8
    window: int                # -1 = global, else |q - k| <= window
    keep: Optional[np.ndarray] = None  # flat (L, L, B) u8 (build_mask)

    @property
    def head_dim(self) -> int:
        return self.hidden // self.heads

    def kept_pairs(self) -> int:
        """Kept (query, key) pairs summed over batch (times heads = P)."""
        if self.keep is not None:
            return int(np.count_nonzero(self.keep))
        L = self.length
        total = 0
        q = np.arange(L)
        for b in range(self.batch):
            v = self.valid[b * L:(b + 1) * L].astype(bool)
            if self.window < 0:
                total += L * int(v.sum())
            else:
                inside = np.abs(q[:, None] - q[None, :]) <= self.window
                inside |= ~v[:, None]
                total += int((inside & v[None, :]).sum())
        return total

    def valid_tokens(self) -> int:
        return int(np.count_nonzero(self.valid))


@dataclass
class JeffWorkload:
    name: str
    rows: int
    length: int
    heads: int
    kv_heads: int
    head_dim: int
    rotary_dim: int
    theta: float
    eps: float
    q: np.ndarray       # flat rows x (L, W) f32
    k: np.ndarray       # flat rows x (L, KW) f32 (kv_heads width)
    v: np.ndarray
    gate: np.ndarray
    q_norm: np.ndarray  # (hd)
    k_norm: np.ndarray
    mask: np.ndarray    # flat rows x (L) f32
    bf16: bool = False
    extra: Dict[str, np.ndarray] = field(default_factory=dict)

    def kept_pairs(self) -> int:
        """Kept (query, key) pairs per head summed over rows (x heads = P)."""
        total = 0
        L = self.length
        for r in range(self.rows):
            act = (self.mask[r * L:(r + 1) * L] != 0.0).astype(np.int64)
            total += int(np.cumsum(act).sum())  # sum over t of #active keys <= t
        return total

    def valid_tokens(self) -> int:
        return int(np.count_nonzero(self.mask))


def _build_keep(valid, L, B, window):
    keep = np.zeros((B, L, L), np.uint8)  # [b, key, query]
    q = np.arange(L)
    for b in range(B):
        v = valid[b * L:(b + 1) * L].astype(bool)
        inside = np.ones((L, L), bool) if window < 0 else (np.abs(q[:, None] - q[None, :]) <= window)
        inside = inside | ~v[None, :]          # [key, query]: padded query keeps every valid key
        keep[b] = (v[:, None] & inside).astype(np.uint8)
    return keep.reshape(-1)


def laya_config(cfg: int, *, with_keep: bool = True) -> LayaWorkload:
    rng = Lcg(cfg)
    if cfg == 1:
        d, H, L, B, base, window, sigma = 64, 4, 32, 1, 160000.0, -1, 1.0
        lens = np.array([L])
    elif cfg == 2:
        d, H, L, B, base, window, sigma = 768, 12, 512, 8, 160000.0, -1, 0.02 * np.sqrt(768.0)
        lens = rng.integers(64, 512, B)
    elif cfg == 3:
        d, H, L, B, base, window, sigma = 768, 12, 2048, 4, 10000.0, 64, 1.0
        lens = np.full(B, L)
    else:
        raise ValueError(f"no Laya config {cfg}")
    qkv = (rng.normal(3 * d * L * B) * sigma).astype(np.float32)
    valid = np.zeros(L * B, np.uint8)
    for b in range(B):
        valid[b * L:b * L + int(lens[b])] = 1
    keep = _build_keep(valid, L, B, window) if with_keep else None
    return LayaWorkload(f"C{cfg}", d, H, L, B, base, qkv, valid, window, keep)


def jeff_config(cfg: int, *, rows: Optional[int] = None, length: Optional[int] = None) -> JeffWorkload:
    """C4 (f32, left-padded) or C5 (bf16-rounded, all active); rows/length
    override the shape for reduced-size parity runs."""
    rng = Lcg(cfg)
    H, KV, hd, rot, theta, eps = 8, 2, 256, 64, 1.0e7, 1.0e-6
    if cfg == 4:
        R, L = 16, 256
    elif cfg == 5:
        R, L = 2, 8192
    else:
        raise ValueError(f"no Jeff config {cfg}")
    R = rows or R
    L = length or L
    W, KW = H * hd, KV * hd
    if cfg == 4:
        lens = rng.integers(min(32, L), L, R)
    else:
        lens = np.full(R, L)
    s = 0.02 * np.sqrt(1024.0)
    q = (rng.normal(R * L * W) * s).astype(np.float32)
    gate = (rng.normal(R * L * W) * s).astype(np.float32)
    k = (rng.normal(R * L * KW) * s).astype(np.float32)
    v = (rng.normal(R * L * KW) * s).astype(np.float32)
    q_norm = (rng.normal(hd) * 0.02).astype(np.float32)
    k_norm = (rng.normal(hd) * 0.02).astype(np.float32)
    mask = np.zeros(R * L, np.float32)
    for r in range(R):
        mask[r * L + (L - int(lens[r])):(r + 1) * L] = 1.0
    bf16 = cfg == 5
    if bf16:
        from . import bf16_bits_to_f32, to_bf16_bits

        q, gate, k, v = (bf16_bits_to_f32(to_bf16_bits(x)) for x in (q, gate, k, v))
    return JeffWorkload(f"C{cfg}", R, L, H, KV, hd, rot, theta, eps, q, k, v, gate, q_norm,
                        k_norm, mask, bf16)


# ------------------------------------------------------------------ layers
#
# Whole-layer inputs for the layer entries: unit activations x and
# N(0, 0.02^2) projection weights (the reading under which configs[1] and
# configs[3] give the projections' scale used above), seeded 100 + cfg.


@dataclass
class LayaLayerWorkload:
    name: str
    hidden: int
    heads: int
    length: int
    batch: int
    rope_base: float
    x: np.ndarray       # flat (d, L, B)
    w_in: np.ndarray    # flat (d, 3d) column-major
    w_out: np.ndarray   # flat (d, d) column-major
    b_in: Optional[np.ndarray]
    b_out: Optional[np.ndarray]
    valid: np.ndarray
    window: int
    keep: np.ndarray

    def gemm_flops(self) -> int:
        n = self.length * self.batch
        return 2 * n * self.hidden * (3 * self.hidden) + 2 * n * self.hidden * self.hidden


def laya_layer_config(cfg: int, *, bias: bool = False) -> LayaLayerWorkload:
    """C1 or C2 shape (valid lengths as laya_config) with x and weights."""
    base = laya_config(cfg)
    d, L, B = base.hidden, base.length, base.batch
    rng = Lcg(100 + cfg)
    x = rng.normal(d * L * B).astype(np.float32)
    w_in = (rng.normal(d * 3 * d) * 0.02).astype(np.float32)
    w_out = (rng.normal(d * d) * 0.02).astype(np.float32)
    b_in = (rng.normal(3 * d) * 0.02).astype(np.float32) if bias else None
    b_out = (rng.normal(d) * 0.02).astype(np.float32) if bias else None
    return LayaLayerWorkload(f"C{cfg}-layer", d, base.heads, L, B, base.rope_base, x, w_in, w_out,
                             b_in, b_out, base.valid, base.window, base.keep)


@dataclass
class JeffLayerWorkload:
    name: str
    rows: int
    length: int
    hidden: int
    heads: int
    kv_heads: int
    head_dim: int
    rotary_dim: int
    theta: float
    eps: float
    x: np.ndarray       # flat rows x (L, hidden)
    w_q: np.ndarray     # (hidden, W) column-major
    w_gate: np.ndarray
    w_k: np.ndarray     # (hidden, KW)
    w_v: np.ndarray
    w_o: np.ndarray     # (W, hidden)
    q_norm: np.ndarray
    k_norm: np.ndarray
    mask: np.ndarray

    def gemm_flops(self) -> int:
        W, KW = self.heads * self.head_dim, self.kv_heads * self.head_dim
        t = self.rows * self.length
        return 2 * t * self.hidden * (2 * W + 2 * KW) + 2 * t * W * self.hidden


def jeff_layer_config(cfg: int = 4, *, rows: Optional[int] = None,
                      length: Optional[int] = None, hidden: int = 1024) -> JeffLayerWorkload:
    """C4 shape (mask as jeff_config) with x and weights."""
    base = jeff_config(cfg, rows=rows, length=length)
    R, L, H, KV, hd = base.rows, base.length, base.heads, base.kv_heads, base.head_dim
    W, KW = H * hd, KV * hd
    rng = Lcg(100 + cfg)
    x = rng.normal(R * L * hidden).astype(np.float32)
    w = lambda n: (rng.normal(n) * 0.02).astype(np.float32)
    return JeffLayerWorkload(f"C{cfg}-layer", R, L, hidden, H, KV, hd, base.rotary_dim, base.theta,
                             base.eps, x, w(hidden * W), w(hidden * W), w(hidden * KW),
                             w(hidden * KW), w(W * hidden), base.q_norm, base.k_norm, base.mask)


# ------------------------------------------------------------------ decision model
#
# Synthetic Laya decision models for the forward entry: the checkpoint
# layout of a given shape with seeded random weights (linears N(0, 1/in),
# norm scales 1 + N(0, 0.1^2), biases N(0, 0.1^2)), so that every component
# of the forward moves its outputs.


def laya_model_checkpoint(*, vocab=263, hidden=32, intermediate=48, layers=2, heads=2,
                          local_attention=16, head_layers=1, actions=2, seed=7, max_len=None,
                          fast=False):
    """A LayaCheckpoint with random weights (see above) and the given shape.
    fast: numpy's PCG64 normals instead of the LCG (model-size checkpoints)."""
    from .laya_model import ACTION_HIDDEN, AgentConfig, EncoderConfig, LayaCheckpoint

    enc = EncoderConfig.from_json({
        "vocab_size": vocab, "hidden_size": hidden, "intermediate_size": intermediate,
        "num_hidden_layers": layers, "num_attention_heads": heads,
        "local_attention": local_attention,
        "max_position_embeddings": max(8192, (max_len or 0) + 1)})
    agent = AgentConfig(head_layers=head_layers, max_len=max_len or 512,
                        head_max_len=min(192, (max_len or 512) - 1),
                        action_names=[f"a{i}" for i in range(actions - 1)])
    rng = Lcg(seed)
    if fast:
        gen = np.random.default_rng(seed)

        class _Fast:
            @staticmethod
            def normal(n):
                return gen.standard_normal(n, dtype=np.float32)
        rng = _Fast()
    d, inter = hidden, intermediate
    lin = lambda n_in, n_out: (rng.normal(n_in * n_out) / np.sqrt(n_in)).astype(np.float32)
    scale = lambda n: (1.0 + 0.1 * rng.normal(n)).astype(np.float32)
    bias = lambda n: (0.1 * rng.normal(n)).astype(np.float32)
    w = {"tok_embeddings": rng.normal(vocab * d).astype(np.float32),
         "embed_norm.w": scale(d), "embed_norm.b": None}
    for i in range(layers):
        p = f"layers.{i}."
        w[p + "attn_norm.w"] = scale(d) if i else None
        w[p + "attn_norm.b"] = None
        w[p + "wqkv.w"], w[p + "wqkv.b"] = lin(d, 3 * d), None
        w[p + "wo.w"], w[p + "wo.b"] = lin(d, d), None
        w[p + "mlp_norm.w"], w[p + "mlp_norm.b"] = scale(d), None
        w[p + "wi.w"], w[p + "wi.b"] = lin(d, 2 * inter), None
        w[p + "wo_mlp.w"], w[p + "wo_mlp.b"] = lin(inter, d), None
    w["final_norm.w"], w["final_norm.b"] = scale(d), None
    for i in range(head_layers):
        p = f"head.{i}."
        for part, n_in, n_out in (("in_proj", d, 3 * d), ("out_proj", d, d),
                                  ("linear1", d, 4 * d), ("linear2", 4 * d, d)):
            w[p + part + ".w"], w[p + part + ".b"] = lin(n_in, n_out), bias(n_out)
        for part in ("norm1", "norm2"):
            w[p + part + ".w"], w[p + part + ".b"] = scale(d), bias(d)
    w["type_emb"] = rng.normal(3 * d).astype(np.float32)
    w["scorer_norm.w"], w["scorer_norm.b"] = scale(d), bias(d)
    w["scorer1.w"], w["scorer1.b"] = lin(d, d), bias(d)
    w["scorer2.w"], w["scorer2.b"] = lin(d, 1), bias(1)
    w["act1.w"], w["act1.b"] = lin(d + 4, ACTION_HIDDEN), bias(ACTION_HIDDEN)
    w["act2.w"], w["act2.b"] = lin(ACTION_HIDDEN, actions), bias(actions)
    return LayaCheckpoint(enc, agent, w, max(1, hidden // 64))


def laya_model_batch(L, B, K, vocab, *, seed=11, min_len=None):
    """Prompts for the forward: right-padded rows of random valid lengths in
    [min_len, L], ids in [0, vocab), K marker slots at distinct valid
    positions (the last slot masked in every other row), qtype cycling 0..2.
    Returns flat column-major (ids, mask, marker_pos, marker_mask, qtype)."""
    rng = Lcg(seed)
    lo = min_len if min_len is not None else max(K + 1, L // 2)
    lens = (lo + (rng.uniform(B) * (L - lo + 1)).astype(np.int64)).clip(lo, L)
    ids = (rng.uniform(L * B) * vocab).astype(np.int64).clip(0, vocab - 1)
    mask = np.zeros(L * B, bool)
    pos = np.zeros(K * B, np.int64)
    mm = np.ones(K * B, bool)
    for b in range(B):
        mask[b * L:b * L + lens[b]] = True
        step = max(1, (int(lens[b]) - 1) // K)
        pos[b * K:(b + 1) * K] = 1 + step * np.arange(K)
        if b % 2:
            mm[b * K + K - 1] = False
    qtype = np.arange(B, dtype=np.int64) % 3
    return ids, mask, pos, mm, qtype
