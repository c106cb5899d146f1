"""Closed forms that pin the Jeff norm convention independently of any
restatement of it.

cpu-kernels' centered RMSNorm (lib.rs:676-691) maps x to
x * scale * (1 + w), scale = 1 / sqrt(mean(x^2) + eps). Two weight values fix
that affine map in w without restating it:

* w = -1 on q and k: every normalized q and k is 0, every kept score is 0,
  and the softmax is uniform over the kept keys (key <= query, mask != 0),
  so out[t] = sigmoid(gate[t]) * mean of v over those keys (0 when there is
  none, lib.rs:743);
* w = 0: the weights drop out, and the output is plain causal attention on
  the RMS-normalized, rotated q and k, computed here in float64 from the
  definitions (no weight term at all).

A third check is the norm's scale invariance: q times 3 leaves the output
unchanged up to the eps term. The planted-mistake test shows that an
implementation using w in place of (1 + w) fails the first two checks.
Each check runs on the oracle (CPU) and, marked gpu, on the f32 rows entry.
"""
import numpy as np
import pytest

import oracle
import tenferro_ext as te

TOL = 2e-5


def make_case(seed, L=48, H=4, KV=2, hd=64, rot=32, scale_q=1.0):
    rng = np.random.default_rng(seed)
    W, KW = H * hd, KV * hd
    q = (rng.standard_normal(L * W) * scale_q).astype(np.float32)
    k = rng.standard_normal(L * KW).astype(np.float32)
    v = rng.standard_normal(L * KW).astype(np.float32)
    gate = rng.standard_normal(L * W).astype(np.float32)
    mask = np.ones(L, np.float32)
    mask[: L // 5] = 0.0            # left padding: the first queries keep nothing
    mask[L // 2] = 0.0              # an interior hole
    return dict(q=q, k=k, v=v, gate=gate, mask=mask, L=L, H=H, KV=KV, hd=hd, rot=rot,
                theta=1e4, eps=1e-6)


def run_oracle(c, qn, kn):
    return oracle.jeff_rows(c["q"], c["k"], c["v"], c["gate"], qn, kn, c["mask"], 1, c["L"],
                            c["H"], c["KV"], c["hd"], c["rot"], c["theta"], c["eps"])


def run_gpu(c, qn, kn, ctx):
    out = te.jeff_full_attention_rows(c["q"], c["k"], c["v"], c["gate"], qn, kn, c["mask"], 1,
                                      c["L"], c["H"], c["KV"], c["hd"], c["rot"], c["theta"],
                                      c["eps"], ctx=ctx)
    return np.asarray(out, np.float32).reshape(-1)


def uniform_average(c):
    """out with every kept score 0: sigmoid(gate) * mean of the kept keys' v."""
    L, H, KV, hd = c["L"], c["H"], c["KV"], c["hd"]
    V = c["v"].astype(np.float64).reshape(KV * hd, L)
    G = c["gate"].astype(np.float64).reshape(H * hd, L)
    out = np.zeros((H * hd, L))
    act = c["mask"] != 0
    for t in range(L):
        keys = [s for s in range(t + 1) if act[s]]
        if not keys:
            continue
        for h in range(H):
            kv = h // (H // KV)
            o = V[kv * hd:(kv + 1) * hd, keys].mean(axis=1)
            out[h * hd:(h + 1) * hd, t] = o / (1.0 + np.exp(-G[h * hd:(h + 1) * hd, t]))
    return out.reshape(-1)


def plain_rms_attention(c, weight=None):
    """Causal attention on q / rms(q) and k / rms(k), RoPE on pairs
    (i, i + rot/2) at angle t * theta^(-2i/rot), in float64 with no norm
    weight; `weight`, if given, multiplies the normalized q and k (the
    planted-mistake test passes w itself)."""
    L, H, KV, hd, rot = c["L"], c["H"], c["KV"], c["hd"], c["rot"]
    Q = c["q"].astype(np.float64).reshape(H * hd, L)
    K = c["k"].astype(np.float64).reshape(KV * hd, L)
    V = c["v"].astype(np.float64).reshape(KV * hd, L)
    G = c["gate"].astype(np.float64).reshape(H * hd, L)
    act = c["mask"] != 0
    pos = np.arange(L, dtype=np.float64)
    half = rot // 2
    ang = pos[:, None] * np.power(c["theta"], -2.0 * np.arange(half) / rot)[None, :]
    cs, sn = np.cos(ang), np.sin(ang)

    def norm_rot(x):  # x: (L, hd)
        y = x / np.sqrt(np.mean(x * x, axis=1, keepdims=True) + c["eps"])
        if weight is not None:
            y = y * weight
        z = y.copy()
        a, b = y[:, :half], y[:, half:rot]
        z[:, :half] = a * cs - b * sn
        z[:, half:rot] = a * sn + b * cs
        return z

    out = np.zeros((H * hd, L))
    allowed = (pos[None, :] <= pos[:, None]) & act[None, :]
    for h in range(H):
        kv = h // (H // KV)
        qh = norm_rot(Q[h * hd:(h + 1) * hd].T)
        kh = norm_rot(K[kv * hd:(kv + 1) * hd].T)
        s = np.where(allowed, qh @ kh.T / np.sqrt(hd), -np.inf)
        with np.errstate(invalid="ignore"):
            e = np.where(allowed, np.exp(s - s.max(axis=1, keepdims=True)), 0.0)
            p = e / e.sum(axis=1, keepdims=True)
        o = np.nan_to_num(p) @ V[kv * hd:(kv + 1) * hd].T
        o[~allowed.any(axis=1)] = 0.0
        out[h * hd:(h + 1) * hd] = (o / (1.0 + np.exp(-G[h * hd:(h + 1) * hd].T))).T
    return out.reshape(-1)


def planted_w_attention(c, qn, kn):
    """The float64 op with the mistake planted: x * scale * w instead of
    x * scale * (1 + w). Only the tests below use it, to show they catch it."""
    assert np.all(qn == kn)
    return plain_rms_attention(c, weight=np.asarray(qn, np.float64))


# ------------------------------------------------------------------ oracle

@pytest.mark.parametrize("seed", [1, 2])
def test_oracle_weights_minus_one_give_the_uniform_average(oracle_lib, seed):
    c = make_case(seed)
    w = np.full(c["hd"], -1.0, np.float32)
    got = run_oracle(c, w, w)
    assert np.abs(got - uniform_average(c)).max() <= 1e-6


@pytest.mark.parametrize("seed", [3, 4])
def test_oracle_weights_zero_give_plain_rms_attention(oracle_lib, seed):
    c = make_case(seed)
    z = np.zeros(c["hd"], np.float32)
    got = run_oracle(c, z, z)
    assert np.abs(got - plain_rms_attention(c)).max() <= TOL


def test_oracle_query_scale_invariance(oracle_lib):
    base = make_case(5)
    big = make_case(5, scale_q=3.0)
    rng = np.random.default_rng(55)
    qn = (rng.standard_normal(base["hd"]) * 0.1).astype(np.float32)
    kn = (rng.standard_normal(base["hd"]) * 0.1).astype(np.float32)
    a, b = run_oracle(base, qn, kn), run_oracle(big, qn, kn)
    assert np.abs(a - b).max() <= TOL


def test_planted_w_for_one_plus_w_fails_both_closed_forms():
    """With w in place of (1 + w): at w = -1 the normalized q and k become -q
    and -k (scores unchanged, not 0), at w = 0 they become 0 (a uniform
    average, not attention). Both closed forms reject it."""
    c = make_case(6)
    m1 = np.full(c["hd"], -1.0, np.float32)
    z = np.zeros(c["hd"], np.float32)
    assert np.abs(planted_w_attention(c, m1, m1) - uniform_average(c)).max() > 1e-2
    assert np.abs(planted_w_attention(c, z, z) - plain_rms_attention(c)).max() > 1e-2


# ------------------------------------------------------------------ GPU

# hd 64 (the general f32 kernel), hd 256 at one short row (the fused
# kernel) and at L 1040 (65 query tiles x 8 heads: the K prep and the
# split-head kernel).
GPU_SHAPES = [dict(hd=64, rot=32, L=48), dict(hd=256, rot=64, L=64, H=8, KV=2),
              dict(hd=256, rot=64, L=1040, H=8, KV=2)]


@pytest.mark.gpu
@pytest.mark.parametrize("shape", range(len(GPU_SHAPES)))
def test_gpu_weights_minus_one_give_the_uniform_average(gpu_ctx, shape):
    c = make_case(11 + shape, **GPU_SHAPES[shape])
    print(f"[closed form] w = -1, {GPU_SHAPES[shape]}", flush=True)
    w = np.full(c["hd"], -1.0, np.float32)
    assert np.abs(run_gpu(c, w, w, gpu_ctx) - uniform_average(c)).max() <= TOL


@pytest.mark.gpu
@pytest.mark.parametrize("shape", range(len(GPU_SHAPES)))
def test_gpu_weights_zero_give_plain_rms_attention(gpu_ctx, shape):
    c = make_case(21 + shape, **GPU_SHAPES[shape])
    print(f"[closed form] w = 0, {GPU_SHAPES[shape]}", flush=True)
    z = np.zeros(c["hd"], np.float32)
    assert np.abs(run_gpu(c, z, z, gpu_ctx) - plain_rms_attention(c)).max() <= TOL


@pytest.mark.gpu
@pytest.mark.parametrize("shape", range(len(GPU_SHAPES)))
def test_gpu_query_scale_invariance(gpu_ctx, shape):
    base = make_case(31 + shape, **GPU_SHAPES[shape])
    big = make_case(31 + shape, scale_q=3.0, **GPU_SHAPES[shape])
    rng = np.random.default_rng(77)
    qn = (rng.standard_normal(base["hd"]) * 0.1).astype(np.float32)
    kn = (rng.standard_normal(base["hd"]) * 0.1).astype(np.float32)
    print(f"[closed form] q x 3, {GPU_SHAPES[shape]}", flush=True)
    a, b = run_gpu(base, qn, kn, gpu_ctx), run_gpu(big, qn, kn, gpu_ctx)
    assert np.abs(a - b).max() <= TOL
