"""Seeded random sweep of the bf16 rows entry at head dim 256 (the wide
32x32x16 kernel and its exact pass) against the oracle, at the bf16
tolerance of 1e-2.

The oracle runs the reference arithmetic in f32 on the bf16-valued inputs
(cpu-kernels lib.rs:609-763 through jeff_rows). Each case draws GQA ratio,
rotary width, L (a multiple of 8, so the wide kernel runs), 1-3 rows, masks
with left padding, all-zero rows, sparse rows and interior holes, trim on
and off, q scales 0.5-3, norm weights ~N(0, 0.1^2), and in about one case of
seven a NaN or an infinity in V (the exact pass). Queries that keep only two
or three keys are the worst case for rounding: their output is a convex
combination of a few V values, so every relative error of a probability or
a score shows at the scale of |v_i - v_j|.
"""
import numpy as np
import pytest

import oracle
import tenferro_ext as te

TOL_BF16 = 1e-2  # north star: max abs error <= 1e-2 for the bf16 variant


def wide_case(seed):
    rng = np.random.default_rng(seed)
    hd = 256
    H, kv = [(8, 2), (4, 2), (2, 2), (8, 1), (6, 2), (4, 4), (16, 4), (2, 1)][int(rng.integers(0, 8))]
    rot = int(rng.choice([0, 32, 64, 64, 128, 256]))
    L = 8 * int(rng.integers(1, 90))
    R = int(rng.integers(1, 4))
    W, KW = H * hd, kv * hd
    mask = np.ones(R * L, np.float32)
    for r in range(R):
        u = rng.random()
        if u < 0.4:
            mask[r * L:r * L + int(rng.integers(0, L + 1))] = 0.0
        elif u < 0.5:
            mask[r * L:(r + 1) * L] = 0.0
        elif u < 0.65:
            mask[r * L:(r + 1) * L] = (rng.random(L) < 0.3).astype(np.float32)
        if L > 8 and rng.random() < 0.3:
            mask[r * L + int(rng.integers(0, L))] = 0.0

    def g(n, s=1.0):
        return (rng.standard_normal(n) * s).astype(np.float32)

    q = g(R * L * W, float(rng.choice([0.5, 1.0, 3.0])))
    k, v, gate = g(R * L * KW), g(R * L * KW), g(R * L * W)
    bits = [te.to_bf16_bits(x) for x in (q, k, v, gate)]
    if rng.random() < 0.15:  # a non-finite value: the exact pass
        vb = bits[2].reshape(R, KW, L)
        vb[int(rng.integers(0, R)), int(rng.integers(0, KW)), int(rng.integers(0, L))] = \
            int(rng.choice([0x7F80, 0xFF80, 0x7FC0]))
    return dict(H=H, kv=kv, rot=rot, L=L, R=R, bits=bits, qn=g(hd, 0.1), kn=g(hd, 0.1),
                mask=mask, theta=float(rng.choice([1e4, 1e7])), trim=bool(rng.random() < 0.5))


def run_case(ctx, c):
    vals = [te.bf16_bits_to_f32(b) for b in c["bits"]]
    dims = (c["R"], c["L"], c["H"], c["kv"], 256, c["rot"], c["theta"], 1e-6)
    want = oracle.jeff_rows(*vals, c["qn"], c["kn"], c["mask"], *dims, trim_leading=c["trim"])
    got = te.jeff_full_attention_rows(*c["bits"], c["qn"], c["kn"], c["mask"], *dims,
                                      trim_leading=c["trim"], bf16=True, ctx=ctx)
    return np.asarray(got, np.float32).reshape(-1), np.asarray(want, np.float32).reshape(-1)


def assert_bf16_close(got, want, what):
    assert np.array_equal(np.isnan(got), np.isnan(want)), f"{what}: NaN positions differ"
    assert np.array_equal(np.isinf(got), np.isinf(want)), f"{what}: inf positions differ"
    ok = np.isfinite(want)
    if ok.any():
        err = float(np.abs(got[ok] - want[ok]).max())
        assert err <= TOL_BF16, f"{what}: max abs error {err}"
        return err
    return 0.0


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(50000, 50300))
def test_bf16_wide_sweep_gpu(gpu_ctx, oracle_lib, seed):
    c = wide_case(seed)
    print(f"[bf16 sweep] seed {seed}: L {c['L']} rows {c['R']} H {c['H']} kv {c['kv']} "
          f"rot {c['rot']} trim {c['trim']}", flush=True)
    got, want = run_case(gpu_ctx, c)
    assert_bf16_close(got, want, f"seed {seed}")


@pytest.mark.gpu
@pytest.mark.parametrize("gap", [2, 5, 31, 32, 33, 200])
def test_bf16_two_active_keys_gpu(gpu_ctx, oracle_lib, gap):
    """Rows whose queries keep exactly two keys (`gap` positions apart), V
    ~N(0, 1) as in the sweep, gate 8 (sigmoid ~1, so nothing damps the error):
    the queries most exposed to rounding. With p1 + p2 = 1 the output is
    p1 v1 + p2 v2, and relative errors d1, d2 of the two weights move it by
    about p1 p2 (d1 - d2)(v1 - v2): up to |v1 - v2| / 1024 for bf16
    probabilities, plus p1 p2 |ds| |v1 - v2| for a score error ds."""
    rng = np.random.default_rng(7000 + gap)
    H, kv, hd, L, R = 8, 2, 256, 256, 2
    W, KW = H * hd, kv * hd
    mask = np.zeros(R * L, np.float32)
    for r in range(R):
        a = int(rng.integers(0, L - gap - 1))
        mask[r * L + a] = 1.0
        mask[r * L + a + gap] = 1.0
    q = rng.standard_normal(R * L * W).astype(np.float32)
    k = rng.standard_normal(R * L * KW).astype(np.float32)
    v = rng.standard_normal(R * L * KW).astype(np.float32)
    gate = np.full(R * L * W, 8.0, np.float32)  # sigmoid ~ 1: the error is not damped
    qn = (rng.standard_normal(hd) * 0.02).astype(np.float32)
    kn = (rng.standard_normal(hd) * 0.02).astype(np.float32)
    c = dict(H=H, kv=kv, rot=64, L=L, R=R, bits=[te.to_bf16_bits(x) for x in (q, k, v, gate)],
             qn=qn, kn=kn, mask=mask, theta=1e7, trim=False)
    print(f"[bf16 two keys] gap {gap}", flush=True)
    got, want = run_case(gpu_ctx, c)
    err = assert_bf16_close(got, want, f"two keys, gap {gap}")
    print(f"[bf16 two keys] gap {gap}: max abs error {err:.2e}", flush=True)


@pytest.mark.gpu
def test_bf16_large_norm_weights_gpu(gpu_ctx, oracle_lib):
    """q norm weights with 1 + w = 3e4 and k norm weights with 1 + w = 1/3e4:
    the scores keep their usual size, but the normalized q reaches 16 * 3e4,
    beyond fp16's range, and k sits near its subnormals. The kernels' power-
    of-two operand scaling must keep every score finite and the output within
    the bf16 tolerance."""
    rng = np.random.default_rng(4242)
    H, kv, hd, L, R = 4, 2, 256, 64, 1
    W, KW = H * hd, kv * hd
    q = rng.standard_normal(R * L * W).astype(np.float32)
    k = rng.standard_normal(R * L * KW).astype(np.float32)
    v = rng.standard_normal(R * L * KW).astype(np.float32)
    gate = rng.standard_normal(R * L * W).astype(np.float32)
    qn = np.full(hd, 3.0e4 - 1.0, np.float32)
    kn = np.full(hd, np.float32(1.0 / 3.0e4) - np.float32(1.0), np.float32)
    mask = np.ones(R * L, np.float32)
    c = dict(H=H, kv=kv, rot=64, L=L, R=R, bits=[te.to_bf16_bits(x) for x in (q, k, v, gate)],
             qn=qn, kn=kn, mask=mask, theta=1e7, trim=False)
    print("[bf16 norm weights] 1 + w_q = 3e4, 1 + w_k = 1/3e4", flush=True)
    got, want = run_case(gpu_ctx, c)
    assert np.isfinite(want).all()
    assert np.isfinite(got).all(), "non-finite output from finite inputs"
    assert_bf16_close(got, want, "large norm weights")
