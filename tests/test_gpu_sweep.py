"""Seeded random sweep of both drop-in ops against the oracle on the GPU.

Each case draws its own shape and mask from a seed (printed before it runs):
Laya head dims 2..128 (even), 1-6 heads, L 1..300, B 1..3, keep tensors that
are dense, padded, windowed or sparse (some queries keep nothing), RoPE on
or off, both entries (keep tensor and, for build_mask-shaped masks, the
structured one); Jeff head dims 4..256, GQA ratios 1..8, rotary widths
0..head_dim, L 1..200, 1-3 rows with left padding and interior holes, trim on
and off; the bf16 rows entry on the same draws (1e-2); both layer entries at
random shapes. f32 tolerance 2e-5 (north star), equal non-finite positions.
"""
import numpy as np
import pytest

import oracle
import tenferro_ext as te

TOL = 2e-5


def assert_close(got, want, what):
    got = np.asarray(got, np.float32).reshape(-1)
    want = np.asarray(want, np.float32).reshape(-1)
    assert np.array_equal(np.isnan(got), np.isnan(want)), f"{what}: NaN positions differ"
    assert np.array_equal(np.isinf(got), np.isinf(want)), f"{what}: inf positions differ"
    ok = np.isfinite(want)
    if ok.any():
        err = float(np.abs(got[ok] - want[ok]).max())
        assert err <= TOL, f"{what}: max abs error {err}"


def laya_case(seed):
    rng = np.random.default_rng(seed)
    hd = int(rng.choice([2, 4, 8, 16, 24, 32, 48, 64, 96, 128]))
    H = int(rng.integers(1, 7 if hd <= 64 else 3))
    L = int(rng.choice([1, 2, 3, 5, 17, 31, 32, 33, 64, 65, 100, 129, 200, 257, 300]))
    B = int(rng.integers(1, 4))
    d = hd * H
    rope = float(rng.choice([0.0, 10000.0, 160000.0]))
    kind = rng.choice(["dense", "padded", "window", "sparse"])
    valid = np.ones(L * B, np.uint8)
    window = -1
    if kind in ("padded", "window"):
        for b in range(B):
            n = int(rng.integers(1, L + 1))
            valid[b * L + n:(b + 1) * L] = 0
        if kind == "window":
            window = int(rng.integers(0, max(1, L // 2) + 1))
    if kind == "sparse":
        keep = (rng.random(L * L * B) < rng.choice([0.05, 0.3, 0.7])).astype(np.uint8)
    else:
        keep = oracle.laya_build_mask(valid, L, B, window)
    qkv = rng.standard_normal(3 * d * L * B).astype(np.float32)
    return dict(hd=hd, H=H, L=L, B=B, d=d, rope=rope, kind=str(kind), valid=valid,
                window=window, keep=keep, qkv=qkv)


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(1000, 1048))
def test_laya_sweep_gpu(gpu_ctx, oracle_lib, seed):
    c = laya_case(seed)
    print(f"[sweep] laya seed {seed}: hd {c['hd']} H {c['H']} L {c['L']} B {c['B']} "
          f"{c['kind']} window {c['window']} rope {c['rope']}", flush=True)
    want = oracle.laya_attention_block(c["qkv"], c["keep"], c["d"], c["H"], c["L"], c["B"],
                                       c["rope"])
    got = te.laya_attention_block(c["qkv"], c["keep"], c["d"], c["H"], c["rope"],
                                  qkv_shape=(3 * c["d"], c["L"], c["B"]), ctx=gpu_ctx)
    assert_close(got, want, "keep entry")
    if c["kind"] != "sparse":
        got_s = te.laya_attention_structured(c["qkv"], c["valid"], c["d"], c["H"], c["L"],
                                             c["B"], c["window"], c["rope"], ctx=gpu_ctx)
        assert_close(got_s, want, "structured entry")


def jeff_case(seed):
    rng = np.random.default_rng(seed)
    hd = int(rng.choice([4, 8, 16, 32, 64, 128, 256]))
    kv = int(rng.choice([1, 2, 3]))
    G = int(rng.choice([1, 2, 3, 4, 8]))
    H = kv * G
    rot = int(rng.choice([0, 2, hd // 4 * 2 if hd >= 4 else 2, hd]))
    rot = min(rot - rot % 2, hd)
    L = int(rng.choice([1, 2, 4, 7, 16, 24, 31, 64, 100, 128, 200]))
    R = int(rng.integers(1, 4))
    W, KW = H * hd, kv * hd
    mask = np.ones(R * L, np.float32)
    for r in range(R):
        lead = int(rng.integers(0, L + 1)) if rng.random() < 0.7 else 0
        mask[r * L:r * L + lead] = 0.0
        if L > 4 and lead < L and rng.random() < 0.4:
            hole = int(rng.integers(lead, L))
            mask[r * L + hole] = 0.0
    g = lambda n, s=1.0: (rng.standard_normal(n) * s).astype(np.float32)
    return dict(hd=hd, kv=kv, H=H, rot=rot, L=L, R=R, q=g(R * L * W), k=g(R * L * KW),
                v=g(R * L * KW), gate=g(R * L * W), qn=g(hd, 0.1), kn=g(hd, 0.1), mask=mask,
                theta=float(rng.choice([1e4, 1e6, 1e7])), eps=1e-6,
                trim=bool(rng.random() < 0.5))


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(2000, 2048))
def test_jeff_sweep_gpu(gpu_ctx, oracle_lib, seed):
    c = jeff_case(seed)
    print(f"[sweep] jeff seed {seed}: hd {c['hd']} H {c['H']} kv {c['kv']} rot {c['rot']} "
          f"L {c['L']} rows {c['R']} trim {c['trim']}", flush=True)
    args = (c["q"], c["k"], c["v"], c["gate"], c["qn"], c["kn"], c["mask"])
    dims = (c["R"], c["L"], c["H"], c["kv"], c["hd"], c["rot"], c["theta"], c["eps"])
    want = oracle.jeff_rows(*args, *dims, trim_leading=c["trim"])
    got = te.jeff_full_attention_rows(*args, *dims, trim_leading=c["trim"], ctx=gpu_ctx)
    assert_close(got, want, "rows entry")


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(3000, 3024))
def test_jeff_bf16_sweep_gpu(gpu_ctx, oracle_lib, seed):
    """bf16 rows: inputs rounded to bf16, compared with the f32 oracle on the
    rounded values (tolerance 1e-2, north star)."""
    c = jeff_case(seed)
    print(f"[sweep] jeff bf16 seed {seed}: hd {c['hd']} H {c['H']} kv {c['kv']} rot {c['rot']} "
          f"L {c['L']} rows {c['R']} trim {c['trim']}", flush=True)
    bits = [te.to_bf16_bits(c[n]) for n in ("q", "k", "v", "gate")]
    rounded = [te.bf16_bits_to_f32(b) for b in bits]
    dims = (c["R"], c["L"], c["H"], c["kv"], c["hd"], c["rot"], c["theta"], c["eps"])
    want = oracle.jeff_rows(*rounded, c["qn"], c["kn"], c["mask"], *dims, trim_leading=c["trim"])
    got = te.jeff_full_attention_rows(*bits, c["qn"], c["kn"], c["mask"], *dims,
                                      trim_leading=c["trim"], bf16=True, ctx=gpu_ctx)
    got = np.asarray(got, np.float32).reshape(-1)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = np.isfinite(want)
    if ok.any():
        err = float(np.abs(got[ok] - want[ok]).max())
        assert err <= 1e-2, f"bf16 rows entry: max abs error {err}"


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(4000, 4012))
def test_layer_sweep_gpu(gpu_ctx, oracle_lib, seed):
    """Both layer entries at random shapes (biases on/off for Laya, GQA for
    Jeff) against the oracle's float32 layers."""
    rng = np.random.default_rng(seed)
    if seed % 2 == 0:
        hd = int(rng.choice([16, 32, 64]))
        H = int(rng.integers(1, 5))
        d, L, B = hd * H, int(rng.choice([7, 32, 65, 128])), int(rng.integers(1, 4))
        print(f"[sweep] laya layer seed {seed}: d {d} H {H} L {L} B {B}", flush=True)
        valid = np.ones(L * B, np.uint8)
        for b in range(B):
            valid[b * L + int(rng.integers(1, L + 1)):(b + 1) * L] = 0
        keep = oracle.laya_build_mask(valid, L, B, int(rng.choice([-1, 4])))
        x = rng.standard_normal(d * L * B).astype(np.float32)
        w_in = (rng.standard_normal(d * 3 * d) / np.sqrt(d)).astype(np.float32)
        w_out = (rng.standard_normal(d * d) / np.sqrt(d)).astype(np.float32)
        bias = rng.random() < 0.5
        b_in = (0.1 * rng.standard_normal(3 * d)).astype(np.float32) if bias else None
        b_out = (0.1 * rng.standard_normal(d)).astype(np.float32) if bias else None
        want = oracle.laya_attention_layer(x, keep, w_in, b_in, w_out, b_out, d, H, L, B, 10000.0)
        got = te.laya_attention_layer(x, keep, w_in, b_in, w_out, b_out, d, H, L, B, 10000.0,
                                      ctx=gpu_ctx)
    else:
        hd = int(rng.choice([16, 64, 256]))
        kv, G = int(rng.choice([1, 2])), int(rng.choice([1, 2, 4]))
        H, hidden = kv * G, int(rng.choice([32, 96, 128]))
        L, R = int(rng.choice([8, 24, 64])), int(rng.integers(1, 4))
        print(f"[sweep] jeff layer seed {seed}: hd {hd} H {H} kv {kv} hidden {hidden} L {L} "
              f"rows {R}", flush=True)
        W, KW = H * hd, kv * hd
        g = lambda n, s: (rng.standard_normal(n) * s).astype(np.float32)
        mask = np.ones(R * L, np.float32)
        for r in range(R):
            mask[r * L:r * L + int(rng.integers(0, L))] = 0.0
        args = (g(R * L * hidden, 1.0), g(hidden * W, hidden ** -0.5), g(hidden * W, hidden ** -0.5),
                g(hidden * KW, hidden ** -0.5), g(hidden * KW, hidden ** -0.5),
                g(W * hidden, W ** -0.5), g(hd, 0.1), g(hd, 0.1), mask)
        dims = (R, L, hidden, H, kv, hd, hd // 4 * 2, 1e6, 1e-6)
        trim = bool(rng.random() < 0.5)
        want = oracle.jeff_layer_rows(*args, *dims, trim_leading=trim)
        got = te.jeff_full_attention_layer_rows(*args, *dims, trim_leading=trim, ctx=gpu_ctx)
    assert_close(got, want, "layer entry")
