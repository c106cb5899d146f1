"""GPU parity tests: the HIP kernels, called through the C ABI, against the
CPU oracle on identical seeded inputs. Tolerances are the north star's:
max-abs <= 2e-5 for f32, <= 1e-2 for bf16; NaN positions must match exactly.
"""
import os
import sys

import numpy as np
import pytest

import oracle
import tenferro_ext as te
from tenferro_ext.workloads import Lcg, jeff_config, laya_config

pytestmark = pytest.mark.gpu

F32_TOL = 2e-5
BF16_TOL = 1e-2


@pytest.fixture(autouse=True)
def _announce(request):
    print(f"\n[gpu] {request.node.nodeid}", flush=True)
    sys.stdout.flush()
    yield


@pytest.fixture(scope="module", autouse=True)
def _oracle_threads():
    oracle.set_threads(16)


def assert_close(got, want, tol):
    got = np.asarray(got, np.float32).reshape(-1)
    want = np.asarray(want, np.float32).reshape(-1)
    assert got.shape == want.shape
    gn, wn = np.isnan(got), np.isnan(want)
    assert np.array_equal(gn, wn), f"NaN mismatch at {np.nonzero(gn != wn)[0][:10]}"
    ok = ~wn
    err = float(np.abs(got[ok] - want[ok]).max()) if ok.any() else 0.0
    assert err <= tol, f"max abs error {err} > {tol}"
    return err


def encoder_valid(length, batch, sparse):
    valid = np.zeros(length * batch, np.uint8)
    for b in range(batch):
        for l in range(length):
            if sparse:
                v = l == 0 or l == length - 1
            elif length == 1:
                v = True
            elif batch == 1 or b == 0:
                v = l != 1
            else:
                v = l < length - 1
            valid[l + length * b] = v
    return valid


# ------------------------------------------------------------------ Laya

def laya_gpu(ctx, qkv, keep, d, heads, L, B, base):
    return te.laya_attention_block(qkv, keep, d, heads, base, qkv_shape=(3 * d, L, B), ctx=ctx)


def test_laya_c1_matches_oracle(gpu_ctx):
    w = laya_config(1)
    got = laya_gpu(gpu_ctx, w.qkv, w.keep, w.hidden, w.heads, w.length, w.batch, w.rope_base)
    want = oracle.laya_attention_block(w.qkv, w.keep, w.hidden, w.heads, w.length, w.batch, w.rope_base)
    assert_close(got, want, F32_TOL)


def test_kernel_timing_events(gpu_ctx):
    """Timed calls give the same outputs and one positive duration per call."""
    w = laya_config(1)
    j = jeff_config(4, rows=2, length=64)
    gpu_ctx.take_kernel_time()
    gpu_ctx.set_timing(True)
    try:
        got = laya_gpu(gpu_ctx, w.qkv, w.keep, w.hidden, w.heads, w.length, w.batch, w.rope_base)
        gj = te.jeff_full_attention_rows(j.q, j.k, j.v, j.gate, j.q_norm, j.k_norm, j.mask, j.rows,
                                         j.length, j.heads, j.kv_heads, j.head_dim, j.rotary_dim,
                                         j.theta, j.eps, ctx=gpu_ctx)
        ms, launches = gpu_ctx.take_kernel_time()
    finally:
        gpu_ctx.set_timing(False)
    assert launches == 2 and 0.0 < ms < 1000.0
    want = oracle.laya_attention_block(w.qkv, w.keep, w.hidden, w.heads, w.length, w.batch, w.rope_base)
    assert_close(got, want, F32_TOL)
    wj = oracle.jeff_rows(j.q, j.k, j.v, j.gate, j.q_norm, j.k_norm, j.mask, j.rows, j.length,
                          j.heads, j.kv_heads, j.head_dim, j.rotary_dim, j.theta, j.eps)
    assert_close(gj, wj, F32_TOL)


@pytest.mark.parametrize("length", [1, 2, 31, 32, 33, 63, 64, 65, 127, 129, 200])
@pytest.mark.parametrize("hd", [4, 16, 64, 128])
def test_laya_sweep_keep_and_structured(gpu_ctx, length, hd):
    """laya-infer tests/model.rs:338-373 masks (interior hole, padded rows,
    sparse rows) on global (rope 160000) and sliding (rope 10000) layers."""
    heads, batch = 2, 2
    d = heads * hd
    rng = Lcg(1000 + length + hd)
    qkv = (rng.uniform(3 * d * length * batch) * 2.0 - 1.0).astype(np.float32)
    for sparse in (False, True):
        valid = encoder_valid(length, batch, sparse)
        for window, base in ((-1, 160000.0), (1, 10000.0), (64, 10000.0)):
            keep = oracle.laya_build_mask(valid, length, batch, window)
            want = oracle.laya_attention_block(qkv, keep, d, heads, length, batch, base)
            got = laya_gpu(gpu_ctx, qkv, keep, d, heads, length, batch, base)
            assert_close(got, want, F32_TOL)
            st = te.laya_attention_structured(qkv, valid, d, heads, length, batch, window, base,
                                              ctx=gpu_ctx)
            # same tiles, same order: the structured entry is bitwise equal
            assert np.array_equal(np.asarray(st).view(np.uint32), np.asarray(got).view(np.uint32))


@pytest.mark.parametrize("L,B,heads,hd,window", [(516, 1, 4, 64, -1), (256, 2, 8, 64, 40),
                                                 (130, 1, 2, 64, -1), (384, 1, 2, 128, -1),
                                                 (96, 1, 3, 32, 9), (512, 1, 24, 64, -1)])
def test_laya_small_grid_teams(gpu_ctx, L, B, heads, hd, window):
    """Grids of at most one 64-query group per CU take the teams variant (key
    tiles dealt to teams of waves, merged at the end; 32-query workgroups
    where half the CUs suffice). With L % 4 == 0 the kernel packs the keep
    bytes itself (no packing pass): L 516 has a partial last query wave and
    key tile; L 130 takes the packing pass; L 512 x 24 heads (192 groups)
    keeps 64-query workgroups. Random keep patterns with queries
    that keep nothing (NaN rows), against the oracle; the structured entry
    must give the same bits as the keep entry."""
    d = heads * hd
    rng = np.random.default_rng(8800 + L + hd)
    qkv = rng.standard_normal(3 * d * L * B).astype(np.float32)
    keep = (rng.random(L * L * B) < 0.6).astype(np.uint8)
    K = keep.reshape(B, L, L)                  # [b][key][query]
    K[:, :, 3] = 0                             # query 3 keeps nothing: NaN row
    K[:, : L // 3, L - 1] = 0                  # the last query keeps only the later keys
    got = laya_gpu(gpu_ctx, qkv, keep, d, heads, L, B, 160000.0)
    want = oracle.laya_attention_block(qkv, keep, d, heads, L, B, 160000.0)
    assert np.isnan(np.asarray(want)).any()
    assert_close(got, want, F32_TOL)
    valid = np.ones(L * B, np.uint8)
    valid[L - 5:L] = 0                          # padded tail of row 0
    sk = oracle.laya_build_mask(valid, L, B, window)
    st = te.laya_attention_structured(qkv, valid, d, heads, L, B, window, 10000.0, ctx=gpu_ctx)
    kp = laya_gpu(gpu_ctx, qkv, sk, d, heads, L, B, 10000.0)
    assert_close(kp, oracle.laya_attention_block(qkv, sk, d, heads, L, B, 10000.0), F32_TOL)
    assert np.array_equal(np.asarray(st).view(np.uint32), np.asarray(kp).view(np.uint32))


@pytest.mark.parametrize("excluded", [1.0, float("nan"), float("inf"), float("-inf")])
def test_laya_masked_nonfinite_values_and_empty_rows(gpu_ctx, excluded):
    """cpu-kernels lib.rs:1212-1250 on the GPU."""
    length, d = 65, 4
    qkv = np.zeros(3 * d * length, np.float32)
    for key in range(length):
        qkv[3 * d * key + 2 * d:3 * d * key + 3 * d] = np.arange(1, d + 1)
    keep = np.ones(length * length, np.uint8)
    keep[np.arange(length) + length * 32] = 0
    keep[length * np.arange(length)] = 0
    keep[length - 1 + length * np.arange(length)] = 0
    qkv[3 * d * 32 + 2 * d:3 * d * 32 + 3 * d] = excluded
    out = np.asarray(laya_gpu(gpu_ctx, qkv, keep, d, 1, length, 1, 0.0)).reshape(length, d)
    assert np.all(np.isnan(out[0])) and np.all(np.isnan(out[-1]))
    assert np.abs(out[1:-1] - np.arange(1, d + 1)).max() <= 1e-6


def test_laya_kept_nonfinite_value_propagates(gpu_ctx):
    """A kept infinite value reaches the rows that keep it (p > 0)."""
    length, d, heads = 40, 8, 1
    rng = Lcg(5)
    qkv = rng.normal(3 * d * length).astype(np.float32)
    qkv[3 * d * 7 + 2 * d + 3] = np.inf
    keep = np.ones(length * length, np.uint8)
    want = oracle.laya_attention_block(qkv, keep, d, heads, length, 1, 0.0)
    got = laya_gpu(gpu_ctx, qkv, keep, d, heads, length, 1, 0.0)
    g, w = np.asarray(got), want
    assert np.array_equal(np.isinf(g), np.isinf(w))
    fin = np.isfinite(w)
    assert np.abs(g[fin] - w[fin]).max() <= F32_TOL


def assert_same_nonfinite(got, want, tol):
    """NaN, +inf and -inf at the same positions; the finite rest within tol."""
    g = np.asarray(got, np.float32).reshape(-1)
    w = np.asarray(want, np.float32).reshape(-1)
    for pick in (np.isnan, np.isposinf, np.isneginf):
        bad = np.nonzero(pick(g) != pick(w))[0]
        assert bad.size == 0, f"{pick.__name__} mismatch at {bad[:10]}"
    fin = np.isfinite(w)
    if fin.any():
        err = float(np.abs(g[fin] - w[fin]).max())
        assert err <= tol, f"max abs error {err} > {tol}"


# (feature block, token, dim, value): q block 0, k block 1. Tokens sit in
# different key tiles, so the walk meets them part-way through.
_SCORE_CASES = {
    "k_nan_kept": [(1, 70, 3, np.nan)],
    "k_inf_kept": [(1, 100, 0, np.inf)],
    "k_neg_inf_kept": [(1, 45, 5, -np.inf)],
    "k_nan_masked": [(1, 33, 2, np.nan)],
    "q_nan": [(0, 12, 1, np.nan), (0, 140, 7, np.inf)],
    "mixed": [(1, 70, 3, np.nan), (1, 130, 1, np.inf), (0, 5, 0, -np.inf)],
}


@pytest.mark.parametrize("case", sorted(_SCORE_CASES))
@pytest.mark.parametrize("scale", [1.0, 6.0])
def test_laya_nonfinite_scores_mid_walk(gpu_ctx, case, scale):
    """NaN / inf scores met part-way through a key walk (reference softmax:
    a non-finite score weighs 0, a +inf one empties its row, lib.rs:1111-1136),
    with q and k scaled so the running max keeps moving across tiles."""
    length, hd, heads, batch = 160, 16, 2, 1
    d = hd * heads
    rng = Lcg(77)
    qkv = rng.normal(3 * d * length).astype(np.float32).reshape(length, 3 * d)
    qkv[:, :2 * d] *= scale
    for blk, tok, dim, val in _SCORE_CASES[case]:
        for h in range(heads):
            qkv[tok, blk * d + h * hd + dim] = val
    qkv = qkv.reshape(-1)
    keep = np.ones((length, length), np.uint8)   # [key][query]: keep[q + L*key]
    keep[33, :] = 0                               # a masked key every query drops
    keep[:, 150:] = 0                             # queries that keep nothing
    keep[100:, 140:150] = 0
    keep = keep.reshape(-1)
    want = oracle.laya_attention_block(qkv, keep, d, heads, length, batch, 160000.0)
    got = laya_gpu(gpu_ctx, qkv, keep, d, heads, length, batch, 160000.0)
    assert_same_nonfinite(got, want, F32_TOL)


@pytest.mark.parametrize("hd", [32, 64, 128])
def test_laya_running_max_growth(gpu_ctx, hd):
    """Scores that climb tile after tile (keys scaled up along the row), so
    the reference max moves on most tiles of the walk; values unscaled."""
    length, heads, batch = 300, 2, 2
    d = hd * heads
    rng = Lcg(hd)
    qkv = rng.normal(3 * d * length * batch).astype(np.float32).reshape(batch, length, 3 * d)
    ramp = np.linspace(0.2, 4.0, length, dtype=np.float32)[None, :, None]
    qkv[:, :, d:2 * d] *= ramp
    qkv[:, :, :d] *= 2.0
    qkv = qkv.reshape(-1)
    valid = np.ones(length * batch, np.uint8)
    valid[length + 250:] = 0
    keep = oracle.laya_build_mask(valid, length, batch, -1)
    want = oracle.laya_attention_block(qkv, keep, d, heads, length, batch, 160000.0)
    got = laya_gpu(gpu_ctx, qkv, keep, d, heads, length, batch, 160000.0)
    assert_close(got, want, F32_TOL)


def test_laya_heads_not_dividing_writes_zeros(gpu_ctx):
    out = np.full(6 * 4, 7.0, np.float32)
    te.laya_attention_block(np.ones(3 * 6 * 4, np.float32), np.ones(16, np.uint8), 6, 4, 0.0,
                            qkv_shape=(18, 4, 1), ctx=gpu_ctx, out=out)
    assert np.all(out == 0.0)


@pytest.mark.parametrize("cfg", [2, 3])
def test_laya_full_config_device_pointers(gpu_ctx, cfg):
    """C2 (global, padded) and C3 (sliding +-64, L 2048) at full size, device
    pointers, against the oracle; the structured entry must agree bitwise."""
    import torch

    w = laya_config(cfg)
    want = oracle.laya_attention_block(w.qkv, w.keep, w.hidden, w.heads, w.length, w.batch, w.rope_base)
    dev = torch.device("cuda:0")
    qkv = torch.from_numpy(w.qkv).to(dev)
    keep = torch.from_numpy(w.keep).to(dev)
    valid = torch.from_numpy(w.valid).to(dev)
    torch.cuda.synchronize()
    got = te.laya_attention_block(qkv, keep, w.hidden, w.heads, w.rope_base,
                                  qkv_shape=(3 * w.hidden, w.length, w.batch), ctx=gpu_ctx)
    st = te.laya_attention_structured(qkv, valid, w.hidden, w.heads, w.length, w.batch, w.window,
                                      w.rope_base, ctx=gpu_ctx)
    err = assert_close(got.cpu().numpy(), want, F32_TOL)
    print(f"C{cfg} max abs error {err:.3e}")
    assert torch.equal(got, st)


# (batch, heads, hd, window): grids of 256 (one round per CU slot), 512 and
# 1024 workgroups at hd 64, 512 at hd 128, 1024 at hd 32, and a sliding
# window (per-group spans differ from the row's).
PLANNED_GRIDS = [(8, 4, 64, -1), (4, 16, 64, -1), (8, 16, 64, 64), (8, 8, 128, -1), (2, 64, 32, -1)]


@pytest.mark.parametrize("batch,heads,hd,window", PLANNED_GRIDS)
def test_laya_planned_grids(gpu_ctx, batch, heads, hd, window):
    """Grids that fit one dispatch round follow a placement plan that each
    workgroup derives from the tile map (rows longest first over the CUs of
    each XCD). Ragged rows with an empty row and an interior hole; each shape
    runs twice, after another planned shape. The drop-in (plan from the keep
    tensor's tile map) must equal the structured entry (plan from the tile
    map of valid + window, the same map) bitwise, and the oracle within
    tolerance on the first shape."""
    import torch

    L = 512
    d = heads * hd
    rng = Lcg(900 + batch * heads + hd)
    valid = np.zeros(L * batch, np.uint8)
    for b in range(batch):
        n = 0 if b == 1 else int(rng.uniform(1)[0] * (L - 64)) + 64
        valid[b * L:b * L + n] = 1
    valid[L // 3] = 0  # a hole in row 0
    qkv = (rng.uniform(3 * d * L * batch) * 2.0 - 1.0).astype(np.float32)
    keep = oracle.laya_build_mask(valid, L, batch, window)
    base = 160000.0 if window < 0 else 10000.0
    dev = torch.device("cuda:0")
    tq = torch.from_numpy(qkv).to(dev)
    tk = torch.from_numpy(keep).to(dev)
    tv = torch.from_numpy(valid).to(dev)
    # another planned shape first (the tile map workspace is reused)
    ob, oh, ohd, ow = PLANNED_GRIDS[(PLANNED_GRIDS.index((batch, heads, hd, window)) + 1) % len(PLANNED_GRIDS)]
    od = oh * ohd
    oqkv = torch.zeros(3 * od * L * ob, dtype=torch.float32, device=dev)
    okeep = torch.ones(L * L * ob, dtype=torch.uint8, device=dev)
    te.laya_attention_block(oqkv, okeep, od, oh, 160000.0, qkv_shape=(3 * od, L, ob), ctx=gpu_ctx)
    st = te.laya_attention_structured(tq, tv, d, heads, L, batch, window, base, ctx=gpu_ctx)
    for _ in range(2):
        got = te.laya_attention_block(tq, tk, d, heads, base, qkv_shape=(3 * d, L, batch), ctx=gpu_ctx)
        assert torch.equal(torch.isnan(got), torch.isnan(st))
        assert torch.equal(got.view(torch.int32), st.view(torch.int32))
    if (batch, heads, hd, window) == PLANNED_GRIDS[0]:
        want = oracle.laya_attention_block(qkv, keep, d, heads, L, batch, base)
        assert_close(got.cpu().numpy(), want, F32_TOL)


def _laya_planned(L, heads, batch, hd_pad, cus=256):
    """Mirror of laya_planned (tfd_internal.hpp) for MI355X's 256 CUs."""
    nqb = (L + 63) // 64
    gpc = 4 if hd_pad <= 64 else 2
    xcd = (nqb * heads * batch <= gpc * cus and (heads * nqb) % 8 == 0 and 32 % batch == 0
           and ((heads * nqb) // 8) % (32 // batch) == 0)
    return xcd and nqb * batch <= 1024


# (L, batch, heads, hd, window): one-round grids (so both entries get the
# placement plan) whose length leaves a partial last 64-query group and a
# partial last key tile.
RAGGED_PLANNED = [(200, 32, 2, 64, -1), (200, 32, 2, 64, 16), (72, 32, 4, 32, 8)]


@pytest.mark.parametrize("L,batch,heads,hd,window", RAGGED_PLANNED)
def test_laya_planned_ragged_lengths(gpu_ctx, L, batch, heads, hd, window):
    """The structured entry's prep pass (valid-key words and the tile map of
    valid + window) at lengths that are not multiples of 32 or 64: ragged rows
    with an empty row, a row of one token, an interior hole and padded queries
    inside windows; against the oracle, and the keep entry bitwise."""
    import torch

    assert _laya_planned(L, heads, batch, hd)
    d = heads * hd
    rng = Lcg(1200 + L + window)
    valid = np.zeros(L * batch, np.uint8)
    for b in range(batch):
        n = {0: L, 1: 0, 2: 1}.get(b, int(rng.uniform(1)[0] * L))
        valid[b * L:b * L + n] = 1
    valid[L // 2] = 0  # a hole in row 0
    qkv = (rng.uniform(3 * d * L * batch) * 2.0 - 1.0).astype(np.float32)
    keep = oracle.laya_build_mask(valid, L, batch, window)
    base = 10000.0
    dev = torch.device("cuda:0")
    tq = torch.from_numpy(qkv).to(dev)
    st = te.laya_attention_structured(tq, torch.from_numpy(valid).to(dev), d, heads, L, batch,
                                      window, base, ctx=gpu_ctx)
    got = te.laya_attention_block(tq, torch.from_numpy(keep).to(dev), d, heads, base,
                                  qkv_shape=(3 * d, L, batch), ctx=gpu_ctx)
    assert torch.equal(torch.isnan(got), torch.isnan(st))
    assert torch.equal(got.view(torch.int32), st.view(torch.int32))
    want = oracle.laya_attention_block(qkv, keep, d, heads, L, batch, base)
    err = assert_close(st.cpu().numpy(), want, F32_TOL)
    print(f"L {L} B {batch} H {heads} hd {hd} window {window}: max abs error {err:.3e}")


# ------------------------------------------------------------------ Jeff

def jeff_case(seed, length, heads, hd, kv_heads, holes):
    rng = Lcg(seed)
    W, KW = heads * hd, kv_heads * hd
    q = rng.normal(length * W).astype(np.float32)
    k = rng.normal(length * KW).astype(np.float32)
    v = rng.normal(length * KW).astype(np.float32)
    g = rng.normal(length * W).astype(np.float32)
    qn = (rng.normal(hd) * 0.1).astype(np.float32)
    kn = (rng.normal(hd) * 0.1).astype(np.float32)
    mask = np.ones(length, np.float32)
    if holes and length > 3:
        mask[: length // 4] = 0.0
        mask[length // 2] = 0.0
    return q, k, v, g, qn, kn, mask


@pytest.mark.parametrize("length", [1, 2, 3, 6, 17, 33, 64, 100])
@pytest.mark.parametrize("hd,rot", [(4, 2), (16, 16), (64, 32), (256, 64)])
def test_jeff_dropin_matches_oracle(gpu_ctx, length, hd, rot):
    heads = 2
    for holes in (False, True):
        q, k, v, g, qn, kn, mask = jeff_case(7 * length + hd, length, heads, hd, heads, holes)
        want = oracle.jeff_full_attention(q, k, v, g, qn, kn, mask, length, heads, hd, rot, 1e7, 1e-6)
        got = te.jeff_full_attention(q, k, v, g, qn, kn, mask, heads, hd, rot, 1e7, 1e-6,
                                     q_shape=(length, heads * hd), ctx=gpu_ctx)
        assert_close(got, want, F32_TOL)


@pytest.mark.parametrize("length,hd,heads,kv_heads,rot", [
    (256, 256, 8, 2, 64),   # one C4 row: the split-head path
    (70, 64, 8, 2, 16),     # the general kernel (L % 4 != 0)
    (33, 128, 6, 3, 0),
    (48, 256, 4, 1, 32),
])
def test_jeff_dropin_gqa_flag_matches_oracle(gpu_ctx, length, hd, heads, kv_heads, rot):
    """The drop-in on GQA-expanded K/V (jeff-infer checkpoint.rs:307-319) with
    TFD_KV_HEADS(kv_heads): reads one head per group, results as the oracle on
    the expanded inputs, and bitwise equal to the call that reads every copy."""
    rng = Lcg(1000 + length + hd + heads)
    W, KW = heads * hd, kv_heads * hd
    q = rng.normal(length * W).astype(np.float32)
    g = rng.normal(length * W).astype(np.float32)
    kc = rng.normal(length * KW).astype(np.float32)
    vc = rng.normal(length * KW).astype(np.float32)
    qn = (rng.normal(hd) * 0.1).astype(np.float32)
    kn = (rng.normal(hd) * 0.1).astype(np.float32)
    mask = np.ones(length, np.float32)
    mask[: length // 5] = 0.0       # left padding
    mask[length // 2] = 0.0         # an interior hole
    k = oracle.expand_kv(kc.reshape(KW, length), length, heads, kv_heads, hd).reshape(-1)
    v = oracle.expand_kv(vc.reshape(KW, length), length, heads, kv_heads, hd).reshape(-1)
    want = oracle.jeff_full_attention(q, k, v, g, qn, kn, mask, length, heads, hd, rot, 1e7, 1e-6)
    got = te.jeff_full_attention(q, k, v, g, qn, kn, mask, heads, hd, rot, 1e7, 1e-6,
                                 q_shape=(length, W), ctx=gpu_ctx, kv_heads=kv_heads)
    assert_close(got, want, F32_TOL)
    every = te.jeff_full_attention(q, k, v, g, qn, kn, mask, heads, hd, rot, 1e7, 1e-6,
                                   q_shape=(length, W), ctx=gpu_ctx)
    assert np.array_equal(np.asarray(got).view(np.uint32), np.asarray(every).view(np.uint32))


@pytest.mark.parametrize("heads,kv_heads", [(8, 2), (4, 4), (6, 3), (8, 1), (2, 1)])
def test_jeff_rows_gqa_matches_oracle(gpu_ctx, heads, kv_heads):
    rows, length, hd, rot = 3, 70, 64, 16
    rng = Lcg(heads * 10 + kv_heads)
    W, KW = heads * hd, kv_heads * hd
    q = rng.normal(rows * length * W).astype(np.float32)
    g = rng.normal(rows * length * W).astype(np.float32)
    k = rng.normal(rows * length * KW).astype(np.float32)
    v = rng.normal(rows * length * KW).astype(np.float32)
    qn = (rng.normal(hd) * 0.1).astype(np.float32)
    kn = (rng.normal(hd) * 0.1).astype(np.float32)
    mask = np.ones(rows * length, np.float32)
    mask[length:length + 9] = 0.0     # row 1 left-padded
    mask[2 * length + 30] = 0.0       # row 2 interior hole
    for trim in (False, True):
        want = oracle.jeff_rows(q, k, v, g, qn, kn, mask, rows, length, heads, kv_heads, hd, rot,
                                1e6, 1e-6, trim_leading=trim)
        got = te.jeff_full_attention_rows(q, k, v, g, qn, kn, mask, rows, length, heads, kv_heads,
                                          hd, rot, 1e6, 1e-6, trim_leading=trim, ctx=gpu_ctx)
        assert_close(got, want, F32_TOL)


def test_jeff_masked_nonfinite_values_and_empty_rows(gpu_ctx):
    length, heads, hd = 40, 2, 64
    q, k, v, g, qn, kn, mask = jeff_case(3, length, heads, hd, heads, False)
    mask[:3] = 0.0
    mask[20] = 0.0
    V = v.reshape(heads * hd, length)
    V[:, 20] = np.nan          # masked key: must not leak
    V[5, 1] = np.inf           # masked leading key
    want = oracle.jeff_full_attention(q, k, v, g, qn, kn, mask, length, heads, hd, 32, 1e7, 1e-6)
    got = te.jeff_full_attention(q, k, v, g, qn, kn, mask, heads, hd, 32, 1e7, 1e-6,
                                 q_shape=(length, heads * hd), ctx=gpu_ctx)
    assert np.all(np.isfinite(want))
    assert_close(got, want, F32_TOL)
    out = np.asarray(got).reshape(heads * hd, length)
    assert np.all(out[:, :3] == 0.0)  # no active key at or before these queries


@pytest.mark.parametrize("rows,length,hd", [(5, 256, 256), (1, 64, 256), (2, 48, 64)])
def test_jeff_nonfinite_gates(gpu_ctx, rows, length, hd):
    """NaN, +inf and -inf gates, on queries that keep keys and on left-padded
    query tiles that keep none: out = o * sigmoid(gate), so a padded query
    gives 0 for every gate but NaN (sigmoid(+-inf) is 1 or 0), and a live one
    gives o, 0 or NaN. Shapes: 5 x 256 rows at hd 256 (640 query tiles: the K
    prep and split-head kernels), one short row at hd 256 (the fused kernel),
    hd 64 (the general kernel)."""
    heads, kv = 8, 2
    rng = np.random.default_rng(9100 + length)
    W, KW = heads * hd, kv * hd
    q = rng.standard_normal(rows * length * W).astype(np.float32)
    k = rng.standard_normal(rows * length * KW).astype(np.float32)
    v = rng.standard_normal(rows * length * KW).astype(np.float32)
    g = rng.standard_normal(rows * length * W).astype(np.float32)
    qn = (rng.standard_normal(hd) * 0.1).astype(np.float32)
    kn = (rng.standard_normal(hd) * 0.1).astype(np.float32)
    mask = np.ones(rows * length, np.float32)
    G = g.reshape(rows, W, length)
    for r in range(rows):
        first = min(length - 8, 16 + 7 * r)
        mask[r * length:r * length + first] = 0.0          # whole padded query tiles
        for j, val in enumerate((np.nan, np.inf, -np.inf)):
            G[r, (37 * j + 5 * r) % W, (3 * j + r) % first] = val      # padded queries
            G[r, (53 * j + 11 * r) % W, first + (5 * j + r) % (length - first)] = val  # live
    for trim in (False, True):
        want = oracle.jeff_rows(q, k, v, g, qn, kn, mask, rows, length, heads, kv, hd, 64,
                                1e7, 1e-6, trim_leading=trim)
        got = te.jeff_full_attention_rows(q, k, v, g, qn, kn, mask, rows, length, heads, kv, hd,
                                          64, 1e7, 1e-6, trim_leading=trim, ctx=gpu_ctx)
        assert np.isnan(want).sum() >= rows, "the case has NaN outputs"
        assert_close(got, want, F32_TOL)


@pytest.mark.parametrize("hd,length", [(16, 50), (256, 50), (256, 52)])
def test_jeff_kept_nonfinite_values_propagate(gpu_ctx, hd, length):
    """Kept inf / NaN values reach exactly the outputs whose p is non-zero."""
    heads = 2
    q, k, v, g, qn, kn, mask = jeff_case(9, length, heads, hd, heads, False)
    mask[:4] = 0.0
    V = v.reshape(heads * hd, length)
    V[3, 10] = np.inf
    V[3, 20] = -np.inf      # +inf and -inf both kept from query 20 on: NaN
    V[hd + 1, 30] = np.nan
    V[5, 2] = np.nan        # masked: must not leak
    want = oracle.jeff_full_attention(q, k, v, g, qn, kn, mask, length, heads, hd, 8, 1e4, 1e-6)
    got = np.asarray(te.jeff_full_attention(q, k, v, g, qn, kn, mask, heads, hd, 8, 1e4, 1e-6,
                                            q_shape=(length, heads * hd), ctx=gpu_ctx))
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(np.isposinf(got), np.isposinf(want))
    assert np.array_equal(np.isneginf(got), np.isneginf(want))
    fin = np.isfinite(want)
    assert np.abs(got[fin] - want[fin]).max() <= F32_TOL


@pytest.mark.parametrize("length", [4, 16, 20, 48, 68, 132, 256])
def test_jeff_split_head_rows_match_oracle(gpu_ctx, length):
    """hd 256 with L % 4 == 0 (the split-head kernel): GQA rows with left
    padding, an interior hole and a fully padded row, with and without
    trimming."""
    rows, heads, kv, hd, rot = 3, 4, 2, 256, 64
    rng = Lcg(length + 1000)
    W, KW = heads * hd, kv * hd
    q = rng.normal(rows * length * W).astype(np.float32)
    g = rng.normal(rows * length * W).astype(np.float32)
    k = rng.normal(rows * length * KW).astype(np.float32)
    v = rng.normal(rows * length * KW).astype(np.float32)
    qn = (rng.normal(hd) * 0.1).astype(np.float32)
    kn = (rng.normal(hd) * 0.1).astype(np.float32)
    mask = np.ones(rows * length, np.float32)
    mask[length // 2] = 0.0                        # row 0: interior hole
    mask[length:length + length // 3 + 1] = 0.0    # row 1: left padding
    mask[2 * length:] = 0.0                        # row 2: nothing active
    for trim in (False, True):
        want = oracle.jeff_rows(q, k, v, g, qn, kn, mask, rows, length, heads, kv, hd, rot,
                                1e7, 1e-6, trim_leading=trim)
        got = te.jeff_full_attention_rows(q, k, v, g, qn, kn, mask, rows, length, heads, kv, hd,
                                          rot, 1e7, 1e-6, trim_leading=trim, ctx=gpu_ctx)
        assert_close(got, want, F32_TOL)


@pytest.mark.parametrize("where", ["k_nan", "k_inf", "q_nan"])
def test_jeff_split_head_nonfinite_scores(gpu_ctx, where):
    """NaN / inf scores on the split-head kernel's path (hd 256, L % 4 == 0)
    match the reference's NaN / inf pattern and finite values."""
    length, heads, hd = 52, 2, 256
    q, k, v, g, qn, kn, mask = jeff_case(11, length, heads, hd, heads, False)
    mask[:3] = 0.0
    K = k.reshape(heads * hd, length)
    Q = q.reshape(heads * hd, length)
    if where == "k_nan":
        K[7, 20] = np.nan      # kept from query 20 on
        K[9, 1] = np.nan       # masked key: must not leak
    elif where == "k_inf":
        K[hd + 3, 30] = np.inf
    else:
        Q[5, 40] = np.nan
    want = oracle.jeff_full_attention(q, k, v, g, qn, kn, mask, length, heads, hd, 64, 1e7, 1e-6)
    got = np.asarray(te.jeff_full_attention(q, k, v, g, qn, kn, mask, heads, hd, 64, 1e7, 1e-6,
                                            q_shape=(length, heads * hd), ctx=gpu_ctx))
    assert_same_nonfinite(got, want, F32_TOL)


def test_jeff_c4_full_gqa_and_dropin(gpu_ctx):
    """C4 at full size: GQA rows entry (k/v at kv width) and the drop-in op
    row by row on expanded K/V, both against the oracle."""
    import torch

    w = jeff_config(4)
    want = oracle.jeff_rows(w.q, w.k, w.v, w.gate, w.q_norm, w.k_norm, w.mask, w.rows, w.length,
                            w.heads, w.kv_heads, w.head_dim, w.rotary_dim, w.theta, w.eps)
    dev = torch.device("cuda:0")
    t = {n: torch.from_numpy(getattr(w, n)).to(dev) for n in ("q", "k", "v", "gate", "q_norm", "k_norm", "mask")}
    torch.cuda.synchronize()
    got = te.jeff_full_attention_rows(t["q"], t["k"], t["v"], t["gate"], t["q_norm"], t["k_norm"],
                                      t["mask"], w.rows, w.length, w.heads, w.kv_heads, w.head_dim,
                                      w.rotary_dim, w.theta, w.eps, ctx=gpu_ctx)
    err = assert_close(got.cpu().numpy(), want, F32_TOL)
    print(f"C4 rows max abs error {err:.3e}")
    L, W, KW = w.length, w.heads * w.head_dim, w.kv_heads * w.head_dim
    for r in (0, w.rows - 1):
        ke = oracle.expand_kv(w.k[r * L * KW:(r + 1) * L * KW], L, w.heads, w.kv_heads, w.head_dim)
        ve = oracle.expand_kv(w.v[r * L * KW:(r + 1) * L * KW], L, w.heads, w.kv_heads, w.head_dim)
        sl = slice(r * L * W, (r + 1) * L * W)
        one = te.jeff_full_attention(w.q[sl], ke, ve, w.gate[sl], w.q_norm, w.k_norm,
                                     w.mask[r * L:(r + 1) * L], w.heads, w.head_dim, w.rotary_dim,
                                     w.theta, w.eps, q_shape=(L, W), ctx=gpu_ctx)
        assert_close(one, want[sl], F32_TOL)


# ------------------------------------------------------------------ Jeff bf16

def bf16_case(seed, rows, length, heads, kv_heads, hd, holes):
    rng = Lcg(seed)
    W, KW = heads * hd, kv_heads * hd
    q, g = (rng.normal(rows * length * W).astype(np.float32) for _ in range(2))
    k, v = (rng.normal(rows * length * KW).astype(np.float32) for _ in range(2))
    qn = (rng.normal(hd) * 0.1).astype(np.float32)
    kn = (rng.normal(hd) * 0.1).astype(np.float32)
    mask = np.ones(rows * length, np.float32)
    if holes and length > 8:
        mask[: length // 3] = 0.0            # row 0 left-padded
        mask[length + length // 2] = 0.0     # row 1 interior hole
    bits = [te.to_bf16_bits(x) for x in (q, k, v, g)]
    vals = [te.bf16_bits_to_f32(b) for b in bits]
    return bits, vals, qn, kn, mask


@pytest.mark.parametrize("length", [1, 17, 64, 100, 257])
@pytest.mark.parametrize("hd,rot,heads,kv", [(16, 8, 2, 2), (64, 32, 4, 2), (256, 64, 8, 2)])
def test_jeff_bf16_rows_match_oracle(gpu_ctx, length, hd, rot, heads, kv):
    rows = 2
    for trim in (False, True):
        bits, vals, qn, kn, mask = bf16_case(length + hd, rows, length, heads, kv, hd, True)
        want = oracle.jeff_rows(*vals, qn, kn, mask, rows, length, heads, kv, hd, rot, 1e7, 1e-6,
                                trim_leading=trim)
        got = te.jeff_full_attention_rows(*bits, qn, kn, mask, rows, length, heads, kv, hd, rot,
                                          1e7, 1e-6, trim_leading=trim, bf16=True, ctx=gpu_ctx)
        assert_close(got, want, BF16_TOL)


def test_jeff_bf16_kept_nonfinite_values_propagate(gpu_ctx):
    rows, length, heads, kv, hd = 1, 70, 4, 2, 64
    bits, vals, qn, kn, mask = bf16_case(3, rows, length, heads, kv, hd, False)
    Vb = bits[2].reshape(kv * hd, length)
    Vb[7, 12] = 0x7F80   # +inf, kept from query 12 on
    Vb[hd + 2, 40] = 0x7FC0  # NaN
    mask[5] = 0.0
    Vb[9, 5] = 0x7FC0    # masked NaN: must not leak
    vals[2] = te.bf16_bits_to_f32(bits[2])
    want = oracle.jeff_rows(*vals, qn, kn, mask, rows, length, heads, kv, hd, 16, 1e4, 1e-6)
    got = np.asarray(te.jeff_full_attention_rows(*bits, qn, kn, mask, rows, length, heads, kv, hd,
                                                 16, 1e4, 1e-6, bf16=True, ctx=gpu_ctx))
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(np.isinf(got), np.isinf(want))
    fin = np.isfinite(want)
    assert np.abs(got[fin] - want[fin]).max() <= BF16_TOL


# Head dim 256 with L % 8 == 0 runs the 32x32x16 kernel (8 wavefronts in two
# groups, each hw heads of a GQA group x 4/hw blocks of 32 queries); other
# RoPE widths fall back to the 16x16x32 kernel.
@pytest.mark.parametrize("length", [8, 40, 96, 264])
@pytest.mark.parametrize("heads,kv,rot", [(8, 2, 64), (4, 2, 32), (2, 2, 0), (6, 2, 64),
                                          (8, 1, 64), (4, 2, 48)])
def test_jeff_bf16_hd256_rows_match_oracle(gpu_ctx, length, heads, kv, rot):
    rows, hd = 2, 256
    for trim in (False, True):
        bits, vals, qn, kn, mask = bf16_case(7 * length + heads + rot, rows, length, heads, kv, hd,
                                             True)
        want = oracle.jeff_rows(*vals, qn, kn, mask, rows, length, heads, kv, hd, rot, 1e7, 1e-6,
                                trim_leading=trim)
        got = te.jeff_full_attention_rows(*bits, qn, kn, mask, rows, length, heads, kv, hd, rot,
                                          1e7, 1e-6, trim_leading=trim, bf16=True, ctx=gpu_ctx)
        assert_close(got, want, BF16_TOL)


@pytest.mark.parametrize("length", [512, 1024])
def test_jeff_bf16_hd256_paired_prep_blocks(gpu_ctx, length):
    """Lengths whose K prep grid is a multiple of 16 blocks, where the prep
    sends the two 32-key halves of each 128-byte run to one XCD (a block
    permutation): left padding, an interior hole and trimming, against the
    oracle, and bitwise equal to the same call again."""
    rows, heads, kv, hd, rot = 2, 8, 2, 256, 64
    bits, vals, qn, kn, mask = bf16_case(900 + length, rows, length, heads, kv, hd, True)
    mask[length + 37] = 0.0  # row 1: a hole inside a prep block
    for trim in (False, True):
        want = oracle.jeff_rows(*vals, qn, kn, mask, rows, length, heads, kv, hd, rot, 1e7, 1e-6,
                                trim_leading=trim)
        got = te.jeff_full_attention_rows(*bits, qn, kn, mask, rows, length, heads, kv, hd, rot,
                                          1e7, 1e-6, trim_leading=trim, bf16=True, ctx=gpu_ctx)
        assert_close(got, want, BF16_TOL)
        again = te.jeff_full_attention_rows(*bits, qn, kn, mask, rows, length, heads, kv, hd, rot,
                                            1e7, 1e-6, trim_leading=trim, bf16=True, ctx=gpu_ctx)
        assert np.array_equal(np.asarray(got).view(np.uint32), np.asarray(again).view(np.uint32))


def test_jeff_f32_general_prep_paired_blocks(gpu_ctx):
    """The general f32 path (hd 128: K prep + jeff_attention_f32_kernel) at a
    length whose prep grid takes the paired block mapping, with left padding,
    a hole and trimming."""
    rows, length, heads, kv, hd, rot = 2, 512, 4, 2, 128, 32
    rng = Lcg(512 + hd)
    W, KW = heads * hd, kv * hd
    q = rng.normal(rows * length * W).astype(np.float32)
    g = rng.normal(rows * length * W).astype(np.float32)
    k = rng.normal(rows * length * KW).astype(np.float32)
    v = rng.normal(rows * length * KW).astype(np.float32)
    qn = (rng.normal(hd) * 0.1).astype(np.float32)
    kn = (rng.normal(hd) * 0.1).astype(np.float32)
    mask = np.ones(rows * length, np.float32)
    mask[:100] = 0.0                   # row 0 left-padded
    mask[length + 333] = 0.0           # row 1 hole
    for trim in (False, True):
        want = oracle.jeff_rows(q, k, v, g, qn, kn, mask, rows, length, heads, kv, hd, rot,
                                1e7, 1e-6, trim_leading=trim)
        got = te.jeff_full_attention_rows(q, k, v, g, qn, kn, mask, rows, length, heads, kv, hd,
                                          rot, 1e7, 1e-6, trim_leading=trim, ctx=gpu_ctx)
        assert_close(got, want, F32_TOL)


@pytest.mark.parametrize("length", [72, 200])
def test_jeff_bf16_hd256_empty_and_sparse_rows(gpu_ctx, length):
    """Head dim 256, 32x32x16 kernel: a row with no active key (its walk has
    no tiles), a row with one active key mid-row, and a row whose active keys
    start in its last tile, against the oracle with and without trim."""
    rows, heads, kv, hd, rot = 3, 8, 2, 256, 64
    bits, vals, qn, kn, _ = bf16_case(4242 + length, rows, length, heads, kv, hd, False)
    mask = np.zeros(rows * length, np.float32)
    mask[length + length // 2] = 1.0
    mask[2 * length + length - 5:] = 1.0
    for trim in (False, True):
        want = oracle.jeff_rows(*vals, qn, kn, mask, rows, length, heads, kv, hd, rot, 1e7, 1e-6,
                                trim_leading=trim)
        got = te.jeff_full_attention_rows(*bits, qn, kn, mask, rows, length, heads, kv, hd, rot,
                                          1e7, 1e-6, trim_leading=trim, bf16=True, ctx=gpu_ctx)
        assert_close(got, want, BF16_TOL)


def test_jeff_bf16_hd256_nonfinite_takes_exact_pass(gpu_ctx):
    """Head dim 256: tiles with non-finite values are left to the exact
    kernel (flags); a clean call on the same context right after must not see
    stale flags."""
    rows, length, heads, kv, hd, rot = 2, 200, 8, 2, 256, 64
    bits, vals, qn, kn, mask = bf16_case(11, rows, length, heads, kv, hd, False)
    clean = [b.copy() for b in bits]
    Vb = bits[2].reshape(rows, kv * hd, length)
    Vb[0, 7, 12] = 0x7F80        # +inf value, kept from query 12 on
    Vb[1, hd + 2, 150] = 0x7FC0  # NaN value in kv head 1 of row 1
    mask[5] = 0.0
    Vb[0, 9, 5] = 0x7FC0         # masked NaN: must not leak
    Kb = bits[1].reshape(rows, kv * hd, length)
    Kb[1, 3, 90] = 0x7FC0        # NaN key: NaN scores for kv head 0 of row 1
    vals = [te.bf16_bits_to_f32(b) for b in bits]
    want = oracle.jeff_rows(*vals, qn, kn, mask, rows, length, heads, kv, hd, rot, 1e7, 1e-6)
    got = np.asarray(te.jeff_full_attention_rows(*bits, qn, kn, mask, rows, length, heads, kv, hd,
                                                 rot, 1e7, 1e-6, bf16=True, ctx=gpu_ctx))
    assert_same_nonfinite(got, want, BF16_TOL)
    cvals = [te.bf16_bits_to_f32(b) for b in clean]
    want = oracle.jeff_rows(*cvals, qn, kn, mask, rows, length, heads, kv, hd, rot, 1e7, 1e-6)
    got = te.jeff_full_attention_rows(*clean, qn, kn, mask, rows, length, heads, kv, hd, rot, 1e7,
                                      1e-6, bf16=True, ctx=gpu_ctx)
    assert_close(got, want, BF16_TOL)


@pytest.mark.parametrize("align", [0.4, 1.0])
def test_jeff_bf16_hd256_score_growth(gpu_ctx, align):
    """Head dim 256, no RoPE: key 200 points (fraction `align`) where query 230
    of head 0 does, so that query's score there towers over every earlier
    one (normalized rows: about 16 * align against ~N(0, 1)). At align 1 the
    walk's reference would have to move by more than its slack under
    accumulated output and the tile takes the exact pass; at 0.4 it stays in
    the walk."""
    rows, length, heads, kv, hd, rot = 1, 256, 4, 1, 256, 0
    bits, vals, qn, kn, mask = bf16_case(13, rows, length, heads, kv, hd, False)
    q, k, v, g = vals
    Q = q.reshape(heads * hd, length)
    K = k.reshape(kv * hd, length)
    u = Q[:hd, 230] / np.linalg.norm(Q[:hd, 230])
    r = K[:, 17] - np.dot(K[:, 17], u) * u
    r /= np.linalg.norm(r)
    K[:, 200] = (align * u + np.sqrt(1.0 - align * align) * r) * 16.0
    bits = [te.to_bf16_bits(x) for x in (q, k, v, g)]
    vals = [te.bf16_bits_to_f32(b) for b in bits]
    want = oracle.jeff_rows(*vals, qn, kn, mask, rows, length, heads, kv, hd, rot, 1e7, 1e-6)
    got = te.jeff_full_attention_rows(*bits, qn, kn, mask, rows, length, heads, kv, hd, rot, 1e7,
                                      1e-6, bf16=True, ctx=gpu_ctx)
    assert_close(got, want, BF16_TOL)


def test_jeff_c5_reduced_matches_oracle(gpu_ctx):
    """C5 shape (GQA 8/2 x 256, causal, all active) at L 1024 against the oracle."""
    w = jeff_config(5, rows=2, length=1024)
    bits = [te.to_bf16_bits(getattr(w, n)) for n in ("q", "k", "v", "gate")]
    want = oracle.jeff_rows(w.q, w.k, w.v, w.gate, w.q_norm, w.k_norm, w.mask, w.rows, w.length,
                            w.heads, w.kv_heads, w.head_dim, w.rotary_dim, w.theta, w.eps)
    got = te.jeff_full_attention_rows(*bits, w.q_norm, w.k_norm, w.mask, w.rows, w.length,
                                      w.heads, w.kv_heads, w.head_dim, w.rotary_dim, w.theta,
                                      w.eps, bf16=True, ctx=gpu_ctx)
    err = assert_close(got, want, BF16_TOL)
    print(f"C5 (L 1024) bf16 max abs error vs oracle {err:.3e}")


@pytest.fixture(scope="module")
def c5_full():
    """C5 at full size (2 rows x 8192, GQA 8/2 x 256, causal, all active) and
    the oracle's output on its bf16-valued inputs, computed on every host
    core the process may use (about 10-20 s)."""
    w = jeff_config(5)
    threads = oracle.get_threads()
    oracle.set_threads(len(os.sched_getaffinity(0)))
    try:
        print(f"[c5] oracle on 2 x 8192 with {oracle.get_threads()} threads", flush=True)
        want = oracle.jeff_rows(w.q, w.k, w.v, w.gate, w.q_norm, w.k_norm, w.mask, w.rows,
                                w.length, w.heads, w.kv_heads, w.head_dim, w.rotary_dim, w.theta,
                                w.eps)
    finally:
        oracle.set_threads(threads)
    return w, want


def _c5_device_inputs(w):
    import torch

    dev = torch.device("cuda:0")
    bits = [torch.from_numpy(te.to_bf16_bits(getattr(w, n)).view(np.int16)).to(dev)
            for n in ("q", "k", "v", "gate")]
    vals = [torch.from_numpy(getattr(w, n)).to(dev) for n in ("q", "k", "v", "gate")]
    rest = [torch.from_numpy(getattr(w, n)).to(dev) for n in ("q_norm", "k_norm", "mask")]
    args = (w.rows, w.length, w.heads, w.kv_heads, w.head_dim, w.rotary_dim, w.theta, w.eps)
    return bits, vals, rest, args


def test_jeff_c5_full_bf16_matches_oracle(gpu_ctx, c5_full):
    """C5 at its workload size: the bf16 kernel (512 query tiles per row, walks
    of up to 8192 keys) against the oracle (cpu-kernels lib.rs:609-763
    restated) on the same bf16-valued inputs, north_star tolerance 1e-2."""
    w, want = c5_full
    bits, _vals, rest, args = _c5_device_inputs(w)
    got = te.jeff_full_attention_rows(*bits, *rest, *args, bf16=True, ctx=gpu_ctx)
    err = assert_close(got.cpu().numpy(), want, BF16_TOL)
    print(f"C5 full (2 x 8192) bf16 max abs error vs oracle {err:.3e}")


def test_jeff_c5_full_f32_matches_oracle(gpu_ctx, c5_full):
    """The f32 hd-256 path at C5's size (L 8192) against the oracle on the same
    values: f32 tolerance 2e-5."""
    w, want = c5_full
    _bits, vals, rest, args = _c5_device_inputs(w)
    got = te.jeff_full_attention_rows(*vals, *rest, *args, ctx=gpu_ctx)
    err = assert_close(got.cpu().numpy(), want, F32_TOL)
    print(f"C5 full (2 x 8192) f32 max abs error vs oracle {err:.3e}")


def test_jeff_c5_full_bf16_matches_f32_gpu(gpu_ctx, c5_full):
    """The bf16 kernel against the f32 kernel at full C5 size (an extra
    comparison beside the oracle's)."""
    w, _want = c5_full
    bits, vals, rest, args = _c5_device_inputs(w)
    got = te.jeff_full_attention_rows(*bits, *rest, *args, bf16=True, ctx=gpu_ctx)
    ref = te.jeff_full_attention_rows(*vals, *rest, *args, ctx=gpu_ctx)
    err = assert_close(got.cpu().numpy(), ref.cpu().numpy(), BF16_TOL)
    print(f"C5 full bf16 vs f32 max abs error {err:.3e}")


# ------------------------------------------------------------------ head dims past the tiles

@pytest.mark.parametrize("hd,heads,length,batch", [(160, 2, 40, 2), (256, 1, 70, 1), (129, 2, 33, 2),
                                                    (512, 2, 20, 1)])
def test_laya_wide_head_dims_match_oracle(gpu_ctx, hd, heads, length, batch):
    """Head dims past 128 (the reference computes any head dim,
    cpu-kernels lib.rs:843-1156): global and windowed masks with padded and
    sparse rows, RoPE on and off, both entries, against the oracle."""
    d = heads * hd
    rng = Lcg(5000 + hd + length)
    qkv = (rng.uniform(3 * d * length * batch) * 2.0 - 1.0).astype(np.float32)
    for sparse in (False, True):
        valid = encoder_valid(length, batch, sparse)
        for window, base in ((-1, 160000.0), (4, 10000.0), (-1, 0.0)):
            keep = oracle.laya_build_mask(valid, length, batch, window)
            want = oracle.laya_attention_block(qkv, keep, d, heads, length, batch, base)
            got = laya_gpu(gpu_ctx, qkv, keep, d, heads, length, batch, base)
            assert_close(got, want, F32_TOL)
            st = te.laya_attention_structured(qkv, valid, d, heads, length, batch, window, base,
                                              ctx=gpu_ctx)
            assert_close(st, want, F32_TOL)


@pytest.mark.parametrize("hd,heads,kv_heads,rot,length", [(320, 4, 2, 64, 50), (512, 2, 1, 0, 33),
                                                          (288, 3, 3, 288, 17)])
def test_jeff_wide_head_dims_match_oracle(gpu_ctx, hd, heads, kv_heads, rot, length):
    """Head dims past 256 (jeff_full_attention_into takes any head dim,
    lib.rs:609-763): rows with left padding and holes, GQA, trim on and off,
    f32 and bf16, against the oracle."""
    rows = 2
    rng = Lcg(7000 + hd + length)
    W, KW = heads * hd, kv_heads * hd
    q = rng.normal(rows * length * W).astype(np.float32)
    g = rng.normal(rows * length * W).astype(np.float32)
    k = rng.normal(rows * length * KW).astype(np.float32)
    v = rng.normal(rows * length * KW).astype(np.float32)
    qn = (rng.normal(hd) * 0.1).astype(np.float32)
    kn = (rng.normal(hd) * 0.1).astype(np.float32)
    mask = np.ones(rows * length, np.float32)
    mask[length:length + length // 3] = 0.0
    mask[length // 2] = 0.0
    for trim in (False, True):
        want = oracle.jeff_rows(q, k, v, g, qn, kn, mask, rows, length, heads, kv_heads, hd, rot,
                                1e7, 1e-6, trim_leading=trim)
        got = te.jeff_full_attention_rows(q, k, v, g, qn, kn, mask, rows, length, heads, kv_heads,
                                          hd, rot, 1e7, 1e-6, trim_leading=trim, ctx=gpu_ctx)
        assert_close(got, want, F32_TOL)
    bits = [te.to_bf16_bits(x) for x in (q, k, v, g)]
    vals = [te.bf16_bits_to_f32(b) for b in bits]
    want = oracle.jeff_rows(*vals, qn, kn, mask, rows, length, heads, kv_heads, hd, rot, 1e7, 1e-6)
    got = te.jeff_full_attention_rows(*bits, qn, kn, mask, rows, length, heads, kv_heads, hd, rot,
                                      1e7, 1e-6, bf16=True, ctx=gpu_ctx)
    assert_close(got, want, BF16_TOL)
    if kv_heads == heads:  # the drop-in, one row
        q0, k0, v0, g0 = (x[: length * W] for x in (q, k, v, g))
        want = oracle.jeff_full_attention(q0, k0, v0, g0, qn, kn, mask[:length], length, heads, hd,
                                          rot, 1e7, 1e-6)
        got = te.jeff_full_attention(q0, k0, v0, g0, qn, kn, mask[:length], heads, hd, rot, 1e7,
                                     1e-6, q_shape=(length, W), ctx=gpu_ctx)
        assert_close(got, want, F32_TOL)
