"""Whole attention layers (the projections around the fused ops).

CPU: the layer entries validate their arguments before touching a GPU, and
the oracle's layers (numpy float32 GEMMs around the C restatement) agree with
float64 brute force of the same layers (laya-infer model.rs:1304-1347,
jeff-infer model.rs:686-780); a transposed weight is caught. GPU: the layer
entries (rocBLAS GEMMs + the HIP attention kernels) against the oracle,
max-abs <= 2e-5 with equal NaN positions, on host and device pointers.
"""
import numpy as np
import pytest

import oracle
import tenferro_ext as te
from oracle import brute
from tenferro_ext.workloads import jeff_layer_config, laya_layer_config

F32_TOL = 2e-5


def expand_cols(w, hidden, heads, kv_heads, hd):
    """GQA expansion of a (hidden, kv_heads*hd) column-major projection to
    every query head (jeff-infer checkpoint.rs:307-319)."""
    m = np.asarray(w, np.float32).reshape(kv_heads * hd, hidden)
    g = heads // kv_heads
    return np.concatenate([m[(h // g) * hd:(h // g + 1) * hd] for h in range(heads)]).reshape(-1)


def jeff_brute_rows(j):
    out = []
    for r in range(j.rows):
        sl = slice(r * j.length * j.hidden, (r + 1) * j.length * j.hidden)
        out.append(brute.jeff_layer_host(
            j.x[sl], j.w_q, j.w_gate,
            expand_cols(j.w_k, j.hidden, j.heads, j.kv_heads, j.head_dim),
            expand_cols(j.w_v, j.hidden, j.heads, j.kv_heads, j.head_dim), j.w_o, j.q_norm,
            j.k_norm, j.mask[r * j.length:(r + 1) * j.length], j.length, j.hidden, j.heads,
            j.head_dim, j.rotary_dim, j.theta, j.eps))
    return np.concatenate(out)


def laya_padded_layer():
    """d 32, 2 heads x 16, L 40, B 2, window +-4, row 1 padded after 23
    tokens, biases on both linears."""
    from tenferro_ext.workloads import Lcg

    d, H, L, B = 32, 2, 40, 2
    rng = Lcg(211)
    valid = np.zeros(L * B, np.uint8)
    valid[:L] = 1
    valid[L:L + 23] = 1
    keep = oracle.laya_build_mask(valid, L, B, 4)
    x = rng.normal(d * L * B).astype(np.float32)
    w_in = (rng.normal(d * 3 * d) * 0.2).astype(np.float32)
    w_out = (rng.normal(d * d) * 0.2).astype(np.float32)
    b_in = (rng.normal(3 * d) * 0.1).astype(np.float32)
    b_out = (rng.normal(d) * 0.1).astype(np.float32)
    return dict(x=x, keep=keep, w_in=w_in, b_in=b_in, w_out=w_out, b_out=b_out, hidden=d,
                heads=H, length=L, batch=B, rope_base=10000.0)


# ------------------------------------------------------------------ CPU


def test_layer_entries_validate_before_gpu(oracle_lib):
    ctx = te.Context(0)
    f = np.zeros(64, np.float32)
    p = f.ctypes.data
    rc = ctx._lib.tfd_jeff_full_attention_layer_rows_f32(ctx.handle, 1, 2, 8, 3, 2, 4, 4, p, p, p,
                                                        p, p, p, p, p, p, 0, 0, p, 0)
    assert rc == te.TFD_EINVAL and "kv_heads" in ctx._lib.tfd_last_error(ctx.handle).decode()
    rc = ctx._lib.tfd_laya_attention_layer_f32(ctx.handle, p, 8, 2, 2, 1, p, p, None, p, None, 0,
                                               p, te.TFD_ASYNC)
    assert rc == te.TFD_EINVAL and "TFD_ASYNC" in ctx._lib.tfd_last_error(ctx.handle).decode()
    rc = ctx._lib.tfd_laya_attention_layer_f32(ctx.handle, None, 8, 2, 2, 1, p, p, None, p, None,
                                               0, p, 0)
    assert rc == te.TFD_EINVAL and "null buffer" in ctx._lib.tfd_last_error(ctx.handle).decode()
    ctx.close()


@pytest.mark.parametrize("case", ["c1_bias", "padded"])
def test_laya_layer_oracle_matches_brute(oracle_lib, case):
    if case == "c1_bias":
        w = laya_layer_config(1, bias=True)
        c = dict(x=w.x, keep=w.keep, w_in=w.w_in, b_in=w.b_in, w_out=w.w_out, b_out=w.b_out,
                 hidden=w.hidden, heads=w.heads, length=w.length, batch=w.batch,
                 rope_base=w.rope_base)
    else:
        c = laya_padded_layer()
    got = oracle_lib.laya_attention_layer(**c)
    want = brute.laya_attention_layer_host(**c)
    assert np.abs(got - want).max() <= F32_TOL
    # teeth: the same layer with W_in read transposed is far off
    d = c["hidden"]
    wt = np.asarray(c["w_in"]).reshape(3 * d, d)
    bad = dict(c, w_in=np.ascontiguousarray(np.tile(wt[:d].T, (1, 3))).reshape(-1))
    assert np.abs(brute.laya_attention_layer_host(**bad) - want).max() > 1e-2


def test_jeff_layer_oracle_matches_brute(oracle_lib):
    j = jeff_layer_config(4, rows=2, length=24, hidden=64)
    got = oracle_lib.jeff_layer_rows(j.x, j.w_q, j.w_gate, j.w_k, j.w_v, j.w_o, j.q_norm, j.k_norm,
                                     j.mask, j.rows, j.length, j.hidden, j.heads, j.kv_heads,
                                     j.head_dim, j.rotary_dim, j.theta, j.eps)
    assert np.abs(got - jeff_brute_rows(j)).max() <= F32_TOL


# ------------------------------------------------------------------ GPU


def assert_close(got, want, tol=F32_TOL):
    got = np.asarray(got, np.float32).reshape(-1)
    want = np.asarray(want, np.float32).reshape(-1)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    err = float(np.abs(got[ok] - want[ok]).max())
    assert err <= tol, f"max abs error {err} > {tol}"
    return err


@pytest.mark.gpu
@pytest.mark.parametrize("case", ["c1_bias", "padded", "c2"])
def test_laya_layer_matches_oracle_gpu(gpu_ctx, case):
    print(f"[layers] Laya layer {case}", flush=True)
    if case == "padded":
        c = laya_padded_layer()
    else:
        w = laya_layer_config(1 if case == "c1_bias" else 2, bias=case == "c1_bias")
        c = dict(x=w.x, keep=w.keep, w_in=w.w_in, b_in=w.b_in, w_out=w.w_out, b_out=w.b_out,
                 hidden=w.hidden, heads=w.heads, length=w.length, batch=w.batch,
                 rope_base=w.rope_base)
    want = oracle.laya_attention_layer(**c)
    if case == "c2":
        import torch

        dev = torch.device("cuda:0")
        t = {k: (torch.from_numpy(np.ascontiguousarray(v)).to(dev) if isinstance(v, np.ndarray)
                 else v) for k, v in c.items()}
        got = te.laya_attention_layer(t["x"], t["keep"], t["w_in"], t["b_in"], t["w_out"],
                                      t["b_out"], c["hidden"], c["heads"], c["length"],
                                      c["batch"], c["rope_base"], ctx=gpu_ctx).cpu().numpy()
    else:
        got = te.laya_attention_layer(c["x"], c["keep"], c["w_in"], c["b_in"], c["w_out"],
                                      c["b_out"], c["hidden"], c["heads"], c["length"],
                                      c["batch"], c["rope_base"], ctx=gpu_ctx)
    assert_close(got, want)


@pytest.mark.gpu
@pytest.mark.parametrize("shape", ["small", "c4"])
def test_jeff_layer_matches_oracle_gpu(gpu_ctx, shape):
    print(f"[layers] Jeff layer {shape}", flush=True)
    if shape == "small":
        j = jeff_layer_config(4, rows=2, length=24, hidden=64)
    else:
        j = jeff_layer_config(4)
    oracle.set_threads(16)
    args = (j.x, j.w_q, j.w_gate, j.w_k, j.w_v, j.w_o, j.q_norm, j.k_norm, j.mask)
    dims = (j.rows, j.length, j.hidden, j.heads, j.kv_heads, j.head_dim, j.rotary_dim, j.theta,
            j.eps)
    for trim in (False, True):
        want = oracle.jeff_layer_rows(*args, *dims, trim_leading=trim)
        got = te.jeff_full_attention_layer_rows(*args, *dims, trim_leading=trim, ctx=gpu_ctx)
        assert_close(got, want)
