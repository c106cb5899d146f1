"""The Laya drop-in's no-allocation variant (tfd_laya_attention_block_noalloc_f32):
its workspace is a static device array per GPU, so it must give the drop-in's
results call after call, with the array keeping the previous call's contents.

The GPU tests run calls in a row through the C ABI, each against
tfd_laya_attention_block_f32 on the same device tensors (bitwise: the kernels
and RoPE tables are the same): two calls, the second on a smaller input with
another RoPE base; RoPE on, off, then on again with the same (L, hd, base),
so the third call reuses the resident table after a call that wrote its keep
words with RoPE off; and a call captured into a HIP graph and replayed three
times with eager calls of other shapes (RoPE off) between the replays. The
CPU tests check the refusals that come before any device access.
"""
import ctypes

import numpy as np
import pytest

import tenferro_ext as te
from tenferro_ext.workloads import Lcg, laya_config


def _call(ctx, fn, qkv_ptr, shape, qkv_len, keep_ptr, keep_len, hidden, heads, base, out_ptr,
          out_len, flags):
    arr = (ctypes.c_size_t * len(shape))(*shape)
    rc = fn(ctx.handle, qkv_ptr, arr, len(shape), qkv_len, keep_ptr, keep_len, hidden, heads,
            te.f32_bits(base), out_ptr, out_len, flags)
    return rc, ctx._lib.tfd_last_error(ctx.handle).decode()


def test_noalloc_refuses_host_pointers():
    ctx = te.Context(0)
    qkv = np.zeros(24 * 4, np.float32)
    keep = np.ones(16, np.uint8)
    out = np.zeros(32, np.float32)
    rc, msg = _call(ctx, ctx._lib.tfd_laya_attention_block_noalloc_f32, qkv.ctypes.data,
                    (24, 4, 1), qkv.size, keep.ctypes.data, keep.size, 8, 2, 0.0,
                    out.ctypes.data, out.size, te.TFD_HOST_PTRS)
    assert rc == te.TFD_EINVAL and "device pointers only" in msg
    ctx.close()


def test_noalloc_refuses_oversized_work_before_device_access():
    """L 4096, B 8 needs 16 MiB of packed keep words: more than the array.
    Checked before the device is touched (any address will do here)."""
    ctx = te.Context(0)
    L, B, d, H = 4096, 8, 64, 1
    fake = 1 << 40
    rc, msg = _call(ctx, ctx._lib.tfd_laya_attention_block_noalloc_f32, fake, (3 * d, L, B),
                    3 * d * L * B, fake, L * L * B, d, H, 0.0, fake, d * L * B,
                    te.TFD_DEVICE_PTRS)
    assert rc == te.TFD_EUNSUPPORTED and "workspace" in msg
    ctx.close()


def _case(cfg_or_shape, seed):
    if cfg_or_shape == "c2":
        w = laya_config(2)
        return w.qkv, w.keep, w.hidden, w.heads, w.length, w.batch, w.rope_base
    d, H, L, B, base = cfg_or_shape
    rng = Lcg(seed)
    qkv = rng.normal(3 * d * L * B).astype(np.float32)
    keep = (rng.uniform(L * L * B) < 0.7).astype(np.uint8)
    keep.reshape(B, L, L)[:, :, 0] = 0  # query 0 keeps nothing: NaN rows as the reference
    return qkv, keep, d, H, L, B, base


@pytest.mark.gpu
def test_noalloc_matches_dropin_two_calls_gpu():
    import torch

    dev = torch.device("cuda:0")
    ctx = te.Context(0)
    cases = [("c2", 1), ((128, 2, 100, 2, 10000.0), 2)]  # the second call is smaller
    for case, seed in cases:
        qkv, keep, d, H, L, B, base = _case(case, seed)
        print(f"[noalloc] d {d} heads {H} L {L} B {B} base {base}", flush=True)
        tq = torch.from_numpy(qkv).to(dev)
        tk = torch.from_numpy(keep).to(dev)
        want = torch.full((d * L * B,), -7.0, dtype=torch.float32, device=dev)
        got = torch.full((d * L * B,), -7.0, dtype=torch.float32, device=dev)
        torch.cuda.synchronize()
        shape = (3 * d, L, B)
        rc, msg = _call(ctx, ctx._lib.tfd_laya_attention_block_f32, tq.data_ptr(), shape,
                        tq.numel(), tk.data_ptr(), tk.numel(), d, H, base, want.data_ptr(),
                        want.numel(), te.TFD_DEVICE_PTRS)
        assert rc == te.TFD_OK, msg
        rc, msg = _call(ctx, ctx._lib.tfd_laya_attention_block_noalloc_f32, tq.data_ptr(), shape,
                        tq.numel(), tk.data_ptr(), tk.numel(), d, H, base, got.data_ptr(),
                        got.numel(), te.TFD_DEVICE_PTRS)
        assert rc == te.TFD_OK, msg
        g, w = got.cpu().numpy(), want.cpu().numpy()
        assert np.array_equal(np.isnan(g), np.isnan(w))
        assert np.array_equal(g.view(np.uint32), w.view(np.uint32))
        # the Python mirror of the entry gives the same
        again = te.laya_attention_block_noalloc(tq, tk, d, H, base, qkv_shape=shape, ctx=ctx)
        assert np.array_equal(again.cpu().numpy().view(np.uint32), w.view(np.uint32))
    ctx.close()


def _dropin_vs_noalloc(ctx, case, seed, dev):
    import torch

    qkv, keep, d, H, L, B, base = _case(case, seed)
    print(f"[noalloc] d {d} heads {H} L {L} B {B} base {base}", flush=True)
    tq = torch.from_numpy(qkv).to(dev)
    tk = torch.from_numpy(keep).to(dev)
    want = torch.full((d * L * B,), -7.0, dtype=torch.float32, device=dev)
    got = torch.full((d * L * B,), -7.0, dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    shape = (3 * d, L, B)
    rc, msg = _call(ctx, ctx._lib.tfd_laya_attention_block_f32, tq.data_ptr(), shape, tq.numel(),
                    tk.data_ptr(), tk.numel(), d, H, base, want.data_ptr(), want.numel(),
                    te.TFD_DEVICE_PTRS)
    assert rc == te.TFD_OK, msg
    rc, msg = _call(ctx, ctx._lib.tfd_laya_attention_block_noalloc_f32, tq.data_ptr(), shape,
                    tq.numel(), tk.data_ptr(), tk.numel(), d, H, base, got.data_ptr(),
                    got.numel(), te.TFD_DEVICE_PTRS)
    assert rc == te.TFD_OK, msg
    g, w = got.cpu().numpy(), want.cpu().numpy()
    assert np.array_equal(g.view(np.uint32), w.view(np.uint32)), f"base {base}: not bitwise equal"


@pytest.mark.gpu
def test_noalloc_rope_table_survives_rope_off_calls_gpu():
    """RoPE 160000, then RoPE off (its keep words go to the scratch), then
    RoPE 160000 again with the same (L, hd): the third call finds its table
    resident and must still read cos/sin, not keep words."""
    import torch

    dev = torch.device("cuda:0")
    ctx = te.Context(0)
    for case, seed in [((128, 2, 96, 2, 160000.0), 11), ((128, 2, 96, 2, 0.0), 12),
                       ((128, 2, 96, 2, 160000.0), 13), ((64, 1, 40, 3, 0.0), 14),
                       ((128, 2, 96, 2, 160000.0), 15)]:
        _dropin_vs_noalloc(ctx, case, seed, dev)
    ctx.close()


@pytest.mark.gpu
def test_noalloc_graph_capture_replays_gpu():
    """One call captured on the context's stream (TFD_ASYNC) after an eager
    call made its RoPE table resident; three replays, each after an eager
    RoPE-off call of another shape, each bitwise equal to the drop-in. Under
    capture, a call without TFD_ASYNC and a call whose table is not resident
    are refused before they record anything."""
    import torch

    dev = torch.device("cuda:0")
    side = torch.cuda.Stream(device=dev)
    ctx = te.Context(0, stream=side.cuda_stream)
    other = te.Context(0)
    qkv, keep, d, H, L, B, base = _case((128, 2, 100, 2, 10000.0), 21)
    shape = (3 * d, L, B)
    tq = torch.from_numpy(qkv).to(dev)
    tk = torch.from_numpy(keep).to(dev)
    want = torch.full((d * L * B,), -7.0, dtype=torch.float32, device=dev)
    got = torch.full((d * L * B,), -7.0, dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    fn = ctx._lib.tfd_laya_attention_block_noalloc_f32
    rc, msg = _call(ctx, ctx._lib.tfd_laya_attention_block_f32, tq.data_ptr(), shape, tq.numel(),
                    tk.data_ptr(), tk.numel(), d, H, base, want.data_ptr(), want.numel(),
                    te.TFD_DEVICE_PTRS)
    assert rc == te.TFD_OK, msg
    # eager call: the RoPE table of (L, hd, base) becomes resident
    rc, msg = _call(ctx, fn, tq.data_ptr(), shape, tq.numel(), tk.data_ptr(), tk.numel(), d, H,
                    base, got.data_ptr(), got.numel(), te.TFD_DEVICE_PTRS)
    assert rc == te.TFD_OK, msg
    w = want.cpu().numpy()
    assert np.array_equal(got.cpu().numpy().view(np.uint32), w.view(np.uint32))
    print("[noalloc capture] capturing one call", flush=True)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        rc_sync, msg_sync = _call(ctx, fn, tq.data_ptr(), shape, tq.numel(), tk.data_ptr(),
                                  tk.numel(), d, H, base, got.data_ptr(), got.numel(),
                                  te.TFD_DEVICE_PTRS)
        rc_new, msg_new = _call(ctx, fn, tq.data_ptr(), shape, tq.numel(), tk.data_ptr(),
                                tk.numel(), d, H, 20000.0, got.data_ptr(), got.numel(),
                                te.TFD_DEVICE_PTRS | te.TFD_ASYNC)
        rc, msg = _call(ctx, fn, tq.data_ptr(), shape, tq.numel(), tk.data_ptr(), tk.numel(), d,
                        H, base, got.data_ptr(), got.numel(), te.TFD_DEVICE_PTRS | te.TFD_ASYNC)
    assert rc_sync == te.TFD_EINVAL and "TFD_ASYNC" in msg_sync, msg_sync
    assert rc_new == te.TFD_EUNSUPPORTED and "capture" in msg_new, msg_new
    assert rc == te.TFD_OK, msg
    for i in range(3):
        got.fill_(-7.0)
        # eager work between replays: a RoPE-off call of another shape on the
        # same GPU rewrites the keep-word region of the scratch
        q2, k2, d2, H2, L2, B2, _ = _case((64, 1, 40 + 8 * i, 3, 0.0), 30 + i)
        t2, m2 = torch.from_numpy(q2).to(dev), torch.from_numpy(k2).to(dev)
        o2 = torch.empty(d2 * L2 * B2, dtype=torch.float32, device=dev)
        torch.cuda.synchronize()
        rc2, msg2 = _call(other, fn, t2.data_ptr(), (3 * d2, L2, B2), t2.numel(), m2.data_ptr(),
                          m2.numel(), d2, H2, 0.0, o2.data_ptr(), o2.numel(), te.TFD_DEVICE_PTRS)
        assert rc2 == te.TFD_OK, msg2
        graph.replay()
        torch.cuda.synchronize()
        print(f"[noalloc capture] replay {i}", flush=True)
        assert np.array_equal(got.cpu().numpy().view(np.uint32), w.view(np.uint32)), \
            f"replay {i} differs from the drop-in"
    other.close()
    ctx.close()
