"""CPU tests of the C ABI library and the host-side mirror: the library loads,
exports every symbol the header declares, validates arguments with the
reference's messages before touching a device, and never falls back to the
CPU. No kernel runs here."""
import ctypes
import os
import re

import numpy as np
import pytest

import tenferro_ext as te

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in ("tfd_attention.h", "tfd_laya_model.h")]


@pytest.fixture(scope="module")
def lib():
    return te.load_library()


@pytest.fixture()
def ctx():
    c = te.Context(0)
    yield c
    c.close()


def header_symbols():
    text = "".join(open(h).read() for h in HEADERS)
    return sorted(set(re.findall(r"\b(tfd_\w+)\s*\(", text)))


def test_every_header_is_checked():
    on_disk = sorted(f for f in os.listdir(os.path.join(ROOT, "include")) if f.endswith(".h"))
    assert on_disk == sorted(os.path.basename(h) for h in HEADERS)


def test_library_exports_every_declared_symbol(lib):
    declared = header_symbols()
    assert declared == sorted(te.EXPORTED_SYMBOLS)
    for name in declared:
        assert hasattr(lib, name), name


def test_abi_version_and_family_ids(lib):
    assert lib.tfd_abi_version() == 2
    # laya_attention.rs:25 and jeff_attention.rs:24
    assert lib.tfd_laya_attention_block_family_id().decode() == "tenferro-decision.laya_attention_block.v1"
    assert lib.tfd_jeff_full_attention_family_id().decode() == "tenferro-decision.jeff_full_attention.v1"


def test_context_does_not_touch_gpu_on_create(ctx):
    assert ctx.retained_bytes() > 0
    ctx.synchronize()  # nothing enqueued yet: a no-op


def _laya_call(ctx, shape, keep_len, hidden=8, heads=2, out_len=None, qkv_len=None):
    qkv = np.zeros(max(1, int(np.prod(shape))), np.float32)
    qkv_len = int(np.prod(shape)) if qkv_len is None else qkv_len
    keep = np.ones(max(1, keep_len), np.uint8)
    out = np.zeros(max(1, out_len if out_len is not None else hidden * (shape[1] if len(shape) == 3 else 1)
                       * (shape[2] if len(shape) == 3 else 1)), np.float32)
    arr = (ctypes.c_size_t * len(shape))(*shape)
    rc = ctx._lib.tfd_laya_attention_block_f32(
        ctx.handle, qkv.ctypes.data, arr, len(shape), qkv_len, keep.ctypes.data, keep_len, hidden,
        heads,
        te.f32_bits(160000.0), out.ctypes.data,
        out_len if out_len is not None else out.size, 0)
    return rc, ctx._lib.tfd_last_error(ctx.handle).decode()


def test_laya_rejects_bad_rank_and_width(ctx):
    # laya_attention.rs:111-114
    rc, msg = _laya_call(ctx, (24, 4), 16)
    assert rc == te.TFD_EINVAL and "attention block expects (3d, L, B)" in msg
    rc, msg = _laya_call(ctx, (23, 4, 1), 16)
    assert rc == te.TFD_EINVAL and "attention block expects (3d, L, B)" in msg


def test_laya_rejects_short_qkv_storage(ctx):
    """cpu-kernels lib.rs:1205-1210: storage shorter than the shape is rejected
    ("qkv length") before any access -- here with an empty slice, as there,
    and one element short; no device is touched (the no-GPU error would
    otherwise come back)."""
    rc, msg = _laya_call(ctx, (24, 32, 1), 32 * 32, hidden=8, heads=1, qkv_len=0)
    assert rc == te.TFD_EINVAL and "qkv length" in msg
    rc, msg = _laya_call(ctx, (24, 4, 1), 16, qkv_len=24 * 4 - 1)
    assert rc == te.TFD_EINVAL and "qkv length" in msg
    rc, msg = _laya_call(ctx, (24, 4, 1), 16, qkv_len=24 * 4 + 1)
    assert rc == te.TFD_EINVAL and "qkv length" in msg
    op = te.LayaAttentionBlockOp(8, 2, te.f32_bits(0.0))
    with pytest.raises(te.InvalidArgument, match="qkv length"):
        op.execute(np.zeros(24 * 4 - 1, np.float32), (24, 4, 1), np.ones(16, np.uint8), ctx=ctx)


def test_laya_rejects_bad_keep_length(ctx):
    # laya_attention.rs:138-140
    rc, msg = _laya_call(ctx, (24, 4, 1), 15)
    assert rc == te.TFD_EINVAL and "keep must be (L, L, B)" in msg


def test_laya_rejects_bad_out_length(ctx):
    rc, msg = _laya_call(ctx, (24, 4, 1), 16, out_len=31)
    assert rc == te.TFD_EINVAL and "out" in msg


def test_laya_python_mirror_raises_invalid_argument(ctx):
    op = te.LayaAttentionBlockOp(8, 2, te.f32_bits(0.0))
    with pytest.raises(te.InvalidArgument, match=r"keep must be \(L, L, B\)"):
        op.execute(np.zeros(24 * 4, np.float32), (24, 4, 1), np.ones(3, np.uint8), ctx=ctx)


def test_laya_empty_problem_is_ok_without_gpu(ctx):
    rc, _ = _laya_call(ctx, (24, 0, 3), 0, out_len=0)
    assert rc == te.TFD_OK


def test_valid_call_without_gpu_reports_no_fallback(ctx):
    """device.rs:131-135 in the reference: no silent CPU fallback."""
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present; this checks the no-GPU error path")
    rc, msg = _laya_call(ctx, (24, 4, 1), 16)
    assert rc == te.TFD_EHIP and "no CPU fallback" in msg


def _jeff_call(ctx, q_shape, heads, hd, qn=None, kn=None, mask=None, klen=None, rot=None):
    L = q_shape[0]
    n = int(np.prod(q_shape))
    buf = np.zeros(max(n, 1), np.float32)
    qn = hd if qn is None else qn
    kn = hd if kn is None else kn
    mask = L if mask is None else mask
    klen = n if klen is None else klen
    vec = np.zeros(max(qn, kn, mask, 1), np.float32)
    arr = (ctypes.c_size_t * len(q_shape))(*q_shape)
    rc = ctx._lib.tfd_jeff_full_attention_f32(
        ctx.handle, buf.ctypes.data, arr, len(q_shape), buf.ctypes.data, klen, buf.ctypes.data, n,
        buf.ctypes.data, n, vec.ctypes.data, qn, vec.ctypes.data, kn, vec.ctypes.data, mask,
        heads, hd, hd if rot is None else rot, te.f32_bits(1e7), te.f32_bits(1e-6),
        buf.ctypes.data, n, 0)
    return rc, ctx._lib.tfd_last_error(ctx.handle).decode()


def test_jeff_rejects_like_reference(ctx):
    # jeff_attention.rs:116-125
    rc, msg = _jeff_call(ctx, (8,), 2, 4)
    assert rc == te.TFD_EINVAL and "full attention expects (length, width)" in msg
    rc, msg = _jeff_call(ctx, (8, 9), 2, 4)
    assert rc == te.TFD_EINVAL and "width must equal heads * head_dim" in msg
    # jeff_attention.rs:159-164
    for kw in ({"qn": 3}, {"kn": 5}, {"mask": 7}):
        rc, msg = _jeff_call(ctx, (8, 8), 2, 4, **kw)
        assert rc == te.TFD_EINVAL and "q_norm/k_norm must be (head_dim) and mask (length)" in msg
    rc, msg = _jeff_call(ctx, (8, 8), 2, 4, klen=63)
    assert rc == te.TFD_EINVAL and "k/v/gate must be (length, width)" in msg
    rc, msg = _jeff_call(ctx, (8, 8), 2, 4, rot=6)
    assert rc == te.TFD_EINVAL and "rotary_dim" in msg


def test_jeff_dropin_kv_heads_flag_validated(ctx):
    """TFD_KV_HEADS(kv) must divide heads; rejected before any device access."""
    n = 8 * 16
    buf = np.zeros(n, np.float32)
    vec = np.zeros(8, np.float32)
    arr = (ctypes.c_size_t * 2)(8, 16)
    p = buf.ctypes.data
    rc = ctx._lib.tfd_jeff_full_attention_f32(
        ctx.handle, p, arr, 2, p, n, p, n, p, n, vec.ctypes.data, 4, vec.ctypes.data, 4,
        vec.ctypes.data, 8, 4, 4, 4, te.f32_bits(1e7), te.f32_bits(1e-6), p, n, te.TFD_KV_HEADS(3))
    assert rc == te.TFD_EINVAL and "kv_heads must divide heads" in ctx._lib.tfd_last_error(
        ctx.handle).decode()


def test_jeff_rows_rejects_bad_gqa_and_flags(ctx):
    f = np.zeros(64, np.float32)
    p = f.ctypes.data
    rc = ctx._lib.tfd_jeff_full_attention_rows_f32(ctx.handle, 1, 2, 3, 2, 4, 4, p, p, p, p, p, p, p,
                                                   0, 0, p, 0)
    assert rc == te.TFD_EINVAL and "kv_heads" in ctx._lib.tfd_last_error(ctx.handle).decode()
    rc = ctx._lib.tfd_jeff_full_attention_rows_f32(ctx.handle, 1, 2, 2, 2, 4, 4, p, p, p, p, p, p, p,
                                                   0, 0, p, te.TFD_ASYNC)
    assert rc == te.TFD_EINVAL and "TFD_ASYNC" in ctx._lib.tfd_last_error(ctx.handle).decode()


def test_op_descriptors_mirror_payloads():
    a = te.LayaAttentionBlockOp(768, 12, te.f32_bits(160000.0))
    b = te.LayaAttentionBlockOp(768, 12, te.f32_bits(160000.0))
    c = te.LayaAttentionBlockOp(768, 12, te.f32_bits(10000.0))
    assert a.payload_eq(b) and not a.payload_eq(c)
    assert a.payload_hash() == b.payload_hash() != c.payload_hash()
    assert a.family_id() == te.LAYA_ATTENTION_BLOCK_FAMILY_ID
    assert (a.input_count(), a.output_count()) == (2, 1)
    assert a.infer_output_shape((2304, 512, 8)) == (768, 512, 8)
    j = te.JeffFullAttentionOp(8, 256, 64, te.f32_bits(1e7), te.f32_bits(1e-6))
    assert (j.input_count(), j.output_count()) == (7, 1)
    assert j.infer_output_shape((256, 2048)) == (256, 2048)
    with pytest.raises(te.InvalidArgument):
        j.infer_output_shape((256,))
    # (rope_base as f32).to_bits(), laya_attention.rs:228
    assert te.f32_bits(160000.0) == np.float32(160000.0).view(np.uint32)
    assert te.f32_bits(1e-6) == np.float32(1e-6).view(np.uint32)


def test_bf16_round_to_nearest_even():
    x = np.array([1.0, 1.00390625, 1.01171875, -2.5, 3.0e38], np.float32)
    b = te.to_bf16_bits(x)
    # 1 + 2^-8 is a tie between 1 and 1 + 2^-7: rounds to even (1.0)
    assert list(te.bf16_bits_to_f32(b)[:4]) == [1.0, 1.0, 1.015625, -2.5]
    y = np.random.default_rng(0).standard_normal(1000).astype(np.float32)
    assert np.abs(te.bf16_bits_to_f32(te.to_bf16_bits(y)) - y).max() <= np.abs(y).max() * 2 ** -8


# ------------------------------------------------ host-side argument checks
#
# Entries whose C ABI carries no storage lengths (structured, rows, layers,
# the model forward) and torch tensors of the wrong element type are
# rejected by the Python mirror before any device call. torch CPU tensors
# stand in for device tensors here: the checks run before the pointer kind
# matters, and nothing reaches the library.

def test_wrapper_rejects_short_buffers(ctx):
    with pytest.raises(te.InvalidArgument, match="qkv: 95 elements"):
        te.laya_attention_structured(np.zeros(95, np.float32), np.ones(4, np.uint8), 8, 2, 4, 1,
                                     -1, 0.0, ctx=ctx)
    with pytest.raises(te.InvalidArgument, match="valid: 3 elements"):
        te.laya_attention_structured(np.zeros(96, np.float32), np.ones(3, np.uint8), 8, 2, 4, 1,
                                     -1, 0.0, ctx=ctx)
    R, L, H, KV, hd = 2, 4, 4, 2, 8
    f = lambda n: np.zeros(n, np.float32)
    nq, nkv = R * L * H * hd, R * L * KV * hd
    good = dict(q=f(nq), k=f(nkv), v=f(nkv), gate=f(nq), q_norm=f(hd), k_norm=f(hd), mask=f(R * L))
    for name, short in (("q", nq - 1), ("k", nkv - 1), ("v", nkv + 1), ("gate", nq - 4),
                        ("q_norm", hd - 1), ("mask", R * L - 1)):
        bad = dict(good, **{name: f(short)})
        with pytest.raises(te.InvalidArgument, match=f"{name}: {short} elements"):
            te.jeff_full_attention_rows(*bad.values(), R, L, H, KV, hd, hd, 1e7, 1e-6, ctx=ctx)
    with pytest.raises(te.InvalidArgument, match="q: 63 elements"):
        te.jeff_full_attention(f(63), f(64), f(64), f(64), f(8), f(8), f(8), 1, 8, 8, 1e7, 1e-6,
                               q_shape=(8, 8), ctx=ctx)


def test_wrapper_rejects_wrong_tensor_dtypes(ctx):
    import torch

    R, L, H, KV, hd = 1, 4, 2, 1, 8
    t = lambda n, dt=torch.float32: torch.zeros(n, dtype=dt)
    nq, nkv = R * L * H * hd, R * L * KV * hd
    # a bf16 tensor handed to an f32 entry: half the bytes the kernel reads
    with pytest.raises(te.InvalidArgument, match="q: tensor dtype bfloat16, expected float32"):
        te.jeff_full_attention_rows(t(nq, torch.bfloat16), t(nkv), t(nkv), t(nq), t(hd), t(hd),
                                    t(R * L), R, L, H, KV, hd, hd, 1e7, 1e-6, ctx=ctx)
    # the drop-in's k_len compares element counts, so a half-width k passes that check
    with pytest.raises(te.InvalidArgument, match="k: tensor dtype float16"):
        te.jeff_full_attention(t(64), t(64, torch.float16), t(64), t(64), t(8), t(8), t(8), 1, 8,
                               8, 1e7, 1e-6, q_shape=(8, 8), ctx=ctx)
    with pytest.raises(te.InvalidArgument, match="keep: tensor dtype int32"):
        te.laya_attention_block(t(96), t(16, torch.int32), 8, 2, 0.0, qkv_shape=(24, 4, 1),
                                ctx=ctx)
    # bf16 entry: 16-bit types only
    with pytest.raises(te.InvalidArgument, match="gate: tensor dtype float32"):
        te.jeff_full_attention_rows(t(nq, torch.bfloat16), t(nkv, torch.bfloat16),
                                    t(nkv, torch.bfloat16), t(nq), t(hd), t(hd), t(R * L), R, L,
                                    H, KV, hd, hd, 1e7, 1e-6, bf16=True, ctx=ctx)


def test_wrapper_rejects_host_device_mix(ctx):
    """Host arrays and device tensors in one call are refused before any device
    call (a stand-in object reports itself as a CUDA tensor)."""

    class FakeCuda:
        __module__ = "torch.fake"

        def __init__(self, n):
            self.dtype = "torch.float32"
            self._n = n
            self.is_cuda = True

        def is_contiguous(self):
            return True

        def data_ptr(self):
            return 1 << 40

        def numel(self):
            return self._n

    with pytest.raises(te.InvalidArgument, match="mix of host arrays and device tensors"):
        te.laya_attention_structured(FakeCuda(96), np.ones(4, np.uint8), 8, 2, 4, 1, -1, 0.0,
                                     ctx=ctx, out=np.zeros(32, np.float32))
