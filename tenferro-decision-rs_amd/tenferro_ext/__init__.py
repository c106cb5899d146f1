"""Python mirror of the reference's tenferro-ext attention ops over the MI355X C ABI.

The reference exposes the two ops as eager-session extension methods:

* ``EagerSessionLayaAttentionExt::laya_attention_block(qkv, keep, hidden, heads,
  rope_base)`` -- crates/tenferro-ext/src/laya_attention.rs:206-249
* ``EagerSessionJeffAttentionExt::jeff_full_attention(q, k, v, gate, q_norm,
  k_norm, mask, heads, head_dim, rotary_dim, theta, eps)`` --
  crates/tenferro-ext/src/jeff_attention.rs:214-275

and as ``ExtensionOp`` descriptors (``LayaAttentionBlockOp``,
``JeffFullAttentionOp``) whose payload stores the f64 parameters as f32 bits.
This module keeps those names, argument meanings and error behaviour, and runs
every call on the GPU through ``libtfd_attention.so``. There is no CPU
fallback: if the library or a GPU is missing, calls raise.

Arrays may be numpy arrays (host pointers: the library uploads, runs and
downloads) or torch CUDA tensors (device pointers, run on the context stream).
Layouts are the reference's column-major ones, flattened (see
``include/tfd_attention.h``).
"""
from __future__ import annotations

import ctypes
import hashlib
import os
import struct
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY_PATH = os.path.join(os.path.dirname(_HERE), "_build", "libtfd_attention.so")

LAYA_ATTENTION_BLOCK_FAMILY_ID = "tenferro-decision.laya_attention_block.v1"
JEFF_FULL_ATTENTION_FAMILY_ID = "tenferro-decision.jeff_full_attention.v1"

TFD_OK = 0
TFD_EINVAL = 1
TFD_EUNSUPPORTED = 2
TFD_EHIP = 3
TFD_HOST_PTRS = 0
TFD_DEVICE_PTRS = 1
TFD_ASYNC = 2
TFD_TRIM_LEADING = 4
TFD_KV_HEADS_MASK = 0xFFFF0000


def TFD_KV_HEADS(kv_heads: int) -> int:
    """Flag for the Jeff drop-in on GQA-expanded K/V (include/tfd_attention.h)."""
    return (int(kv_heads) & 0xFFFF) << 16

# Every entry point the header declares, in declaration order.
EXPORTED_SYMBOLS = (
    "tfd_abi_version",
    "tfd_laya_attention_block_family_id",
    "tfd_jeff_full_attention_family_id",
    "tfd_ctx_create",
    "tfd_ctx_create_on_stream",
    "tfd_ctx_destroy",
    "tfd_last_error",
    "tfd_ctx_synchronize",
    "tfd_ctx_stream",
    "tfd_ctx_retained_bytes",
    "tfd_ctx_set_timing",
    "tfd_ctx_take_kernel_time",
    "tfd_laya_attention_block_f32",
    "tfd_laya_attention_block_noalloc_f32",
    "tfd_laya_attention_structured_f32",
    "tfd_jeff_full_attention_f32",
    "tfd_jeff_full_attention_rows_f32",
    "tfd_jeff_full_attention_rows_bf16",
    "tfd_laya_attention_layer_f32",
    "tfd_jeff_full_attention_layer_rows_f32",
    "tfd_laya_forward_f32",
)


class TenferroExtError(RuntimeError):
    """A non-zero status from the C ABI; ``code`` is the TFD_* status."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[{_STATUS.get(code, code)}] {message}")
        self.code = code
        self.message = message


class InvalidArgument(TenferroExtError):
    """``tenferro_tensor::Error::invalid_argument`` of the reference."""


class Unsupported(TenferroExtError):
    pass


class DeviceError(TenferroExtError):
    pass


_STATUS = {TFD_EINVAL: "EINVAL", TFD_EUNSUPPORTED: "EUNSUPPORTED", TFD_EHIP: "EHIP"}
_ERROR_TYPES = {TFD_EINVAL: InvalidArgument, TFD_EUNSUPPORTED: Unsupported, TFD_EHIP: DeviceError}

_lib = None


def load_library(path: Optional[str] = None) -> ctypes.CDLL:
    """Load libtfd_attention.so and declare its signatures (raises if absent)."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    path = path or LIBRARY_PATH
    if not os.path.exists(path):
        raise ImportError(
            f"{path} is not built; run `make -C tenferro-decision-rs_amd` "
            "(there is no CPU fallback for these ops)"
        )
    # torch ships its own HIP runtime with the same soname (libamdhip64.so.7)
    # but loads it under another name, so two runtimes end up in one process
    # if the library is loaded first. Loading torch first makes the library
    # bind to the runtime torch already holds: one HIP runtime per process.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(path)
    P, S, U32, I, F = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint32, ctypes.c_int, ctypes.c_uint
    SP = ctypes.POINTER(ctypes.c_size_t)
    sig = {
        "tfd_abi_version": (I, []),
        "tfd_laya_attention_block_family_id": (ctypes.c_char_p, []),
        "tfd_jeff_full_attention_family_id": (ctypes.c_char_p, []),
        "tfd_ctx_create": (I, [I, ctypes.POINTER(P)]),
        "tfd_ctx_create_on_stream": (I, [I, P, ctypes.POINTER(P)]),
        "tfd_ctx_destroy": (None, [P]),
        "tfd_last_error": (ctypes.c_char_p, [P]),
        "tfd_ctx_synchronize": (I, [P]),
        "tfd_ctx_stream": (P, [P]),
        "tfd_ctx_retained_bytes": (S, [P]),
        "tfd_ctx_set_timing": (I, [P, I]),
        "tfd_ctx_take_kernel_time": (I, [P, ctypes.POINTER(ctypes.c_double),
                                         ctypes.POINTER(ctypes.c_uint64)]),
        "tfd_laya_attention_block_f32": (I, [P, P, SP, S, S, P, S, S, S, U32, P, S, F]),
        "tfd_laya_attention_block_noalloc_f32": (I, [P, P, SP, S, S, P, S, S, S, U32, P, S, F]),
        "tfd_laya_attention_structured_f32": (I, [P, P, S, S, S, S, P, ctypes.c_int64, U32, P, F]),
        "tfd_jeff_full_attention_f32": (
            I, [P, P, SP, S, P, S, P, S, P, S, P, S, P, S, P, S, S, S, S, U32, U32, P, S, F]),
        "tfd_jeff_full_attention_rows_f32": (
            I, [P, S, S, S, S, S, S, P, P, P, P, P, P, P, U32, U32, P, F]),
        "tfd_jeff_full_attention_rows_bf16": (
            I, [P, S, S, S, S, S, S, P, P, P, P, P, P, P, U32, U32, P, F]),
        "tfd_laya_attention_layer_f32": (I, [P, P, S, S, S, S, P, P, P, P, P, U32, P, F]),
        "tfd_jeff_full_attention_layer_rows_f32": (
            I, [P, S, S, S, S, S, S, S, P, P, P, P, P, P, P, P, P, U32, U32, P, F]),
        "tfd_laya_forward_f32": (I, [P, P, P, P, S, S, P, P, S, P, P, P, F]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path == LIBRARY_PATH:
        _lib = lib
    return lib


def f32_bits(value: float) -> int:
    """``(value as f32).to_bits()`` as the reference stores its f64 parameters."""
    return struct.unpack("<I", struct.pack("<f", float(value)))[0]


class Context:
    """Owns a tfd_ctx: one HIP stream, the RoPE table cache and device workspace.

    Creation does not touch the GPU. ``stream`` adopts a caller-owned
    hipStream_t (for example ``torch.cuda.current_stream().cuda_stream``).
    """

    def __init__(self, device: int = 0, stream: Optional[int] = None):
        self._lib = load_library()
        handle = ctypes.c_void_p()
        if stream is None:
            rc = self._lib.tfd_ctx_create(device, ctypes.byref(handle))
        else:
            rc = self._lib.tfd_ctx_create_on_stream(device, ctypes.c_void_p(stream), ctypes.byref(handle))
        if rc != TFD_OK:
            raise DeviceError(rc, "tfd_ctx_create failed")
        self._h = handle
        self.device = device

    @property
    def handle(self) -> ctypes.c_void_p:
        return self._h

    def check(self, rc: int) -> None:
        if rc != TFD_OK:
            msg = self._lib.tfd_last_error(self._h).decode()
            raise _ERROR_TYPES.get(rc, TenferroExtError)(rc, msg)

    def synchronize(self) -> None:
        self.check(self._lib.tfd_ctx_synchronize(self._h))

    def stream(self) -> int:
        return self._lib.tfd_ctx_stream(self._h) or 0

    def retained_bytes(self) -> int:
        return self._lib.tfd_ctx_retained_bytes(self._h)

    def set_timing(self, enabled: bool) -> None:
        self.check(self._lib.tfd_ctx_set_timing(self._h, 1 if enabled else 0))

    def take_kernel_time(self):
        """(summed ms, launches) of attention kernels timed since the last take."""
        ms, n = ctypes.c_double(), ctypes.c_uint64()
        self.check(self._lib.tfd_ctx_take_kernel_time(self._h, ctypes.byref(ms), ctypes.byref(n)))
        return ms.value, n.value

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.tfd_ctx_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


_default_ctx: Optional[Context] = None


def default_context() -> Context:
    global _default_ctx
    if _default_ctx is None:
        _default_ctx = Context(0)
    return _default_ctx


# ------------------------------------------------------------------ buffers

def _is_torch(x) -> bool:
    return type(x).__module__.startswith("torch")


# torch dtypes accepted for each host dtype: f32 operands, keep/valid bytes,
# bf16 bits (any 16-bit type, read as raw bits).
_TORCH_DTYPES = {
    np.dtype(np.float32): ("float32",),
    np.dtype(np.uint8): ("uint8", "bool"),
    np.dtype(np.uint16): ("uint16", "int16", "bfloat16"),
}


class _Arg:
    """A flat buffer argument: host numpy array or torch tensor (CUDA: device
    pointer; CPU: host pointer).

    ``count`` is the element count the call's shape implies; entries whose C
    ABI carries no lengths pass it, so a short buffer is rejected here before
    any device access. A torch tensor must already have the element type the
    entry reads (no silent reinterpretation of a half-width type)."""

    def __init__(self, x, dtype, name, count: Optional[int] = None):
        self.obj = x
        self.name = name
        if x is None:
            self.ptr, self.n, self.device = None, 0, None
            return
        if _is_torch(x):
            allowed = _TORCH_DTYPES[np.dtype(dtype)]
            got = str(x.dtype).replace("torch.", "")
            if got not in allowed:
                raise InvalidArgument(
                    TFD_EINVAL, f"{name}: tensor dtype {got}, expected {' or '.join(allowed)}")
            if not x.is_contiguous():
                raise InvalidArgument(TFD_EINVAL, f"{name}: tensor must be contiguous")
            self.ptr = x.data_ptr()
            self.n = x.numel()
            self.device = x.is_cuda
        else:
            arr = np.ascontiguousarray(x, dtype=dtype)
            self.obj = arr
            self.ptr = arr.ctypes.data
            self.n = arr.size
            self.device = False
        if count is not None and self.n != count:
            raise InvalidArgument(
                TFD_EINVAL, f"{name}: {self.n} elements, the shape needs {count}")


_async = False


class asynchronous:
    """Within this block, calls on device tensors are enqueued on the context
    stream and return without synchronizing (TFD_ASYNC)."""

    def __enter__(self):
        global _async
        self._prev, _async = _async, True

    def __exit__(self, *exc):
        global _async
        _async = self._prev


def _flags(args: Sequence[_Arg], ctx: Optional["Context"] = None) -> int:
    kinds = {a.device for a in args if a.obj is not None}
    if len(kinds) > 1:
        raise InvalidArgument(TFD_EINVAL, "mix of host arrays and device tensors")
    if kinds == {True}:
        if ctx is not None:
            for a in args:
                if a.obj is not None and a.obj.device.index not in (None, ctx.device):
                    raise InvalidArgument(
                        TFD_EINVAL, f"{a.name}: tensor on cuda:{a.obj.device.index}, "
                        f"the context runs on device {ctx.device}")
        return TFD_DEVICE_PTRS | (TFD_ASYNC if _async else 0)
    return TFD_HOST_PTRS


class _StreamOrder:
    """Orders a device-pointer call against torch's current stream.

    The library runs on the context's own stream. Before the call, that
    stream waits for the work torch has queued so far (the kernels that
    produce the inputs); after an asynchronous call, torch's current stream
    waits for the context stream (so later torch work sees the outputs and
    the caching allocator does not reuse them early). A synchronous call
    returns after its stream has drained, so nothing more is needed then."""

    def __init__(self, ctx: "Context", flags: int):
        self.stream = None
        if not flags & TFD_DEVICE_PTRS:
            return
        import torch

        cur = torch.cuda.current_stream(ctx.device)
        handle = ctx.stream()
        if not handle or handle == cur.cuda_stream:
            return
        self.torch_stream = cur
        self.stream = torch.cuda.ExternalStream(handle, device=ctx.device)
        self.stream.wait_stream(cur)
        self.flags = flags

    def done(self) -> None:
        if self.stream is not None and self.flags & TFD_ASYNC:
            self.torch_stream.wait_stream(self.stream)


def _call(ctx: "Context", flags: int, fn, *args) -> None:
    """Runs one C ABI call with stream ordering and error mapping. torch's
    stream waits for the context stream also when the call fails: kernels it
    enqueued before the failing step may still read the inputs."""
    order = _StreamOrder(ctx, flags)
    try:
        ctx.check(fn(*args))
    finally:
        order.done()


def _shape_arr(shape):
    return (ctypes.c_size_t * len(shape))(*shape)


def _new_out(like: _Arg, n: int):
    if like.device:
        import torch

        return torch.empty(n, dtype=torch.float32, device=like.obj.device)
    return np.empty(n, dtype=np.float32)


# ------------------------------------------------------------------ op descriptors

@dataclass(frozen=True)
class LayaAttentionBlockOp:
    """laya_attention.rs:27-36: payload {hidden, heads, rope_base_bits}."""

    hidden: int
    heads: int
    rope_base_bits: int

    def family_id(self) -> str:
        return LAYA_ATTENTION_BLOCK_FAMILY_ID

    def input_count(self) -> int:
        return 2

    def output_count(self) -> int:
        return 1

    def payload_hash(self) -> str:
        h = hashlib.sha256()
        h.update(struct.pack("<QQI", self.hidden, self.heads, self.rope_base_bits))
        return h.hexdigest()

    def payload_eq(self, other) -> bool:
        return isinstance(other, LayaAttentionBlockOp) and (
            (self.hidden, self.heads, self.rope_base_bits)
            == (other.hidden, other.heads, other.rope_base_bits))

    def infer_output_shape(self, qkv_shape: Sequence[int]):
        """laya_attention.rs:75-97: (3d, L, B) -> (hidden, L, B)."""
        if len(qkv_shape) != 3:
            raise InvalidArgument(TFD_EINVAL, "attention block expects (3d, L, B)")
        return (self.hidden, qkv_shape[1], qkv_shape[2])

    def execute(self, qkv, qkv_shape, keep, *, ctx: Optional[Context] = None, out=None):
        """execute_laya_attention_block_in_session (laya_attention.rs:99-176)."""
        ctx = ctx or default_context()
        a_qkv = _Arg(qkv, np.float32, "qkv")
        a_keep = _Arg(keep, np.uint8, "keep")
        n = self.hidden * (qkv_shape[1] if len(qkv_shape) == 3 else 0) * (
            qkv_shape[2] if len(qkv_shape) == 3 else 0)
        if out is None:
            out = _new_out(a_qkv, n)
        a_out = _Arg(out, np.float32, "out")
        flags = _flags([a_qkv, a_keep, a_out], ctx)
        shape = _shape_arr(qkv_shape)
        # The storage lengths go to the library, which rejects a short qkv
        # ("qkv length"), keep or out with the reference's messages.
        _call(ctx, flags, ctx._lib.tfd_laya_attention_block_f32,
              ctx.handle, a_qkv.ptr, shape, len(qkv_shape), a_qkv.n, a_keep.ptr, a_keep.n,
              self.hidden, self.heads, self.rope_base_bits, a_out.ptr, a_out.n, flags)
        return a_out.obj


@dataclass(frozen=True)
class JeffFullAttentionOp:
    """jeff_attention.rs:27-39: payload {heads, head_dim, rotary_dim, theta_bits, eps_bits}."""

    heads: int
    head_dim: int
    rotary_dim: int
    theta_bits: int
    eps_bits: int

    def family_id(self) -> str:
        return JEFF_FULL_ATTENTION_FAMILY_ID

    def input_count(self) -> int:
        return 7

    def output_count(self) -> int:
        return 1

    def payload_hash(self) -> str:
        h = hashlib.sha256()
        h.update(struct.pack("<QQQII", self.heads, self.head_dim, self.rotary_dim,
                             self.theta_bits, self.eps_bits))
        return h.hexdigest()

    def payload_eq(self, other) -> bool:
        return isinstance(other, JeffFullAttentionOp) and (
            (self.heads, self.head_dim, self.rotary_dim, self.theta_bits, self.eps_bits)
            == (other.heads, other.head_dim, other.rotary_dim, other.theta_bits, other.eps_bits))

    def infer_output_shape(self, q_shape: Sequence[int]):
        """jeff_attention.rs:88-100: (length, width) -> (length, width)."""
        if len(q_shape) != 2:
            raise InvalidArgument(TFD_EINVAL, "full attention expects (length, width)")
        return tuple(q_shape)

    def execute(self, q, q_shape, k, v, gate, q_norm, k_norm, mask, *,
                ctx: Optional[Context] = None, out=None, kv_heads: Optional[int] = None):
        """execute_jeff_full_attention_in_session (jeff_attention.rs:103-184).

        kv_heads: k and v are GQA-expanded (heads / kv_heads consecutive heads
        are copies, jeff-infer checkpoint.rs:307-319); only the first head
        of each group is read (TFD_KV_HEADS)."""
        ctx = ctx or default_context()
        n = 1
        for s in q_shape:
            n *= s
        # q's storage length is not an ABI argument (its shape is): checked here.
        args = [_Arg(x, np.float32, nm, c) for x, nm, c in
                ((q, "q", n), (k, "k", None), (v, "v", None), (gate, "gate", None),
                 (q_norm, "q_norm", None), (k_norm, "k_norm", None), (mask, "mask", None))]
        if out is None:
            out = _new_out(args[0], n)
        a_out = _Arg(out, np.float32, "out")
        flags = _flags(args + [a_out], ctx)
        if kv_heads is not None:
            flags |= TFD_KV_HEADS(kv_heads)
        shape = _shape_arr(q_shape)
        aq, ak, av, ag, aqn, akn, am = args
        _call(ctx, flags, ctx._lib.tfd_jeff_full_attention_f32,
              ctx.handle, aq.ptr, shape, len(q_shape), ak.ptr, ak.n, av.ptr, av.n, ag.ptr, ag.n,
              aqn.ptr, aqn.n, akn.ptr, akn.n, am.ptr, am.n, self.heads, self.head_dim,
              self.rotary_dim, self.theta_bits, self.eps_bits, a_out.ptr, a_out.n, flags)
        return a_out.obj


# ------------------------------------------------------------------ eager entry points

def laya_attention_block(qkv, keep, hidden: int, heads: int, rope_base: float, *,
                         qkv_shape: Optional[Sequence[int]] = None,
                         ctx: Optional[Context] = None, out=None):
    """``session.laya_attention_block(qkv, keep, hidden, heads, rope_base)``.

    ``qkv`` is the (3d, L, B) column-major tensor; pass it as an array of that
    shape in Fortran order, or flat with ``qkv_shape``. ``keep`` is the
    (L, L, B) bool tensor. ``rope_base == 0`` disables RoPE. Returns the
    (d, L, B) output flat.
    """
    if qkv_shape is None:
        qkv_shape = tuple(qkv.shape)
        if not _is_torch(qkv):
            qkv = np.asarray(qkv).reshape(-1, order="F")
            keep = np.asarray(keep).reshape(-1, order="F")
    op = LayaAttentionBlockOp(hidden, heads, f32_bits(rope_base))
    return op.execute(qkv, qkv_shape, keep, ctx=ctx, out=out)


def laya_attention_block_noalloc(qkv, keep, hidden: int, heads: int, rope_base: float, *,
                                 qkv_shape: Sequence[int], ctx: Optional[Context] = None,
                                 out=None):
    """The Laya drop-in's no-allocation variant (device tensors only; its
    workspace is a static 16 MiB device array per GPU, shared by every call
    on that GPU, so overlapping calls on one GPU race)."""
    ctx = ctx or default_context()
    a_qkv = _Arg(qkv, np.float32, "qkv")
    a_keep = _Arg(keep, np.uint8, "keep")
    n = hidden * qkv_shape[1] * qkv_shape[2] if len(qkv_shape) == 3 else 0
    if out is None:
        out = _new_out(a_qkv, n)
    a_out = _Arg(out, np.float32, "out")
    flags = _flags([a_qkv, a_keep, a_out], ctx)
    _call(ctx, flags, ctx._lib.tfd_laya_attention_block_noalloc_f32,
          ctx.handle, a_qkv.ptr, _shape_arr(qkv_shape), len(qkv_shape), a_qkv.n, a_keep.ptr,
          a_keep.n, hidden, heads, f32_bits(rope_base), a_out.ptr, a_out.n, flags)
    return a_out.obj


def laya_attention_structured(qkv, valid, hidden: int, heads: int, length: int, batch: int,
                              window: int, rope_base: float, *,
                              ctx: Optional[Context] = None, out=None):
    """Laya with ``valid (L, B)`` + ``window`` (-1 = global) instead of keep."""
    ctx = ctx or default_context()
    n = hidden * length * batch
    a_qkv = _Arg(qkv, np.float32, "qkv", 3 * n)
    a_valid = _Arg(valid, np.uint8, "valid", length * batch)
    if out is None:
        out = _new_out(a_qkv, n)
    a_out = _Arg(out, np.float32, "out", n)
    flags = _flags([a_qkv, a_valid, a_out], ctx)
    _call(ctx, flags, ctx._lib.tfd_laya_attention_structured_f32,
          ctx.handle, a_qkv.ptr, hidden, heads, length, batch, a_valid.ptr, int(window),
          f32_bits(rope_base), a_out.ptr, flags)
    return a_out.obj


def jeff_full_attention(q, k, v, gate, q_norm, k_norm, mask, heads: int, head_dim: int,
                        rotary_dim: int, theta: float, eps: float, *,
                        q_shape: Optional[Sequence[int]] = None,
                        ctx: Optional[Context] = None, out=None,
                        kv_heads: Optional[int] = None):
    """``session.jeff_full_attention(q, k, v, gate, q_norm, k_norm, mask, heads,
    head_dim, rotary_dim, theta, eps)``; q/k/v/gate are (length, width).
    kv_heads: k/v are GQA-expanded copies; read one head per group."""
    if q_shape is None:
        q_shape = tuple(q.shape)
        if not _is_torch(q):
            q, k, v, gate = (np.asarray(x).reshape(-1, order="F") for x in (q, k, v, gate))
    op = JeffFullAttentionOp(heads, head_dim, rotary_dim, f32_bits(theta), f32_bits(eps))
    return op.execute(q, q_shape, k, v, gate, q_norm, k_norm, mask, ctx=ctx, out=out,
                      kv_heads=kv_heads)


def jeff_full_attention_rows(q, k, v, gate, q_norm, k_norm, mask, rows: int, length: int,
                             heads: int, kv_heads: int, head_dim: int, rotary_dim: int,
                             theta: float, eps: float, *, trim_leading: bool = False,
                             bf16: bool = False, ctx: Optional[Context] = None, out=None):
    """Batched rows with native GQA (k/v at kv_heads width); bf16 takes q/k/v/gate
    as uint16 bf16 bits."""
    ctx = ctx or default_context()
    dt = np.uint16 if bf16 else np.float32
    nq = rows * length * heads * head_dim
    nkv = rows * length * kv_heads * head_dim
    aq, ak, av, ag = (_Arg(x, dt, nm, c) for x, nm, c in
                      ((q, "q", nq), (k, "k", nkv), (v, "v", nkv), (gate, "gate", nq)))
    aqn, akn, am = (_Arg(x, np.float32, nm, c) for x, nm, c in
                    ((q_norm, "q_norm", head_dim), (k_norm, "k_norm", head_dim),
                     (mask, "mask", rows * length)))
    if out is None:
        out = _new_out(aq, nq)
    a_out = _Arg(out, np.float32, "out", nq)
    flags = _flags([aq, ak, av, ag, aqn, akn, am, a_out], ctx)
    if trim_leading:
        flags |= TFD_TRIM_LEADING
    fn = ctx._lib.tfd_jeff_full_attention_rows_bf16 if bf16 else ctx._lib.tfd_jeff_full_attention_rows_f32
    _call(ctx, flags, fn, ctx.handle, rows, length, heads, kv_heads, head_dim, rotary_dim,
          aq.ptr, ak.ptr, av.ptr, ag.ptr, aqn.ptr, akn.ptr, am.ptr,
          f32_bits(theta), f32_bits(eps), a_out.ptr, flags)
    return a_out.obj


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16 bits (uint16)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    rounding = ((u >> 16) & 1) + 0x7FFF
    return ((u + rounding) >> 16).astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ------------------------------------------------------------------ layers

def laya_attention_layer(x, keep, w_in, b_in, w_out, b_out, hidden: int, heads: int,
                         length: int, batch: int, rope_base: float, *,
                         ctx: Optional[Context] = None, out=None):
    """A Laya attention layer (laya-infer model.rs:1304-1347, f32 path):
    qkv = W_in^T x (+ b_in), the fused attention op, out = W_out^T attended
    (+ b_out). x and out are (hidden, L, B) flat, W_in (hidden, 3*hidden) and
    W_out (hidden, hidden) column-major; biases may be None."""
    ctx = ctx or default_context()
    n = hidden * length * batch
    ax, ak = _Arg(x, np.float32, "x", n), _Arg(keep, np.uint8, "keep", length * length * batch)
    awi = _Arg(w_in, np.float32, "w_in", hidden * 3 * hidden)
    awo = _Arg(w_out, np.float32, "w_out", hidden * hidden)
    abi = _Arg(b_in, np.float32, "b_in", 3 * hidden if b_in is not None else None)
    abo = _Arg(b_out, np.float32, "b_out", hidden if b_out is not None else None)
    if out is None:
        out = _new_out(ax, n)
    a_out = _Arg(out, np.float32, "out", n)
    flags = _flags([ax, ak, awi, awo, abi, abo, a_out], ctx)
    _call(ctx, flags, ctx._lib.tfd_laya_attention_layer_f32,
          ctx.handle, ax.ptr, hidden, heads, length, batch, ak.ptr, awi.ptr, abi.ptr, awo.ptr,
          abo.ptr, f32_bits(rope_base), a_out.ptr, flags)
    return a_out.obj


def jeff_full_attention_layer_rows(x, w_q, w_gate, w_k, w_v, w_o, q_norm, k_norm, mask,
                                   rows: int, length: int, hidden: int, heads: int,
                                   kv_heads: int, head_dim: int, rotary_dim: int, theta: float,
                                   eps: float, *, trim_leading: bool = False,
                                   ctx: Optional[Context] = None, out=None):
    """A Jeff full-attention layer over rows (jeff-infer model.rs:686-780, f32
    path): q/gate/k/v = x W, the fused rows op with native GQA, out = merged
    W_o. x and out are rows x (L, hidden) flat; weights (in, out) column-major."""
    ctx = ctx or default_context()
    W, KW, n = heads * head_dim, kv_heads * head_dim, rows * length * hidden
    args = [_Arg(a, np.float32, nm, c) for a, nm, c in
            ((x, "x", n), (w_q, "w_q", hidden * W), (w_gate, "w_gate", hidden * W),
             (w_k, "w_k", hidden * KW), (w_v, "w_v", hidden * KW), (w_o, "w_o", W * hidden),
             (q_norm, "q_norm", head_dim), (k_norm, "k_norm", head_dim),
             (mask, "mask", rows * length))]
    if out is None:
        out = _new_out(args[0], n)
    a_out = _Arg(out, np.float32, "out", n)
    flags = _flags(args + [a_out], ctx)
    if trim_leading:
        flags |= TFD_TRIM_LEADING
    _call(ctx, flags, ctx._lib.tfd_jeff_full_attention_layer_rows_f32,
          ctx.handle, rows, length, hidden, heads, kv_heads, head_dim, rotary_dim,
          *[a.ptr for a in args], f32_bits(theta), f32_bits(eps), a_out.ptr, flags)
    return a_out.obj
