"""The Laya decision-model forward (laya-infer model.rs:867-977) end to end.

Golden vector: ``fixtures/laya-tiny`` (checkpoint + ``reference.json``, the
Julia reference's outputs; native_fixture.rs:75-139 asserts 1e-5), copied
under tests/golden/laya_tiny as data.

CPU: the checkpoint loader's rules; the oracle (oracle/laya_model.py, f32 and
f64) against reference.json; the oracle against an independent assembly from
library modules (tests/laya_modules.py: transformers' ModernBertModel,
torch's TransformerEncoderLayer, nn.Linear/LayerNorm/GELU) on random weights
where every component moves the outputs, with planted mistakes that the
comparison must catch; argument validation of the C entry before any device
access. GPU: tfd_laya_forward_f32 against reference.json and the oracle.
"""
import ctypes
import json
import os

import numpy as np
import pytest

import tenferro_ext as te
from oracle import laya_model as om
from tenferro_ext import laya_model as tlm
from tenferro_ext.workloads import laya_model_batch, laya_model_checkpoint

HERE = os.path.dirname(os.path.abspath(__file__))
TINY = os.path.join(HERE, "golden", "laya_tiny")
TOL = 1e-5  # native_fixture.rs:130-137


@pytest.fixture(scope="module")
def tiny():
    ckpt = tlm.load_checkpoint(TINY)
    with open(os.path.join(TINY, "reference.json")) as f:
        ref = json.load(f)
    batch = (np.array(ref["input_ids"][0]), np.array(ref["attention_mask"][0]),
             np.array(ref["marker_pos"][0]), np.array(ref["marker_mask"][0]),
             np.array(ref["qtype"]))
    return ckpt, batch, np.array(ref["logits"][0], np.float32), np.array(ref["action"][0],
                                                                          np.float32)


@pytest.fixture(scope="module")
def random_case():
    ckpt = laya_model_checkpoint()
    return ckpt, laya_model_batch(40, 3, 4, ckpt.encoder.vocab_size)


def oracle_forward(ckpt, batch, **kw):
    return om.forward(ckpt.encoder, ckpt.agent.action_count(), ckpt.weights, ckpt.head_heads,
                      *batch, **kw)


# ------------------------------------------------------------------ CPU


def test_checkpoint_loader_reads_the_fixture(tiny):
    ckpt = tiny[0]
    e = ckpt.encoder
    assert (e.hidden_size, e.num_attention_heads, e.intermediate_size, e.num_hidden_layers) == \
        (32, 2, 48, 2)
    assert e.layer_types == ["full_attention", "sliding_attention"]  # every 3rd layer global
    assert (e.local_attention, e.global_rope_theta, e.local_rope_theta) == (16, 160000.0, 10000.0)
    assert ckpt.agent.action_count() == 2 and ckpt.head_heads == 1
    w = ckpt.weights
    assert w["layers.0.attn_norm.w"] is None and w["layers.1.attn_norm.w"].shape == (32,)
    assert w["layers.0.wqkv.w"].shape == (32 * 96,) and w["layers.0.wqkv.b"] is None
    assert w["act1.w"].shape == (36 * 256,) and w["act2.b"].shape == (2,)


def test_checkpoint_loader_rules():
    """checkpoint.rs:71-168: name normalisation, exact shapes, each tensor once,
    nothing left over except `temperature`."""
    t = {"scorer.0.weight": np.zeros(4, np.float32),
         "x.in_proj_weight": np.zeros((2, 2), np.float32),
         "temperature": np.zeros(1, np.float32), "extra": np.zeros(1, np.float32)}
    ts = tlm._TensorSet(t)
    assert ts.take("scorer.layers.0.weight", [4]).shape == (4,)
    assert ts.take("x.in_proj.weight", [2, 2]).shape == (4,)
    with pytest.raises(te.InvalidArgument, match="referenced more than once"):
        ts.take("scorer.layers.0.weight", [4])
    with pytest.raises(te.InvalidArgument, match="unexpected checkpoint parameter `extra`"):
        ts.finish()
    with pytest.raises(te.InvalidArgument, match="has shape"):
        tlm._TensorSet({"a": np.zeros(3, np.float32)}).take("a", [4])
    with pytest.raises(te.InvalidArgument, match="duplicate parameter"):
        tlm._TensorSet({"scorer.0.weight": np.zeros(1), "scorer.layers.0.weight": np.zeros(1)})


@pytest.mark.parametrize("f64", [False, True])
def test_oracle_matches_reference_json(oracle_lib, tiny, f64):
    ckpt, batch, want_logits, want_action = tiny
    logits, action = oracle_forward(ckpt, batch, f64=f64)
    assert np.abs(logits - want_logits).max() < TOL
    assert np.abs(action - want_action).max() < TOL


def test_module_assembly_matches_reference_json(tiny):
    import laya_modules as lm

    ckpt, batch, want_logits, want_action = tiny
    logits, action = lm.forward(ckpt, *batch)
    assert np.abs(logits.reshape(-1) - want_logits).max() < TOL
    assert np.abs(action.reshape(-1) - want_action).max() < TOL


def test_oracle_encoder_matches_modernbert(oracle_lib, tiny, random_case):
    import laya_modules as lm

    ckpt, batch = tiny[0], tiny[1]
    got = om.encoder(ckpt.encoder, ckpt.weights, batch[0], batch[1], 1)
    want = lm.encode(ckpt.encoder, ckpt.weights, batch[0], batch[1], 1).numpy().reshape(-1)
    assert np.abs(got - want).max() < TOL
    ckpt, (ids, mask, *_rest) = random_case
    B, L = 3, 40
    got = om.encoder(ckpt.encoder, ckpt.weights, ids, mask, B).reshape(B, L, -1)
    want = lm.encode(ckpt.encoder, ckpt.weights, ids, mask, B).numpy()
    v = mask.reshape(B, L)
    assert np.abs(want[v]).max() > 1.0  # outputs of unit scale
    assert np.abs(got - want)[v].max() < 2 * TOL


@pytest.fixture(scope="module")
def module_random(random_case):
    import laya_modules as lm

    ckpt, batch = random_case
    logits, action = lm.forward(ckpt, *batch)
    return logits.reshape(-1), action.reshape(-1)


def test_oracle_matches_module_assembly(oracle_lib, random_case, module_random):
    ckpt, batch = random_case
    logits, action = oracle_forward(ckpt, batch)
    assert np.abs(logits - module_random[0]).max() < TOL
    assert np.abs(action - module_random[1]).max() < TOL
    assert (logits == -1.0e4).sum() == 1  # the masked slot of row 1


def test_edge_batch_reads_padded_columns(oracle_lib, random_case):
    """The module assembly and the oracle agree where the outputs read padded
    columns (token 0 padded, a marker on a padded position, a negative
    marker position): those states are computed like any other."""
    import laya_modules as lm

    ckpt = random_case[0]
    batch = edge_batch(ckpt.encoder.vocab_size)
    logits, action = oracle_forward(ckpt, batch)
    # the module assembly zeroes padded states (see laya_modules); compare
    # only what does not read them: prompt 2's other markers
    m_logits, _ = lm.forward(ckpt, *batch)
    assert np.abs(logits[9:12] - m_logits.reshape(-1)[9:12]).max() < TOL
    assert np.isfinite(logits).all() and np.isfinite(action).all()


@pytest.mark.parametrize("plant", ["no_embed_norm", "tanh_gelu", "no_mlp", "swap_geglu",
                                   "no_head_layer", "qtype0", "no_rope", "global_only"])
def test_planted_mistakes_are_caught(oracle_lib, random_case, module_random, plant):
    """Each mistake, planted in the oracle, moves the outputs far past TOL on
    these inputs; so the same comparison would catch it in the GPU path."""
    ckpt, batch = random_case
    logits, action = oracle_forward(ckpt, batch, plant=plant)
    err = max(np.abs(logits - module_random[0]).max(), np.abs(action - module_random[1]).max())
    assert err > 10 * TOL


def _host_model():
    """A tfd_laya_model whose pointers are non-null host addresses: enough
    for the entry's validation, which runs before any device access."""
    keep = np.zeros(16, np.float32)
    p = keep.ctypes.data
    layers = (tlm._EncoderLayer * 2)()
    for i in range(2):
        for name, _ in tlm._EncoderLayer._fields_[2:]:
            setattr(layers[i], name, p)
        layers[i].rope_base_bits = te.f32_bits(10000.0)
    head = (tlm._HeadLayer * 1)()
    head[0].heads, head[0].ff = 1, 128
    for name, _ in tlm._HeadLayer._fields_[2:]:
        setattr(head[0], name, p)
    m = tlm._Model()
    m.hidden, m.heads, m.intermediate, m.vocab, m.window = 32, 2, 48, 263, 8
    m.eps_bits = te.f32_bits(1e-5)
    m.n_layers, m.n_head_layers, m.action_hidden, m.actions = 2, 1, 256, 2
    for name, typ in tlm._Model._fields_:
        if typ is ctypes.c_void_p:
            setattr(m, name, p)
    m.layers = ctypes.cast(layers, ctypes.POINTER(tlm._EncoderLayer))
    m.head = ctypes.cast(head, ctypes.POINTER(tlm._HeadLayer))
    return m, (keep, layers, head)


@pytest.mark.parametrize("case,field,msg", [
    ("empty", "laya.qtype", "the batch must be non-empty"),
    ("vocab", "laya.ids", "token id is outside the vocabulary"),
    ("qtype", "laya.qtype", "qtype must be 0 (choice), 1 (score) or 2 (noul)"),
    ("markers", "laya.marker_pos", "at least two marker slots are required"),
    ("heads", "laya.layers[0].num_heads", "must divide hidden_size"),
    ("flags", "flags", "TFD_ASYNC requires TFD_DEVICE_PTRS"),
])
def test_forward_validates_before_gpu(case, field, msg):
    """forward_reference's checks (model.rs:877-911, 661-669, 920-927) and
    LayaWeights::validate (187-295), in this container (no GPU)."""
    ctx = te.Context(0)
    m, _keep = _host_model()
    L, B, K = 8, 1, 3
    ids = np.arange(L, dtype=np.int64)
    mask = np.ones(L, np.uint8)
    mp = np.array([1, 3, 5], np.int64)
    mm = np.ones(K, np.uint8)
    qt = np.zeros(B, np.int64)
    out = np.zeros(8, np.float32)
    flags = 0
    if case == "empty":
        B = 0
    elif case == "vocab":
        ids[3] = 263
    elif case == "qtype":
        qt[0] = 3
    elif case == "markers":
        K = 1
    elif case == "heads":
        m.heads = 3
    elif case == "flags":
        flags = te.TFD_ASYNC
    rc = ctx._lib.tfd_laya_forward_f32(ctx.handle, ctypes.byref(m), ids.ctypes.data,
                                       mask.ctypes.data, L, B, mp.ctypes.data, mm.ctypes.data, K,
                                       qt.ctypes.data, out.ctypes.data, out.ctypes.data, flags)
    err = ctx._lib.tfd_last_error(ctx.handle).decode()
    assert rc == te.TFD_EINVAL and f"`{field}`" in err and msg in err, err
    ctx.close()


def test_forward_output_kinds_checked_before_gpu(tiny):
    """LayaModel.forward picks host or device pointers from its outputs: a
    missing output, a short one, or a host array next to a device tensor is
    refused before any device call (the model is assembled without uploading
    weights; a stand-in object reports itself as a CUDA tensor)."""

    class FakeCuda:
        __module__ = "torch.fake"
        dtype = "torch.float32"
        is_cuda = True

        def __init__(self, n):
            self._n = n

        def is_contiguous(self):
            return True

        def data_ptr(self):
            return 1 << 40

        def numel(self):
            return self._n

    ckpt = tiny[0]
    model = tlm.LayaModel.__new__(tlm.LayaModel)
    model.ckpt, model.ctx = ckpt, te.Context(0)
    ids, mask, pos, mm, qt = laya_model_batch(8, 1, 3, ckpt.encoder.vocab_size, seed=3)
    A = ckpt.agent.action_count()
    with pytest.raises(te.InvalidArgument, match="both outputs"):
        model.forward(ids, mask, pos, mm, qt, logits=np.zeros(3, np.float32))
    with pytest.raises(te.InvalidArgument, match="logits: 2 elements"):
        model.forward(ids, mask, pos, mm, qt, logits=np.zeros(2, np.float32),
                      action=np.zeros(A, np.float32))
    with pytest.raises(te.InvalidArgument, match="mix of host arrays and device tensors"):
        model.forward(ids, mask, pos, mm, qt, logits=np.zeros(3, np.float32),
                      action=FakeCuda(A))
    model.ctx.close()


# ------------------------------------------------------------------ GPU


@pytest.mark.gpu
def test_laya_tiny_forward_gpu(gpu_ctx, tiny):
    print("[laya-model] laya-tiny fixture", flush=True)
    ckpt, batch, want_logits, want_action = tiny
    model = tlm.LayaModel(ckpt, ctx=gpu_ctx)
    logits, action = model.forward(*batch)
    assert np.abs(logits - want_logits).max() < TOL
    assert np.abs(action - want_action).max() < TOL
    o_logits, o_action = oracle_forward(ckpt, batch)
    assert np.abs(logits - o_logits).max() < TOL
    assert np.abs(action - o_action).max() < TOL


def edge_batch(vocab):
    """Padded columns that the outputs read: prompt 0 starts with 3 padded
    tokens (token 0 is pooled), prompt 1 has an unmasked marker on a padded
    position and prompt 2 a negative marker position (read as token 0)."""
    L, B, K = 40, 3, 4
    ids, mask, pos, mm, qtype = laya_model_batch(L, B, K, vocab, min_len=K + 2, seed=29)
    mask = mask.copy()
    pos = pos.copy()
    mm = mm.copy()
    mask[0:3] = False
    n1 = int(mask[L:2 * L].sum())
    pos[K + 2] = min(L - 1, n1 + 2)   # past prompt 1's last valid token
    mm[K + 2] = True
    assert not mask[L + pos[K + 2]]
    pos[2 * K] = -3
    mm[2 * K] = True
    return ids, mask, pos, mm, qtype


@pytest.mark.gpu
@pytest.mark.parametrize("shape", ["small", "wide", "edge"])
def test_random_forward_matches_oracle_gpu(gpu_ctx, shape):
    """Padded rows, sliding and global layers, masked marker slots, every
    qtype; device outputs (torch) on the second call."""
    import torch

    print(f"[laya-model] random {shape}", flush=True)
    if shape in ("small", "edge"):
        ckpt = laya_model_checkpoint()
        L, B, K = 40, 3, 4
    else:
        ckpt = laya_model_checkpoint(vocab=1000, hidden=768, intermediate=1152, layers=4,
                                     heads=12, local_attention=128, seed=21)
        L, B, K = 256, 4, 6
    batch = laya_model_batch(L, B, K, ckpt.encoder.vocab_size, min_len=K + 2)
    if shape == "edge":
        batch = edge_batch(ckpt.encoder.vocab_size)
    want_logits, want_action = oracle_forward(ckpt, batch)
    model = tlm.LayaModel(ckpt, ctx=gpu_ctx)
    logits, action = model.forward(*batch)
    tol = 1e-4 if shape == "wide" else 2 * TOL
    assert np.abs(logits - want_logits).max() < tol
    assert np.abs(action - want_action).max() < tol
    dl = torch.empty(K * B, dtype=torch.float32, device="cuda")
    da = torch.empty(ckpt.agent.action_count() * B, dtype=torch.float32, device="cuda")
    model.forward(*batch, logits=dl, action=da)
    assert np.array_equal(dl.cpu().numpy(), logits)
    assert np.array_equal(da.cpu().numpy(), action)
