"""The Laya decision model on the GPU.

Checkpoint loading mirrors laya-infer's host side: ``encoder/config.json``
(config.rs:136-235), ``rl_agent_config.json`` (config.rs:287-339) and
``model.safetensors`` with the name normalisation and strict consumption of
checkpoint.rs:47-340. Weights keep the file's bytes: a PyTorch ``(out, in)``
row-major linear is the host's ``(in, out)`` column-major matrix
(checkpoint.rs:9-18).

``LayaModel`` uploads the weights once (device-resident, torch allocations
as plumbing) and runs ``tfd_laya_forward_f32`` (include/tfd_laya_model.h),
the GPU forward of ``forward_reference`` (model.rs:867-977).
"""
from __future__ import annotations

import ctypes
import json
import math
import os
from dataclasses import dataclass, field
from typing import Dict, List, Optional

import numpy as np

from . import (TFD_EINVAL, Context, InvalidArgument, _Arg, _call, _flags,
               default_context, f32_bits)

ACTION_HIDDEN = 256  # checkpoint.rs:33


def _invalid(field_name: str, message: str) -> InvalidArgument:
    return InvalidArgument(TFD_EINVAL, f"invalid argument `{field_name}`: {message}")


# ------------------------------------------------------------------ configs


@dataclass
class EncoderConfig:
    """``EncoderConfig`` (config.rs:38-235): defaults and checks as there."""
    vocab_size: int
    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    num_attention_heads: int
    norm_eps: float = 1e-5
    norm_bias: bool = False
    attention_bias: bool = False
    mlp_bias: bool = False
    local_attention: int = 128
    global_attn_every_n_layers: int = 3
    global_rope_theta: float = 160000.0
    local_rope_theta: float = 10000.0
    max_position_embeddings: int = 8192
    layer_types: List[str] = field(default_factory=list)

    @classmethod
    def from_json(cls, obj: dict) -> "EncoderConfig":
        def req(key):
            v = obj.get(key)
            if not isinstance(v, int) or isinstance(v, bool) or v <= 0:
                raise _invalid(f"encoder.{key}", "expected a positive integer")
            return v

        layers = req("num_hidden_layers")
        every = obj.get("global_attn_every_n_layers", 3)
        if "layer_types" in obj and isinstance(obj["layer_types"], list):
            kinds = []
            for name in obj["layer_types"]:
                if name not in ("full_attention", "sliding_attention"):
                    raise _invalid("encoder.layer_types", f"unknown layer type `{name}`")
                kinds.append(name)
        else:
            kinds = ["full_attention" if every and i % every == 0 else "sliding_attention"
                     for i in range(layers)]
        cfg = cls(vocab_size=req("vocab_size"), hidden_size=req("hidden_size"),
                  intermediate_size=req("intermediate_size"), num_hidden_layers=layers,
                  num_attention_heads=req("num_attention_heads"),
                  norm_eps=float(obj.get("norm_eps", 1e-5)),
                  norm_bias=bool(obj.get("norm_bias", False)),
                  attention_bias=bool(obj.get("attention_bias", False)),
                  mlp_bias=bool(obj.get("mlp_bias", False)),
                  local_attention=int(obj.get("local_attention", 128)),
                  global_attn_every_n_layers=int(every),
                  global_rope_theta=float(obj.get("global_rope_theta", 160000.0)),
                  local_rope_theta=float(obj.get("local_rope_theta", 10000.0)),
                  max_position_embeddings=int(obj.get("max_position_embeddings", 8192)),
                  layer_types=kinds)
        model_type = obj.get("model_type", "modernbert")
        if model_type != "modernbert":
            raise _invalid("encoder.model_type", f"expected `modernbert`, found `{model_type}`")
        act = obj.get("hidden_activation", "gelu")
        if act != "gelu":
            raise _invalid("encoder.hidden_activation", f"expected `gelu`, found `{act}`")
        if cfg.hidden_size % cfg.num_attention_heads != 0:
            raise _invalid("encoder.hidden_size",
                           "hidden_size must be divisible by num_attention_heads")
        if (cfg.hidden_size // cfg.num_attention_heads) % 2 != 0:
            raise _invalid("encoder.num_attention_heads",
                           "the attention head dimension must be even for RoPE")
        if len(kinds) != layers:
            raise _invalid("encoder.layer_types",
                           f"expected {layers} entries, found {len(kinds)}")
        if cfg.global_attn_every_n_layers == 0:
            raise _invalid("encoder.global_attn_every_n_layers", "must be positive")
        return cfg

    def rope_base(self, kind: str) -> float:
        return self.global_rope_theta if kind == "full_attention" else self.local_rope_theta


@dataclass
class AgentConfig:
    """``AgentConfig`` (config.rs:250-339)."""
    head_layers: int
    max_len: int = 512
    head_max_len: int = 192
    action_names: List[str] = field(default_factory=list)

    @classmethod
    def from_json(cls, obj: dict) -> "AgentConfig":
        if not isinstance(obj.get("head_layers"), int):
            raise _invalid("rl_agent.head_layers", "missing `head_layers`")
        costs = obj.get("act_costs")
        if isinstance(costs, dict):
            names = sorted(costs)  # serde_json's map iterates its keys in order
        elif isinstance(costs, list):
            if not all(isinstance(x, str) for x in costs):
                raise _invalid("rl_agent.act_costs", "array entries must be strings")
            names = list(costs)
        elif costs is None:
            names = []
        else:
            raise _invalid("rl_agent.act_costs", "expected an object or array")
        return cls(head_layers=obj["head_layers"], max_len=int(obj.get("max_len", 512)),
                   head_max_len=int(obj.get("head_max_len", 192)), action_names=names)

    def action_count(self) -> int:
        return len(self.action_names) + 1

    def validate(self, enc: EncoderConfig) -> None:
        if not (4 < self.head_max_len < self.max_len):
            raise _invalid("rl_agent.head_max_len", "expected 4 < head_max_len < max_len")
        if self.max_len > enc.max_position_embeddings:
            raise _invalid("rl_agent.max_len", "max_len exceeds max_position_embeddings")


# ------------------------------------------------------------------ checkpoint


def _normalize_name(name: str) -> str:
    """checkpoint.rs:71-83."""
    name = name.replace(".in_proj_weight", ".in_proj.weight").replace(".in_proj_bias",
                                                                      ".in_proj.bias")
    for prefix in ("scorer", "act_head"):
        if name.startswith(prefix + ".") and not name.startswith(prefix + ".layers."):
            name = f"{prefix}.layers.{name[len(prefix) + 1:]}"
    return name


class _TensorSet:
    """Tensors by normalised name, each consumed exactly once (checkpoint.rs:86-168)."""

    def __init__(self, tensors: Dict[str, np.ndarray]):
        self.tensors = tensors
        self.originals: Dict[str, str] = {}
        for name in tensors:
            norm = _normalize_name(name)
            if norm in self.originals:
                raise _invalid("checkpoint.tensor",
                               f"duplicate parameter `{norm}` after conversion (from "
                               f"`{self.originals[norm]}` and `{name}`)")
            self.originals[norm] = name
        self.used = set()

    def take(self, name: str, shape) -> np.ndarray:
        original = self.originals.get(name)
        if original is None:
            raise _invalid("checkpoint.tensor", f"missing checkpoint parameter `{name}`")
        if original in self.used:
            raise _invalid("checkpoint.tensor", f"parameter `{name}` is referenced more than once")
        self.used.add(original)
        t = self.tensors[original]
        if list(t.shape) != list(shape):
            raise _invalid("checkpoint.tensor",
                           f"parameter `{name}` has shape {list(t.shape)}, expected {list(shape)}")
        return np.ascontiguousarray(t, dtype=np.float32).reshape(-1)

    def finish(self) -> None:
        for name in self.tensors:
            if name != "temperature" and name not in self.used:
                raise _invalid("checkpoint.tensor", f"unexpected checkpoint parameter `{name}`")


@dataclass
class LayaCheckpoint:
    encoder: EncoderConfig
    agent: AgentConfig
    # Host-layout f32 weights by canonical key: "tok_embeddings", "embed_norm.w",
    # "layers.{i}.wqkv", "head.{i}.in_proj.b", "act1.w", ... (see build_weights).
    weights: Dict[str, Optional[np.ndarray]]
    head_heads: int

    @property
    def hidden(self) -> int:
        return self.encoder.hidden_size


def build_weights(enc: EncoderConfig, agent: AgentConfig, ts: _TensorSet):
    """checkpoint.rs:200-330: the expected tensors, in the reference's order."""
    d, inter = enc.hidden_size, enc.intermediate_size
    w: Dict[str, Optional[np.ndarray]] = {}

    def norm(key, name, bias):
        w[key + ".w"] = ts.take(name + ".weight", [d])
        w[key + ".b"] = ts.take(name + ".bias", [d]) if bias else None

    def linear(key, name, n_in, n_out, bias):
        w[key + ".w"] = ts.take(name + ".weight", [n_out, n_in])
        w[key + ".b"] = ts.take(name + ".bias", [n_out]) if bias else None

    w["tok_embeddings"] = ts.take("encoder.embeddings.tok_embeddings.weight", [enc.vocab_size, d])
    norm("embed_norm", "encoder.embeddings.norm", enc.norm_bias)
    for i in range(enc.num_hidden_layers):
        p = f"encoder.layers.{i}"
        if i == 0:  # the first layer's attention normalisation is the identity
            w[f"layers.{i}.attn_norm.w"] = w[f"layers.{i}.attn_norm.b"] = None
        else:
            norm(f"layers.{i}.attn_norm", p + ".attn_norm", enc.norm_bias)
        linear(f"layers.{i}.wqkv", p + ".attn.Wqkv", d, 3 * d, enc.attention_bias)
        linear(f"layers.{i}.wo", p + ".attn.Wo", d, d, enc.attention_bias)
        norm(f"layers.{i}.mlp_norm", p + ".mlp_norm", enc.norm_bias)
        linear(f"layers.{i}.wi", p + ".mlp.Wi", d, 2 * inter, enc.mlp_bias)
        linear(f"layers.{i}.wo_mlp", p + ".mlp.Wo", inter, d, enc.mlp_bias)
    norm("final_norm", "encoder.final_norm", enc.norm_bias)
    for i in range(agent.head_layers):
        p = f"head.layers.{i}"
        norm(f"head.{i}.norm1", p + ".norm1", True)
        linear(f"head.{i}.in_proj", p + ".self_attn.in_proj", d, 3 * d, True)
        linear(f"head.{i}.out_proj", p + ".self_attn.out_proj", d, d, True)
        norm(f"head.{i}.norm2", p + ".norm2", True)
        linear(f"head.{i}.linear1", p + ".linear1", d, 4 * d, True)
        linear(f"head.{i}.linear2", p + ".linear2", 4 * d, d, True)
    w["type_emb"] = ts.take("type_emb.weight", [3, d])
    norm("scorer_norm", "scorer.layers.0", True)
    linear("scorer1", "scorer.layers.1", d, d, True)
    linear("scorer2", "scorer.layers.3", d, 1, True)
    linear("act1", "act_head.layers.0", d + 4, ACTION_HIDDEN, True)
    linear("act2", "act_head.layers.2", ACTION_HIDDEN, agent.action_count(), True)
    return w


def load_checkpoint(directory: str) -> LayaCheckpoint:
    """load_checkpoint (checkpoint.rs:57-69)."""
    from safetensors.numpy import load_file

    with open(os.path.join(directory, "encoder", "config.json")) as f:
        enc = EncoderConfig.from_json(json.load(f))
    with open(os.path.join(directory, "rl_agent_config.json")) as f:
        agent = AgentConfig.from_json(json.load(f))
    agent.validate(enc)
    ts = _TensorSet(load_file(os.path.join(directory, "model.safetensors")))
    weights = build_weights(enc, agent, ts)
    ts.finish()
    return LayaCheckpoint(enc, agent, weights, max(1, enc.hidden_size // 64))


# ------------------------------------------------------------------ C structs

_P = ctypes.c_void_p
_S = ctypes.c_size_t


class _EncoderLayer(ctypes.Structure):
    _fields_ = [("sliding", ctypes.c_int), ("rope_base_bits", ctypes.c_uint32)] + [
        (n, _P) for n in ("attn_norm_w", "attn_norm_b", "wqkv", "bqkv", "wo", "bo", "mlp_norm_w",
                          "mlp_norm_b", "wi", "bi", "wo_mlp", "bo_mlp")]


class _HeadLayer(ctypes.Structure):
    _fields_ = [("heads", _S), ("ff", _S)] + [
        (n, _P) for n in ("norm1_w", "norm1_b", "in_proj_w", "in_proj_b", "out_proj_w",
                          "out_proj_b", "norm2_w", "norm2_b", "linear1_w", "linear1_b",
                          "linear2_w", "linear2_b")]


class _Model(ctypes.Structure):
    _fields_ = [(n, _S) for n in ("hidden", "heads", "intermediate", "vocab", "window")] + [
        ("eps_bits", ctypes.c_uint32)] + [
        (n, _S) for n in ("n_layers", "n_head_layers", "action_hidden", "actions")] + [
        ("tok_embeddings", _P), ("embed_norm_w", _P), ("embed_norm_b", _P),
        ("layers", ctypes.POINTER(_EncoderLayer)), ("final_norm_w", _P), ("final_norm_b", _P),
        ("head", ctypes.POINTER(_HeadLayer))] + [
        (n, _P) for n in ("type_emb", "scorer_norm_w", "scorer_norm_b", "scorer1_w", "scorer1_b",
                          "scorer2_w", "scorer2_b", "act1_w", "act1_b", "act2_w", "act2_b")]


class LayaModel:
    """A checkpoint resident on one GPU, run by tfd_laya_forward_f32."""

    def __init__(self, ckpt: LayaCheckpoint, *, ctx: Optional[Context] = None, device: int = 0):
        import torch

        self.ckpt = ckpt
        self.ctx = ctx or default_context()
        dev = torch.device("cuda", device)
        self._dev = {k: (torch.from_numpy(v).to(dev) if v is not None else None)
                     for k, v in ckpt.weights.items()}
        # The uploads run on torch's stream; the forward reads the weights on
        # the context's stream, so they must have landed first.
        torch.cuda.synchronize(dev)
        ptr = lambda k: self._dev[k].data_ptr() if self._dev.get(k) is not None else None
        enc, agent = ckpt.encoder, ckpt.agent
        d = enc.hidden_size
        self._layers = (_EncoderLayer * max(1, enc.num_hidden_layers))()
        for i, kind in enumerate(enc.layer_types):
            L = self._layers[i]
            L.sliding = 0 if kind == "full_attention" else 1
            L.rope_base_bits = f32_bits(enc.rope_base(kind))
            for fld, key in (("attn_norm_w", "attn_norm.w"), ("attn_norm_b", "attn_norm.b"),
                             ("wqkv", "wqkv.w"), ("bqkv", "wqkv.b"), ("wo", "wo.w"), ("bo", "wo.b"),
                             ("mlp_norm_w", "mlp_norm.w"), ("mlp_norm_b", "mlp_norm.b"),
                             ("wi", "wi.w"), ("bi", "wi.b"), ("wo_mlp", "wo_mlp.w"),
                             ("bo_mlp", "wo_mlp.b")):
                setattr(L, fld, ptr(f"layers.{i}.{key}"))
        self._head = (_HeadLayer * max(1, agent.head_layers))()
        for i in range(agent.head_layers):
            H = self._head[i]
            H.heads = ckpt.head_heads
            H.ff = 4 * d
            for part in ("norm1", "in_proj", "out_proj", "norm2", "linear1", "linear2"):
                setattr(H, part + "_w", ptr(f"head.{i}.{part}.w"))
                setattr(H, part + "_b", ptr(f"head.{i}.{part}.b"))
        m = _Model()
        m.hidden, m.heads, m.intermediate = d, enc.num_attention_heads, enc.intermediate_size
        m.vocab, m.window = enc.vocab_size, enc.local_attention // 2
        m.eps_bits = f32_bits(enc.norm_eps)
        m.n_layers, m.n_head_layers = enc.num_hidden_layers, agent.head_layers
        m.action_hidden, m.actions = ACTION_HIDDEN, agent.action_count()
        m.tok_embeddings = ptr("tok_embeddings")
        m.embed_norm_w, m.embed_norm_b = ptr("embed_norm.w"), ptr("embed_norm.b")
        m.layers = ctypes.cast(self._layers, ctypes.POINTER(_EncoderLayer))
        m.final_norm_w, m.final_norm_b = ptr("final_norm.w"), ptr("final_norm.b")
        m.head = ctypes.cast(self._head, ctypes.POINTER(_HeadLayer))
        m.type_emb = ptr("type_emb")
        for part in ("scorer_norm", "scorer1", "scorer2", "act1", "act2"):
            setattr(m, part + "_w", ptr(part + ".w"))
            setattr(m, part + "_b", ptr(part + ".b"))
        self._model = m

    def forward(self, ids, mask, marker_pos, marker_mask, qtype, *, logits=None, action=None):
        """forward_reference (model.rs:867-977): ids, mask (L, B) and marker_pos,
        marker_mask (K, B) column-major host arrays, qtype (B). Returns the masked
        marker logits (K, B) and the action logits (actions, B), flat column-major
        (numpy, or the given device tensors)."""
        ids = np.ascontiguousarray(ids, dtype=np.int64).reshape(-1)
        mask = np.ascontiguousarray(mask, dtype=bool).astype(np.uint8).reshape(-1)
        marker_pos = np.ascontiguousarray(marker_pos, dtype=np.int64).reshape(-1)
        marker_mask = np.ascontiguousarray(marker_mask, dtype=bool).astype(np.uint8).reshape(-1)
        qtype = np.ascontiguousarray(qtype, dtype=np.int64).reshape(-1)
        B = len(qtype)
        if B and (len(ids) % B or len(marker_pos) % B):
            raise _invalid("laya.ids", "ids must be a non-empty (L, B) batch")
        if len(mask) != len(ids):
            raise _invalid("laya.mask", "mask length must match the token batch")
        if len(marker_mask) != len(marker_pos):
            raise _invalid("laya.marker_mask", "marker_mask must match marker_pos")
        L = len(ids) // B if B else 0
        K = len(marker_pos) // B if B else 0
        A = self.ckpt.agent.action_count()
        if logits is None and action is None:
            logits = np.zeros(K * B, np.float32)
            action = np.zeros(A * B, np.float32)
        elif logits is None or action is None:
            raise _invalid("laya.logits", "pass both outputs (logits and action) or neither")
        # Outputs decide the pointer kind (token inputs are always host arrays):
        # both host arrays, or both CUDA tensors on the model's device; checked
        # before any device call.
        a_log = _Arg(logits, np.float32, "logits", K * B)
        a_act = _Arg(action, np.float32, "action", A * B)
        flags = _flags([a_log, a_act], self.ctx)
        c = self.ctx
        _call(c, flags, c._lib.tfd_laya_forward_f32,
              c.handle, ctypes.byref(self._model), ids.ctypes.data, mask.ctypes.data, L, B,
              marker_pos.ctypes.data, marker_mask.ctypes.data, K, qtype.ctypes.data, a_log.ptr,
              a_act.ptr, flags)
        return a_log.obj, a_act.obj
