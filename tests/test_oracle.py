"""CPU tests that pin the oracle (oracle/tfd_oracle.c) before it is trusted.

Each check is one the reference's own tests or the mathematics fixes:
known-answer tests from crates/tenferro-infer/tests/primitives.rs:299-519,
the cpu-kernels unit tests (crates/cpu-kernels/src/lib.rs:1205-1290), the
micro-benchmark's scalar-vs-tile assertion
(fixtures/bench-laya-attention-gemm-2026-10-09/microbenchmark.rs:142-210),
the laya-infer sweep (tests/model.rs:338-373), the jeff-infer op-vs-host test
(src/model.rs:1332-1404), invariants, and a float64 brute force that follows
the reference's host oracles rather than the kernels the C code restates.
"""
import math

import numpy as np
import pytest

from oracle import brute
from tenferro_ext.workloads import Lcg, laya_config


def rope_rotate_with_table(x, cos, sin, rot):
    """Rotate rows x[t] with the oracle's f32 table, pairs (i, i + rot/2)."""
    half = rot // 2
    y = x.astype(np.float32).copy()
    a, b = x[:, :half].astype(np.float32), x[:, half:2 * half].astype(np.float32)
    y[:, :half] = a * cos - b * sin
    y[:, half:2 * half] = a * sin + b * cos
    return y


# ----------------------------------------------------------------- generator

def test_lcg_jump_ahead_matches_sequential_loop():
    rng = Lcg(3)
    u = rng.uniform(20000)
    s, ref = 3, []
    for _ in range(20000):
        s = (s * 6364136223846793005 + 1442695040888963407) % (1 << 64)
        ref.append((s >> 40) / float(1 << 24))
    assert np.array_equal(u, np.array(ref))
    assert rng.state == s


# ----------------------------------------------------------------- RoPE KATs

def test_rope_table_modernbert_kat(oracle_lib):
    """primitives.rs:299-340: seq 3, head 4, base 10000."""
    seq, head, base = 3, 4, 10000.0
    xv = [1.0, 0.0, 0.0, 1.0, 2.0, 1.0, 3.0, 0.0, 0.5, -1.0, 2.0, 2.0]
    x = np.array([[xv[p + i * seq] for i in range(head)] for p in range(seq)])
    half = head // 2
    expected = np.zeros_like(x)
    for p in range(seq):
        for i in range(half):
            theta = p * base ** (-2.0 * i / head)
            first, second = x[p, i], x[p, i + half]
            expected[p, i] = first * math.cos(theta) - second * math.sin(theta)
            expected[p, i + half] = first * math.sin(theta) + second * math.cos(theta)
    cos, sin = oracle_lib.rope_table(seq, head, base)
    got = rope_rotate_with_table(x, cos, sin, head)
    assert np.abs(got - expected).max() <= 1e-6
    assert np.array_equal(got[0], x[0].astype(np.float32))  # position 0 unchanged


def test_rope_table_qwen_partial_kat(oracle_lib):
    """primitives.rs:342-372: heads 2, seq 3, head 4, rotary 2 (Jeff's angles
    t * theta^(-2i/rot) are the same table with dim = rot)."""
    heads, seq, head, rot, base = 2, 3, 4, 2, 10000.0
    data = np.array([i * 0.1 - 0.3 for i in range(heads * seq * head)])
    cos, sin = oracle_lib.rope_table(seq, rot, base)
    half = rot // 2
    for h in range(heads):
        x = np.array([[data[h + heads * t + heads * seq * d] for d in range(head)] for t in range(seq)])
        expected = x.copy()
        for t in range(seq):
            for i in range(half):
                ang = t * base ** (-2.0 * i / rot)
                f, s = x[t, i], x[t, i + half]
                expected[t, i] = f * math.cos(ang) - s * math.sin(ang)
                expected[t, i + half] = f * math.sin(ang) + s * math.cos(ang)
        got = rope_rotate_with_table(x, cos, sin, rot)
        assert np.abs(got - expected).max() <= 1e-6
        assert np.array_equal(got[:, rot:], x[:, rot:].astype(np.float32))


def test_rope_rotation_preserves_pair_norm(oracle_lib):
    cos, sin = oracle_lib.rope_table(64, 16, 160000.0)
    assert np.abs(cos ** 2 + sin ** 2 - 1.0).max() <= 1e-6
    assert np.all(cos[0] == 1.0) and np.all(sin[0] == 0.0)


# ----------------------------------------------------------------- attention KATs

def _laya_from_bhld(q, k, v, B, H, L, hd):
    """Pack (B, H, L, hd) column-major KAT tensors into Laya's (3d, L, B)."""
    d = H * hd
    idx = lambda b, h, l, i: b + B * h + B * H * l + B * H * L * i
    qkv = np.zeros(3 * d * L * B, np.float32)
    for b in range(B):
        for h in range(H):
            for l in range(L):
                for i in range(hd):
                    base = 3 * d * (l + L * b) + h * hd + i
                    qkv[base] = q[idx(b, h, l, i)]
                    qkv[base + d] = k[idx(b, h, l, i)]
                    qkv[base + 2 * d] = v[idx(b, h, l, i)]
    return qkv


def test_attention_masked_multi_head_kat(oracle_lib):
    """primitives.rs:374-443: b 1, h 2, l 2, hd 2, causal keep."""
    B, H, L, hd = 1, 2, 2, 2
    qv = [1.0, 0.0, 0.0, 1.0, 0.5, 0.5, 0.2, 0.4]
    kv = [1.0, 0.0, 0.0, 1.0, 0.3, 0.7, 0.1, 0.9]
    vv = [1.0, 2.0, 3.0, 4.0, 5.0, 6.0, 7.0, 8.0]
    qkv = _laya_from_bhld(qv, kv, vv, B, H, L, hd)
    keep = np.array([1, 1, 0, 1], np.uint8)  # keep[q + L*k] = k <= q
    out = oracle_lib.laya_attention_block(qkv, keep, H * hd, H, L, B, 0.0)
    idx = lambda hh, ll, d: hh + ll * H + d * H * L
    scale = 1.0 / math.sqrt(hd)
    for hh in range(H):
        for qq in range(L):
            scores = [sum(qv[idx(hh, qq, d)] * kv[idx(hh, kk, d)] for d in range(hd)) * scale
                      if kk <= qq else -math.inf for kk in range(L)]
            mx = max(scores)
            ex = [math.exp(s - mx) if math.isfinite(s) else 0.0 for s in scores]
            tot = sum(ex)
            for d in range(hd):
                want = sum(vv[idx(hh, kk, d)] * ex[kk] / tot for kk in range(L))
                got = out[hh * hd + d + H * hd * qq]
                assert abs(got - want) <= 1e-6


def test_attention_unmasked_kat(oracle_lib):
    """primitives.rs:482-519."""
    q = [1.0, 0.0, 0.0, 1.0]
    k = [1.0, 0.0, 0.0, 1.0]
    v = [1.0, 2.0, 3.0, 4.0]
    qkv = _laya_from_bhld(q, k, v, 1, 1, 2, 2)
    out = oracle_lib.laya_attention_block(qkv, np.ones(4, np.uint8), 2, 1, 2, 1, 0.0)
    s = 1.0 / math.sqrt(2.0)
    e0, e1 = math.exp(s - s), math.exp(0.0 - s)
    p = [[e0 / (e0 + e1), e1 / (e0 + e1)], [e1 / (e0 + e1), e0 / (e0 + e1)]]
    vv = [[1.0, 3.0], [2.0, 4.0]]
    for l in range(2):
        for d in range(2):
            assert abs(out[d + 2 * l] - (p[l][0] * vv[0][d] + p[l][1] * vv[1][d])) <= 1e-6


# ----------------------------------------------------------------- cpu-kernels unit tests

def test_laya_rejects_short_storage(oracle_lib):
    """lib.rs:1205-1210: short qkv storage is rejected before any access."""
    with pytest.raises(ValueError, match="qkv length"):
        oracle_lib.laya_attention_block(np.zeros(0, np.float32), np.ones(32 * 32, np.uint8),
                                        4, 1, 32, 1, 0.0, out=np.zeros(4 * 32, np.float32))


def nonfinite_case(length=65, d=4):
    """lib.rs:1212-1250: key 32 masked for every query, keys' V = feature+1,
    queries 0 and L-1 keep nothing."""
    qkv = np.zeros(3 * d * length, np.float32)
    for key in range(length):
        for f in range(d):
            qkv[3 * d * key + 2 * d + f] = f + 1
    keep = np.ones(length * length, np.uint8)
    for query in range(length):
        keep[query + length * 32] = 0
    for key in range(length):
        keep[length * key] = 0
        keep[length - 1 + length * key] = 0
    return qkv, keep


@pytest.mark.parametrize("excluded", [1.0, float("nan"), float("inf")])
def test_laya_masked_nonfinite_values_and_empty_rows(oracle_lib, excluded):
    length, d = 65, 4
    qkv, keep = nonfinite_case(length, d)
    qkv[3 * d * 32 + 2 * d:3 * d * 32 + 3 * d] = excluded
    out = oracle_lib.laya_attention_block(qkv, keep, d, 1, length, 1, 0.0).reshape(length, d)
    assert np.all(np.isnan(out[0])) and np.all(np.isnan(out[length - 1]))
    want = np.arange(1, d + 1, dtype=np.float32)
    assert np.abs(out[1:length - 1] - want).max() <= 1e-6


def test_laya_deterministic_across_calls_and_threads(oracle_lib):
    """lib.rs:1252-1290 requires bitwise-equal results with a reused workspace;
    here repeated calls and different thread counts must agree bit for bit."""
    rng = Lcg(654321)
    for length, batch, heads, base in [(8, 8, 2, 10000.0), (65, 2, 2, 10000.0), (3, 1, 1, 160000.0),
                                        (32, 3, 4, 0.0), (65, 2, 2, 160000.0)]:
        d = 8
        qkv = (rng.uniform(3 * d * length * batch) - 0.5).astype(np.float32)
        keep = (np.arange(length * length * batch) % 7 != 0).astype(np.uint8)
        oracle_lib.set_threads(1)
        a = oracle_lib.laya_attention_block(qkv, keep, d, heads, length, batch, base)
        oracle_lib.set_threads(8)
        b = oracle_lib.laya_attention_block(qkv, keep, d, heads, length, batch, base)
        c = oracle_lib.laya_attention_block(qkv, keep, d, heads, length, batch, base)
        for x in (b, c):
            assert np.array_equal(a.view(np.uint32), x.view(np.uint32)) or (
                np.array_equal(np.isnan(a), np.isnan(x)) and np.array_equal(a[~np.isnan(a)], x[~np.isnan(x)]))


def test_laya_zero_output_when_heads_do_not_divide(oracle_lib):
    """lib.rs:870-872 returns early; the op's freshly zeroed output stays 0."""
    out = oracle_lib.laya_attention_block(np.ones(3 * 6 * 4, np.float32), np.ones(16, np.uint8),
                                          6, 4, 4, 1, 0.0)
    assert np.all(out == 0.0)


# ----------------------------------------------------------------- tile vs scalar policy

@pytest.mark.parametrize("length", [31, 32, 33, 63, 64, 65, 128, 129])
@pytest.mark.parametrize("window", [None, 1, 64])
def test_laya_tile_path_matches_scalar_path(oracle_lib, length, window):
    """microbenchmark.rs:142-210: d 1024, 16 heads, rope 160000, keys k%13 != 7,
    optionally |q-k| <= w; the reference asserts error <= 1e-5 and all finite."""
    d, heads, batch = 1024, 16, 1
    qkv = (((np.arange(3 * d * length * batch) * 17) % 101).astype(np.float32) - 50.0) * 0.002
    i = np.arange(length * length * batch)
    q, k = i % length, (i // length) % length
    keep = (k % 13 != 7) & (True if window is None else (np.abs(q - k) <= window))
    keep = keep.astype(np.uint8)
    tile = oracle_lib.laya_attention_block(qkv, keep, d, heads, length, batch, 160000.0)
    scalar = oracle_lib.laya_attention_block(qkv, keep, d, heads, length, batch, 160000.0,
                                             scalar_only=True)
    assert np.all(np.isfinite(tile)) and np.all(np.isfinite(scalar))
    assert np.abs(tile - scalar).max() <= 1e-5


# ----------------------------------------------------------------- brute force sweep

def encoder_valid(length, batch, sparse):
    """laya-infer tests/model.rs:160-179 masks (and the sparse variant of 349-353)."""
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


@pytest.mark.parametrize("length", [31, 32, 33, 63, 64, 65, 127, 129])
@pytest.mark.parametrize("local_attention", [2, 128])
@pytest.mark.parametrize("sparse", [False, True])
def test_laya_oracle_matches_brute_force_sweep(oracle_lib, length, local_attention, sparse):
    """model.rs:338-373 shapes (bound 3e-5): global layer at rope 160000 and
    sliding layer (window = local_attention/2) at rope 10000, padded rows."""
    d, heads, batch = 8, 2, 2
    rng = Lcg(67 + length)
    qkv = (rng.uniform(3 * d * length * batch) * 2.0 - 1.0).astype(np.float32)
    valid = encoder_valid(length, batch, sparse)
    for window, base in ((-1, 160000.0), (local_attention // 2, 10000.0)):
        keep = oracle_lib.laya_build_mask(valid, length, batch, window)
        got = oracle_lib.laya_attention_block(qkv, keep, d, heads, length, batch, base)
        want = brute.laya_attention_host(qkv, keep, d, heads, length, batch, base)
        assert np.array_equal(np.isnan(got), np.isnan(want))
        ok = ~np.isnan(want)
        assert np.abs(got[ok] - want[ok]).max() <= 3e-5


@pytest.mark.parametrize("cfg", [1])
def test_laya_config_matches_brute_force(oracle_lib, cfg):
    w = laya_config(cfg)
    got = oracle_lib.laya_attention_block(w.qkv, w.keep, w.hidden, w.heads, w.length, w.batch,
                                          w.rope_base)
    want = brute.laya_attention_host(w.qkv, w.keep, w.hidden, w.heads, w.length, w.batch,
                                     w.rope_base)
    assert np.abs(got - want).max() <= 1e-5


# ----------------------------------------------------------------- invariants

def test_single_kept_key_copies_its_value(oracle_lib):
    d, heads, L, B = 8, 2, 40, 1
    rng = Lcg(11)
    qkv = (rng.normal(3 * d * L * B)).astype(np.float32)
    keep = np.zeros(L * L, np.uint8)
    for q in range(L):
        keep[q + L * ((3 * q + 1) % L)] = 1
    out = oracle_lib.laya_attention_block(qkv, keep, d, heads, L, B, 160000.0).reshape(L, d)
    x = qkv.reshape(L, 3 * d)
    for q in range(L):
        assert np.array_equal(out[q], x[(3 * q + 1) % L, 2 * d:3 * d])


def test_uniform_scores_average_values(oracle_lib):
    d, heads, L, B = 8, 2, 48, 1
    rng = Lcg(12)
    qkv = rng.normal(3 * d * L).astype(np.float32)
    qkv.reshape(L, 3 * d)[:, :d] = 0.0  # q = 0: every kept key scores 0
    keep = (np.arange(L * L) % 5 != 0).astype(np.uint8)
    out = oracle_lib.laya_attention_block(qkv, keep, d, heads, L, B, 0.0).reshape(L, d)
    x = qkv.reshape(L, 3 * d)
    kp = keep.reshape(L, L)  # [key, query]
    for q in range(L):
        sel = kp[:, q].astype(bool)
        assert np.abs(out[q] - x[sel, 2 * d:].mean(axis=0)).max() <= 1e-6


def test_key_permutation_equivariance_without_rope(oracle_lib):
    d, heads, L = 16, 2, 37
    rng = Lcg(13)
    qkv = rng.normal(3 * d * L).astype(np.float32)
    keep = np.ones(L * L, np.uint8)
    out = oracle_lib.laya_attention_block(qkv, keep, d, heads, L, 1, 0.0).reshape(L, d)
    perm = np.array([(7 * i + 3) % L for i in range(L)])
    x = qkv.reshape(L, 3 * d).copy()
    x2 = x.copy()
    x2[:, d:] = x[perm, d:]  # permute keys and values together
    out2 = oracle_lib.laya_attention_block(x2.reshape(-1), keep, d, heads, L, 1, 0.0).reshape(L, d)
    assert np.abs(out - out2).max() <= 1e-6


# ----------------------------------------------------------------- Jeff

def jeff_inputs(seed, length, heads, hd, kv_heads=None, lo=-1.0, hi=1.0):
    rng = Lcg(seed)
    kv_heads = kv_heads or heads
    W, KW = heads * hd, kv_heads * hd
    q = (lo + (hi - lo) * rng.uniform(length * W)).astype(np.float32)
    k = (lo + (hi - lo) * rng.uniform(length * KW)).astype(np.float32)
    v = (lo + (hi - lo) * rng.uniform(length * KW)).astype(np.float32)
    gate = (lo + (hi - lo) * rng.uniform(length * W)).astype(np.float32)
    qn = (0.5 + rng.uniform(hd)).astype(np.float32)
    kn = (0.5 + rng.uniform(hd)).astype(np.float32)
    return q, k, v, gate, qn, kn


@pytest.mark.parametrize("length", [1, 2, 3, 6])
def test_jeff_oracle_matches_host_small(oracle_lib, length):
    """jeff-infer model.rs:1332-1404 shape: heads 2, hd 4, rotary 2, eps 1e-5."""
    heads, hd, rot, theta, eps = 2, 4, 2, 10000.0, 1e-5
    q, k, v, g, qn, kn = jeff_inputs(1 + length, length, heads, hd)
    mask = np.ones(length, np.float32)
    got = oracle_lib.jeff_full_attention(q, k, v, g, qn, kn, mask, length, heads, hd, rot, theta, eps)
    want = brute.jeff_full_attention_host(q, k, v, g, qn, kn, mask, length, heads, hd, rot, theta, eps)
    assert np.abs(got - want).max() <= 1e-5


def test_jeff_oracle_matches_host_hd256(oracle_lib):
    length, heads, hd, rot, theta, eps = 48, 2, 256, 64, 1e7, 1e-6
    q, k, v, g, qn, kn = jeff_inputs(21, length, heads, hd)
    mask = np.ones(length, np.float32)
    mask[[0, 1, 7, 20]] = 0.0  # leading and interior holes
    got = oracle_lib.jeff_full_attention(q, k, v, g, qn, kn, mask, length, heads, hd, rot, theta, eps)
    want = brute.jeff_full_attention_host(q, k, v, g, qn, kn, mask, length, heads, hd, rot, theta, eps)
    assert np.abs(got - want).max() <= 1e-5


def test_jeff_empty_rows_are_zero(oracle_lib):
    """lib.rs:743-754: a query with no kept key writes 0 (times the gate)."""
    length, heads, hd = 5, 1, 4
    q, k, v, g, qn, kn = jeff_inputs(5, length, heads, hd)
    mask = np.array([0, 0, 1, 1, 1], np.float32)
    out = oracle_lib.jeff_full_attention(q, k, v, g, qn, kn, mask, length, heads, hd, 2, 1e4, 1e-6)
    out = out.reshape(hd, length)
    assert np.all(out[:, :2] == 0.0)
    assert np.all(out[:, 2:] != 0.0)


def test_jeff_gqa_expansion_matches_grouped_host(oracle_lib):
    """checkpoint.rs:307-319: head h reads kv head h // (heads/kv)."""
    length, heads, kvh, hd = 20, 8, 2, 16
    q, k, v, g, qn, kn = jeff_inputs(31, length, heads, hd, kv_heads=kvh)
    mask = np.ones(length, np.float32)
    got = oracle_lib.jeff_rows(q, k, v, g, qn, kn, mask, 1, length, heads, kvh, hd, 8, 1e4, 1e-6)
    K = k.reshape(kvh * hd, length)
    V = v.reshape(kvh * hd, length)
    Ke = np.concatenate([K[(h // 4) * hd:(h // 4 + 1) * hd] for h in range(heads)])
    Ve = np.concatenate([V[(h // 4) * hd:(h // 4 + 1) * hd] for h in range(heads)])
    want = brute.jeff_full_attention_host(q, Ke.reshape(-1), Ve.reshape(-1), g, qn, kn, mask,
                                          length, heads, hd, 8, 1e4, 1e-6)
    assert np.abs(got - want).max() <= 1e-5


def test_jeff_trim_rebases_positions(oracle_lib):
    """engine.rs:317-329: leading inactive keys dropped, positions restart at 0."""
    length, heads, hd, rot = 24, 2, 8, 8
    q, k, v, g, qn, kn = jeff_inputs(41, length, heads, hd)
    mask = np.ones(length, np.float32)
    mask[:5] = 0.0
    mask[11] = 0.0
    got = oracle_lib.jeff_rows(q, k, v, g, qn, kn, mask, 1, length, heads, heads, hd, rot, 1e4,
                               1e-6, trim_leading=True).reshape(heads * hd, length)
    s = 5
    Q, K, V, G = (x.reshape(heads * hd, length)[:, s:].copy() for x in (q, k, v, g))
    want = brute.jeff_full_attention_host(Q, K, V, G, qn, kn, mask[s:], length - s, heads, hd,
                                          rot, 1e4, 1e-6).reshape(heads * hd, length - s)
    assert np.all(got[:, :s] == 0.0)
    assert np.abs(got[:, s:] - want).max() <= 1e-5


# ----------------------------------------------------------------- the checks have teeth

def _brute_variant(kind):
    """Plausible mistakes planted in a copy of the float64 brute force."""
    def run(qkv, keep, d, heads, length, batch, base):
        x = np.asarray(qkv, np.float64).copy()
        kp = np.asarray(keep).copy()
        if kind == "rope_sign":
            return _rope_sign_flip(x, kp, d, heads, length, batch, base)
        if kind == "no_scale":
            return _no_scale(x, kp, d, heads, length, batch, base)
        if kind == "transposed_keep":
            kt = kp.reshape(batch, length, length).transpose(0, 2, 1).reshape(-1)
            return brute.laya_attention_host(x, kt, d, heads, length, batch, base)
        raise ValueError(kind)
    return run


def _rope_sign_flip(x, kp, d, heads, length, batch, base):
    hd = d // heads
    y = x.reshape(batch, length, 3 * d).copy()
    pos = np.arange(length, dtype=np.float64)
    for b in range(batch):
        for h in range(heads):
            for off in (0, d):
                f = slice(off + h * hd, off + (h + 1) * hd)
                y[b, :, f] = brute._rotate(y[b, :, f], -pos, base, hd)
    return brute.laya_attention_host(y.reshape(-1), kp, d, heads, length, batch, 0.0)


def _no_scale(x, kp, d, heads, length, batch, base):
    y = x.reshape(batch, length, 3 * d).copy()
    y[:, :, :d] *= math.sqrt(d // heads)  # as if s = q.k without 1/sqrt(hd)
    return brute.laya_attention_host(y.reshape(-1), kp, d, heads, length, batch, base)


@pytest.mark.parametrize("kind", ["rope_sign", "no_scale", "transposed_keep"])
def test_planted_mistakes_are_caught(oracle_lib, kind):
    d, heads, length, batch = 8, 2, 33, 1
    rng = Lcg(77)
    qkv = rng.normal(3 * d * length).astype(np.float32)
    valid = encoder_valid(length, 1, False)
    keep = oracle_lib.laya_build_mask(valid, length, batch, 1)
    good = oracle_lib.laya_attention_block(qkv, keep, d, heads, length, batch, 10000.0)
    bad = _brute_variant(kind)(qkv, keep, d, heads, length, batch, 10000.0)
    ok = ~np.isnan(good) & ~np.isnan(bad)
    assert np.abs(good[ok] - bad[ok]).max() > 1e-2
