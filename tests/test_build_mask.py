"""Pins of the oracle's build_mask (laya-infer src/model.rs:465-490), the keep
tensor that the structured entry reproduces on the GPU.

keep[q + L*(k + L*b)] = valid_k && (FullAttention || |q - k| <= window || !valid_q)

The reference holds no independent implementation or fixture of this mask
(its encoder test compares two forwards that both call build_mask, and the
Julia `attention_masks` it mirrors is an empty submodule). So the pins are:

* keep tensors written out by hand, entry by entry, for the reference test's
  own `encoder_batch` masks (laya-infer tests/model.rs:160-179: an interior
  key hole in row 0, a padded last query in row 1), global and with
  windows 1 and 2;
* mistakes a restatement could plausibly make (valid_q and valid_k swapped,
  the padded-query exemption dropped, `<` for `<=`, the window applied to
  keys of padded queries), each of which fails those hand-written tables;
* structural facts checked exhaustively on tiny shapes: a padded query keeps
  exactly the valid keys, a valid query keeps the valid keys within the
  window, windows that span the row equal global attention;
* the second copy of the formula the workloads use (`_build_keep`) equals
  the oracle on every tiny shape.
"""
import itertools

import numpy as np
import pytest

import oracle
from tenferro_ext.workloads import _build_keep


def encoder_batch_valid(length, batch):
    """The `mask` of encoder_batch (laya-infer tests/model.rs:160-179), (L, B)."""
    valid = np.zeros(length * batch, np.uint8)
    for b in range(batch):
        for l in range(length):
            if length == 1:
                v = True
            elif batch == 1 or b == 0:
                v = l != 1  # an interior key hole
            else:
                v = l < length - 1  # a padded query position at the end
            valid[l + length * b] = v
    return valid


def as_rows(keep, length, batch):
    """keep (L, L, B) flat -> [b][q] = list of kept keys as 0/1."""
    k = np.asarray(keep).reshape(batch, length, length)  # [b, key, query]
    return [[list(map(int, k[b, :, q])) for q in range(length)] for b in range(batch)]


# Hand-written expectations for encoder_batch(4, 2):
#   row 0 valid = 1 0 1 1 (token 1 is a key hole)
#   row 1 valid = 1 1 1 0 (token 3 is padding)
# Each line is one query; entries are keys 0..3.
EXPECTED = {
    -1: [  # FullAttention: every query keeps exactly the valid keys
        [[1, 0, 1, 1], [1, 0, 1, 1], [1, 0, 1, 1], [1, 0, 1, 1]],
        [[1, 1, 1, 0], [1, 1, 1, 0], [1, 1, 1, 0], [1, 1, 1, 0]],
    ],
    1: [  # SlidingAttention, local_attention 2 -> window 1
        [[1, 0, 0, 0],   # q0: keys 0..1, key 1 invalid
         [1, 0, 1, 1],   # q1 is itself invalid (the hole): every valid key
         [0, 0, 1, 1],   # q2: keys 1..3, key 1 invalid
         [0, 0, 1, 1]],  # q3: keys 2..3
        [[1, 1, 0, 0],   # q0: keys 0..1
         [1, 1, 1, 0],   # q1: keys 0..2
         [0, 1, 1, 0],   # q2: keys 1..3, key 3 invalid
         [1, 1, 1, 0]],  # q3 is padding: every valid key
    ],
    2: [  # window 2
        [[1, 0, 1, 0],
         [1, 0, 1, 1],
         [1, 0, 1, 1],
         [0, 0, 1, 1]],
        [[1, 1, 1, 0],
         [1, 1, 1, 0],
         [1, 1, 1, 0],
         [1, 1, 1, 0]],
    ],
}


def _mask_variant(valid, L, B, window, variant):
    """build_mask with one planted mistake (test-side only)."""
    keep = np.zeros(L * L * B, np.uint8)
    for b, q, k in itertools.product(range(B), range(L), range(L)):
        vq, vk = bool(valid[q + L * b]), bool(valid[k + L * b])
        d = abs(q - k)
        if variant == "swap_valid":
            inside = window < 0 or d <= window or not vk
            val = vq and inside
        elif variant == "no_exemption":
            val = vk and (window < 0 or d <= window)
        elif variant == "strict":
            val = vk and (window < 0 or d < window or not vq)
        elif variant == "exempt_keys":  # padded queries also limited to the window
            val = vk and (window < 0 or d <= window) if not vq else vk and d <= max(window, 0)
        else:
            raise ValueError(variant)
        keep[q + L * (k + L * b)] = val
    return keep


@pytest.mark.parametrize("window", [-1, 1, 2])
def test_oracle_matches_hand_written_tables(oracle_lib, window):
    valid = encoder_batch_valid(4, 2)
    keep = oracle.laya_build_mask(valid, 4, 2, window)
    assert as_rows(keep, 4, 2) == EXPECTED[window]


def test_encoder_batch_shapes_of_the_reference_test(oracle_lib):
    """The four (L, B) cases of encoder_parity (tests/model.rs:181-200)."""
    for L, B in ((1, 1), (1, 2), (4, 1), (4, 2)):
        valid = encoder_batch_valid(L, B)
        for window in (-1, 0, 1, 2, 8):
            keep = np.asarray(oracle.laya_build_mask(valid, L, B, window)).reshape(B, L, L)
            for b, q, k in itertools.product(range(B), range(L), range(L)):
                vq, vk = valid[q + L * b], valid[k + L * b]
                if not vk:
                    assert keep[b, k, q] == 0
                elif not vq or window < 0:
                    assert keep[b, k, q] == 1
                else:
                    assert keep[b, k, q] == (abs(q - k) <= window)


@pytest.mark.parametrize("variant", ["swap_valid", "no_exemption", "strict", "exempt_keys"])
def test_planted_mistakes_fail_the_tables(variant):
    """Each plausible mistake changes at least one hand-written entry."""
    valid = encoder_batch_valid(4, 2)
    failed = 0
    for window in (1, 2):
        got = as_rows(_mask_variant(valid, 4, 2, window, variant), 4, 2)
        failed += got != EXPECTED[window]
    assert failed >= 1


def test_structure_exhaustive_tiny(oracle_lib):
    """Every validity pattern of L <= 5 (B = 1) and random patterns at B = 3,
    every window: padded queries keep exactly the valid keys; valid queries
    keep valid keys within the window; a window of L - 1 or more is global;
    workloads._build_keep agrees with the oracle bit for bit."""
    rng = np.random.default_rng(7)
    cases = []
    for L in range(1, 6):
        for bits in range(1 << L):
            cases.append((L, 1, np.array([(bits >> i) & 1 for i in range(L)], np.uint8)))
    for L in (6, 7, 9):
        for _ in range(20):
            cases.append((L, 3, (rng.random(L * 3) < 0.7).astype(np.uint8)))
    for L, B, valid in cases:
        full = np.asarray(oracle.laya_build_mask(valid, L, B, -1)).reshape(B, L, L)
        for window in range(-1, L + 1):
            keep = np.asarray(oracle.laya_build_mask(valid, L, B, window))
            assert np.array_equal(keep, _build_keep(valid, L, B, window)), (L, B, window)
            k3 = keep.reshape(B, L, L)  # [b, key, query]
            v = valid.reshape(B, L).astype(bool)
            for b in range(B):
                for q in range(L):
                    col = k3[b, :, q].astype(bool)
                    if not v[b, q]:
                        assert np.array_equal(col, v[b])
                    else:
                        dist = np.abs(np.arange(L) - q)
                        want = v[b] & ((dist <= window) if window >= 0 else True)
                        assert np.array_equal(col, want)
            if window >= L - 1:
                assert np.array_equal(k3, full)
