"""CPU pins of the padded-prefill rule for prefix rows -- no GPU.

The prefill pads every row to a multiple of 256 tokens after its ``n_valid`` real tokens and
runs the training forward with ``cls_n = n_valid``: the classification counts only the real
positions, and a prefix row's segment list is the combined label order with the padding
entries removed (prefix_compact_kernel).  The CPU model never pads: it runs the real tokens.
These tests pin that the two agree by definition:
  * the combined order (label, position, key before query) of a padded row, filtered to the
    real positions, is the combined order of the unpadded row -- for pad labels equal to,
    below and above the real labels, and real lengths on and off the 64-entry segment grid;
  * the row modes of the unpadded rows of the inference tests' patterns
    (dism_v3/tests/test_sam_inference.py:32-45 shapes: N = 79, alphabet 4);
  * the CPU model's prefix definition at that unpadded length (segments not a multiple of
    64 entries) against the direct pairwise definition (fp32 association) and the FP64
    dense restatement."""
import numpy as np
import pytest

import oracle
from oracle import dense


def _combined_order(q, k):
    """entries e = 2p + s (s = 0 key, 1 query) sorted by (unsigned label, p, s): brute force"""
    n = len(q)
    lab = np.empty(2 * n, np.uint32)
    lab[0::2] = k.view(np.uint32)
    lab[1::2] = q.view(np.uint32)
    return sorted(range(2 * n), key=lambda e: (int(lab[e]), e))


@pytest.mark.parametrize("cn", [1, 31, 32, 79, 128, 200])
@pytest.mark.parametrize("pad", [0, -5, 7])
def test_compacted_order_is_the_unpadded_order(cn, pad):
    rng = np.random.default_rng(cn * 31 + pad)
    n = 256
    q = rng.integers(0, 5, n).astype(np.int32)
    k = rng.integers(0, 5, n).astype(np.int32)
    q[cn:] = pad
    k[cn:] = pad
    full = _combined_order(q, k)
    compact = [e for e in full if (e >> 1) < cn]
    assert len(compact) == 2 * cn
    assert compact == _combined_order(q[:cn], k[:cn])
    # the segment of each compacted entry (64 per segment) is its rank // 64 in that order
    segs = [x // 64 for x in range(len(compact))]
    assert max(segs) + 1 == (2 * cn + 63) // 64


def _sam(pattern, n=79, seed=83):
    rng = np.random.default_rng(seed)
    iq = rng.integers(0, 4, (2, 2, n)).astype(np.int32)
    ik = rng.integers(0, 4, (2, 2, n)).astype(np.int32)
    if pattern == "repeat":
        iq[:] = 0
        ik[:] = 0
    elif pattern == "mismatch":
        iq[:] = 0
        ik[:] = 1
    sq, sk, v = (oracle.bf16_round(rng.standard_normal((2, n, 2, c)) * 0.2)
                 for c in (16, 16, 32))
    return iq, ik, sq, sk, v


def test_inference_patterns_row_modes():
    iq, ik, *_ = _sam("repeat")
    assert (oracle.row_modes(iq, ik, 16, 32) == 4).all()
    # padded with label 0 the all-zero rows stay prefix rows over the padded length too
    pad = np.zeros((2, 2, 256), np.int32)
    assert (oracle.row_modes(pad, pad, 16, 32) == 4).all()
    iq, ik, *_ = _sam("mismatch")
    assert (oracle.row_modes(iq, ik, 16, 32) == 0).all()


def test_unpadded_prefix_rows_match_direct_and_fp64():
    iq, ik, sq, sk, v = _sam("repeat")
    tau = np.array([0.0, 0.35], np.float32)
    hard = np.ones((2, 2), bool)
    lut = oracle.log_weights(tau, 79)
    o4, l4, m4, a4 = oracle.forward(sq, sk, v, iq, ik, hard, lut, dense=4)
    o1, l1, m1, a1 = oracle.forward(sq, sk, v, iq, ik, hard, lut, dense=1)
    o0, l0, _, _ = oracle.forward(sq, sk, v, iq, ik, hard, lut)
    assert np.array_equal(o0.view(np.uint32), o4.view(np.uint32))  # chosen mode: prefix
    assert np.array_equal(m4, m1) and np.array_equal(a4, a1)
    np.testing.assert_allclose(o4, o1, atol=1e-6, rtol=1e-5)
    np.testing.assert_allclose(l4, l1, atol=1e-5, rtol=1e-6)
    ref, lref = dense.dense_forward(sq, sk, v, iq, ik, hard, tau)
    np.testing.assert_allclose(o4, ref, atol=2e-6, rtol=2e-4)
    np.testing.assert_allclose(l4, lref, atol=1e-4, rtol=1e-5)
