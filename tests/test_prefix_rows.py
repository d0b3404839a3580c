"""CPU pins of the prefix-row definition and classification (oracle/dism_cpu_model.c:
prefix_labels, prefix_forward_row, prefix_backward_row) -- no GPU.

A dense row in which every label has one predecessor label has L[i,j] = j + 1 on every valid
pair, so its sums over valid keys are prefix sums with per-key weights (and a running
maximum).  These tests pin:
  * the classification against a brute-force predecessor check and the match lengths of the
    textbook recurrence (dism_v3/tests/test_hard_chunk.py:24-36) -- L = j + 1 on every valid
    pair exactly when the rule holds, on patterns that pass and fail it;
  * the prefix definition (oracle row mode 4) against the direct pairwise definition
    (dense=1, the reference's quadratic loop) to fp32 association, lmax / argmax exactly, and
    against the FP64 dense restatement (oracle/dense.py);
  * long rows, where LUT[j + 1] spans more than the fp32 range of exp2 (the running maximum
    and the chains' rescaling), and tau of both signs."""
import numpy as np
import pytest

import oracle
from oracle import dense
from tests._data import labels, vectors
from tests.test_oracle import _brute_L


def _brute_prefix(q, k):
    """every label's predecessors over both sides, by brute force"""
    pred = {}
    for L in (q, k):
        for p in range(1, len(L)):
            pred.setdefault(int(L[p]), set()).add(int(L[p - 1]))
    return all(len(s) == 1 for s in pred.values())


def _shifted(n, period, shift, seed=0):
    base = np.random.default_rng(seed).permutation(1000)[:period].astype(np.int32) - 500
    return base[np.arange(n) % period], base[(np.arange(n) + shift) % period]


CASES = {
    "equal": lambda n: labels(n, "equal", b=1, h=1)[0][0, 0].copy(),
}


@pytest.mark.parametrize("case", ["equal", "periodic", "shift7", "shift64", "alphabet4",
                                  "boundary", "twopred", "random"])
def test_classification_and_lengths(case):
    n = 300
    if case in ("equal", "periodic", "alphabet4", "boundary", "random"):
        q, k = labels(n, case, b=1, h=1)
        q, k = q[0, 0], k[0, 0]
    elif case == "shift7":
        q, k = _shifted(n, 7, 3)
    elif case == "shift64":
        q, k = _shifted(n, 64, 10)
    else:  # one label with two predecessors
        q = np.full(n, 4, np.int32)
        q[::50] = 9
        k = q.copy()
    brute = _brute_prefix(q, k)
    dense_row = oracle.dense_rows(q[None, None], k[None, None], np.ones((1, 1), bool))[0, 0]
    assert oracle.prefix_row(q, k) == int(brute and dense_row)
    if brute:
        # the rule makes every valid pair's match reach the key's row start
        L = _brute_L(q, k)
        i, j = np.nonzero(L)
        assert (L[i, j] == j + 1).all()
    want = {"equal": 1, "periodic": 1, "shift7": 1, "shift64": 1, "alphabet4": 0,
            "boundary": 0, "twopred": 0, "random": 0}[case]
    assert oracle.prefix_row(q, k) == want


def _pair_check(q, k, r, dv, tau, seed=0, fp64=True):
    n = q.shape[-1]
    b, h = q.shape[:2]
    sq, sk, v = vectors(n, b=b, h=h, r=r, dv=dv, seed=seed)
    hard = np.ones((b, h), bool)
    lut = oracle.log_weights(tau, n)
    dl = oracle.dlog_weights(tau, n)
    assert (oracle.row_modes(q, k, r, dv) == 4).all()
    o4 = oracle.forward(sq, sk, v, q, k, hard, lut)
    o1 = oracle.forward(sq, sk, v, q, k, hard, lut, dense=1)
    np.testing.assert_allclose(o4[0], o1[0], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(o4[1], o1[1], rtol=5e-6, atol=1e-6)
    np.testing.assert_array_equal(o4[2], o1[2])
    np.testing.assert_array_equal(o4[3], o1[3])
    do = oracle.bf16_round(np.random.default_rng(seed + 1).standard_normal(v.shape))
    g4 = oracle.backward(sq, sk, v, do, q, k, hard, lut, dl, o1[1])
    g1 = oracle.backward(sq, sk, v, do, q, k, hard, lut, dl, o1[1], dense=1)
    for a, c in zip(g4[:3], g1[:3]):
        assert np.abs(a - c).max() <= 1e-5 * max(np.abs(c).max(), 1e-30)
    np.testing.assert_allclose(g4[3], g1[3], rtol=1e-4, atol=1e-5)
    if fp64:
        od, _ = dense.dense_forward(sq, sk, v, q, k, hard, tau)
        np.testing.assert_allclose(o4[0], od, rtol=1e-4, atol=1e-5)
        gd = dense.dense_backward(sq, sk, v, do, q, k, hard, tau)
        for a, c in zip(g4[:3], gd[:3]):
            assert np.abs(a - c).max() <= 1e-3 * max(np.abs(c).max(), 1e-30)
        np.testing.assert_allclose(g4[3], gd[3], rtol=1e-3, atol=1e-4)


@pytest.mark.parametrize("r,dv", [(2, 32), (8, 64), (32, 128)])
def test_identical_against_direct_and_fp64(r, dv):
    q, k = labels(260, "equal", b=1, h=3)
    _pair_check(q, k, r, dv, np.array([-0.5, 0.0, 0.7], np.float32), seed=r)


@pytest.mark.parametrize("period,shift", [(7, 0), (7, 3), (40, 10), (40, 39)])
def test_shifted_periods_against_direct_and_fp64(period, shift):
    q, k = _shifted(333, period, shift, seed=period)
    _pair_check(q[None, None], k[None, None], 4, 32, np.array([0.4], np.float32), seed=shift)


def test_long_row_rescaling():
    """N = 1500 at tau = 1: LUT[N] is about 2160 (log2), far past exp2's fp32 range, so the
    segment totals, chains and queries all rescale; and tau < 0, where LUT saturates."""
    q, k = labels(1500, "equal", b=1, h=2)
    _pair_check(q, k, 8, 32, np.array([1.0, -0.7], np.float32), seed=5, fp64=False)


def test_random_predecessor_functions_against_direct():
    """Rows generated from random predecessor functions (each label's successor chosen at
    random, some labels only on one side): whenever the rule holds the row is a prefix row,
    and its prefix definition matches the direct one; rows that break the rule are not."""
    rng = np.random.default_rng(77)
    for trial in range(12):
        n = int(rng.integers(70, 260))
        alpha = int(rng.integers(1, 9))
        succ = rng.integers(0, alpha, alpha)        # label -> next label
        q = np.empty(n, np.int32)
        q[0] = rng.integers(0, alpha)
        for p in range(1, n):
            q[p] = succ[q[p - 1]]
        shift = int(rng.integers(0, 3))
        k = np.concatenate([q[shift:], q[:shift]])  # the same chain, started later
        for p in range(n - shift, n):
            k[p] = succ[k[p - 1]] if p > 0 else k[p]
        if trial % 4 == 3:                          # break the rule once
            k[n // 2] = (k[n // 2] + 1) % max(alpha, 2)
        qq, kk = q[None, None], k[None, None]
        is_prefix = oracle.prefix_row(q, k)
        assert is_prefix == int(_brute_prefix(q, k) and oracle.dense_rows(
            qq, kk, np.ones((1, 1), bool))[0, 0])
        if not is_prefix:
            continue
        L = _brute_L(q, k)
        i, j = np.nonzero(L)
        assert (L[i, j] == j + 1).all()
        _pair_check(qq, kk, 4, 32, np.array([0.3], np.float32), seed=trial, fp64=False)
