"""CPU pins of the dense-row definition and classification (oracle/dism_cpu_model.c:
orc_dense_row, orc_label_collisions, the direct per-row forward/backward) -- no GPU.

A hard row whose labels collide often (W = sum over labels of #queries x #keys > N^2/64)
is computed by the HIP path with the direct (pairwise) definition, its match lengths from the
diagonal recurrence L[i,j] = L[i-1,j-1] + 1 (dism_v3/tests/test_hard_chunk.py:24-36).  These
tests pin that definition against brute force, FP64 and the decomposed definition, and the
classification rule against a numpy count."""
import numpy as np
import pytest

import oracle
from oracle import dense
from tests import _data
from tests.test_oracle import _brute_L


def _np_collisions(q, k):
    """exact W: sum over labels of #queries x #keys"""
    vals = np.union1d(q, k)
    cq = np.array([(q == x).sum() for x in vals], np.int64)
    ck = np.array([(k == x).sum() for x in vals], np.int64)
    return int((cq * ck).sum())


def _np_buckets(q, k):
    """bucketed M with the bucket map written out in numpy (uint64 product, top 12 bits)"""
    bq = ((q.astype(np.uint32).astype(np.uint64) * 0x9E3779B1) & 0xFFFFFFFF) >> 20
    bk = ((k.astype(np.uint32).astype(np.uint64) * 0x9E3779B1) & 0xFFFFFFFF) >> 20
    cq = np.bincount(bq.astype(np.int64), minlength=4096)
    ck = np.bincount(bk.astype(np.int64), minlength=4096)
    return int((cq * ck).sum())


@pytest.mark.parametrize("pattern", ["random", "equal", "disjoint", "periodic", "boundary",
                                     "alphabet256", "alphabet4", "collide"])
def test_bucket_collisions_count(pattern):
    q, k = _data.labels(700, pattern, b=1, h=1)
    m = oracle.bucket_collisions(q[0, 0], k[0, 0])
    assert m == _np_buckets(q[0, 0], k[0, 0])
    w = _np_collisions(q[0, 0], k[0, 0])
    assert w <= m <= w + 700 * 700 // 64  # equal labels share a bucket; sharing is rare


def test_classification_rule():
    n = 1024
    rows = {p: _data.labels(n, p, b=1, h=1) for p in
            ("equal", "alphabet4", "periodic", "alphabet256", "disjoint", "collide")}
    got = {p: int(oracle.dense_rows(q, k, np.ones((1, 1), bool))[0, 0])
           for p, (q, k) in rows.items()}
    assert got == {"equal": 1, "alphabet4": 1, "periodic": 1, "alphabet256": 0,
                   "disjoint": 0, "collide": 1}
    q, k = rows["equal"]
    assert oracle.dense_rows(q, k, np.zeros((1, 1), bool))[0, 0] == 0  # soft rows never
    # the threshold is strict: W * 64 > N^2
    n = 64
    q = np.arange(n, dtype=np.int32).reshape(1, 1, n)
    k = q.copy()                                   # W = 64 = N^2 / 64: not dense
    assert oracle.dense_rows(q, k, np.ones((1, 1), bool))[0, 0] == 0
    q[0, 0, 0] = 1
    k[0, 0, 0] = 1                                 # label 1 twice on each side: W = 66
    assert oracle.dense_rows(q, k, np.ones((1, 1), bool))[0, 0] == 1
    # rows longer than 65536 stay on the decomposed path
    big = np.zeros((1, 1, 65537), np.int32)
    assert oracle.dense_rows(big, big, np.ones((1, 1), bool))[0, 0] == 0
    big = np.zeros((1, 1, 65536), np.int32)
    assert oracle.dense_rows(big, big, np.ones((1, 1), bool))[0, 0] == 1


def _inputs(n, pattern, b=2, h=3, r=8, dv=64, seed=11):
    q, k = _data.labels(n, pattern, b=b, h=h)
    sq, sk, v = _data.vectors(n, b=b, h=h, r=r, dv=dv, seed=seed)
    return sq, sk, v, q, k, _data.flags(b, h), _data.taus(h)


@pytest.mark.parametrize("pattern", ["random", "alphabet256", "equal", "periodic"])
def test_forced_dense_is_the_direct_definition(pattern):
    """dense=1 on every row is the pairwise definition bit for bit; dense=0 is the decomposed
    one; the two agree to fp32 association (and to FP64)."""
    sq, sk, v, q, k, hard, tau = _inputs(150, pattern)
    lut = oracle.log_weights(tau, 150)
    d1 = oracle.forward(sq, sk, v, q, k, hard, lut, dense=1)
    dd = oracle.forward(sq, sk, v, q, k, hard, lut, direct=True)
    for a, b in zip(d1, dd):
        assert np.array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32))
    d0 = oracle.forward(sq, sk, v, q, k, hard, lut, dense=0)
    np.testing.assert_allclose(d0[0], d1[0], rtol=1e-5, atol=1e-6)
    np.testing.assert_array_equal(d0[2], d1[2])
    np.testing.assert_array_equal(d0[3], d1[3])
    ref, rl2 = dense.dense_forward(sq, sk, v, q, k, hard, tau)
    np.testing.assert_allclose(d1[0], ref, rtol=1e-4, atol=2e-6)
    np.testing.assert_allclose(d1[1], rl2, rtol=1e-5, atol=1e-5)
    rng = np.random.default_rng(3)
    do = oracle.bf16_round(rng.standard_normal(v.shape).astype(np.float32))
    dl = oracle.dlog_weights(tau, 150)
    l2 = d1[1]
    g1 = oracle.backward(sq, sk, v, do, q, k, hard, lut, dl, l2, dense=1)
    gd = oracle.backward(sq, sk, v, do, q, k, hard, lut, dl, l2, direct=True)
    for a, b in zip(g1, gd):
        assert np.array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32))
    g0 = oracle.backward(sq, sk, v, do, q, k, hard, lut, dl, l2, dense=0)
    for a, b in zip(g0[:3], g1[:3]):
        assert np.abs(a - b).max() <= 1e-5 * max(np.abs(b).max(), 1e-30)


def test_auto_classification_routes_rows():
    """Without an override each row takes the definition its classification names."""
    b, h, n = 1, 2, 256
    q = np.empty((b, h, n), np.int32)
    k = np.empty((b, h, n), np.int32)
    rng = np.random.default_rng(4)
    q[0, 0] = rng.integers(0, 256, n)
    k[0, 0] = rng.integers(0, 256, n)
    q[0, 1] = 5
    k[0, 1] = 5
    sq, sk, v = _data.vectors(n, b=b, h=h, r=4, dv=32, seed=2)
    hard = np.ones((b, h), bool)
    lut = oracle.log_weights(_data.taus(h), n)
    flags = oracle.dense_rows(q, k, hard)
    assert flags.tolist() == [[0, 1]]
    modes = oracle.row_modes(q, k, 4, 32)
    assert modes.tolist() == [[0, 4]]  # the identical row is a prefix row
    auto = oracle.forward(sq, sk, v, q, k, hard, lut)[0]
    forced = oracle.forward(sq, sk, v, q, k, hard, lut, dense=modes)[0]
    assert np.array_equal(auto.view(np.uint32), forced.view(np.uint32))
    dec = oracle.forward(sq, sk, v, q, k, hard, lut, dense=0)[0]
    dirc = oracle.forward(sq, sk, v, q, k, hard, lut, direct=True)[0]
    assert np.array_equal(auto[:, :, 0].view(np.uint32), dec[:, :, 0].view(np.uint32))
    np.testing.assert_allclose(auto[:, :, 1], dirc[:, :, 1], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("alphabet", [1, 2, 3])
def test_dense_lengths_brute_force(alphabet):
    """Longest match and its key on dense rows (diagonal recurrence) against brute force."""
    rng = np.random.default_rng(alphabet)
    n = 120
    q = rng.integers(0, alphabet, (1, 1, n)).astype(np.int32)
    k = rng.integers(0, alphabet, (1, 1, n)).astype(np.int32)
    sq, sk, v = _data.vectors(n, b=1, h=1, r=4, dv=32, seed=5)
    lut = oracle.log_weights(np.array([0.2], np.float32), n)
    _, _, lmax, jarg = oracle.forward(sq, sk, v, q, k, np.ones((1, 1), bool), lut, dense=1)
    L = _brute_L(q[0, 0], k[0, 0])
    for i in range(n):
        best = L[i, :i + 1].max()
        assert lmax[0, 0, i] == best
        assert jarg[0, 0, i] == (-1 if best == 0 else int(np.nonzero(L[i, :i + 1] == best)[0].max()))


def test_dense_rows_with_resets_pinned_by_fp64():
    """The direct definition with query resets (prefill) against the FP64 reset recurrence."""
    rng = np.random.default_rng(85)
    b, h, n, r, dv = 1, 2, 97, 8, 32
    for alphabet in (1, 3):
        iq = rng.integers(0, alphabet, (b, h, n)).astype(np.int32)
        ik = rng.integers(0, alphabet, (b, h, n)).astype(np.int32)
        sq, sk, v = (oracle.bf16_round(rng.standard_normal((b, n, h, c)) * 0.3)
                     for c in (r, r, dv))
        tau = np.array([0.0, 0.4], np.float32)
        hard = np.ones((b, h), bool)
        lut = oracle.log_weights(tau, n)
        reset = np.zeros((b, h, n), bool)
        reset[..., 11::23] = True
        got, l2, lmax, _ = oracle.forward(sq, sk, v, iq, ik, hard, lut, reset=reset, dense=1)
        ref, l2d = dense.dense_forward(sq, sk, v, iq, ik, hard, tau, reset=reset)
        np.testing.assert_allclose(got, ref, atol=2e-6, rtol=2e-4)
        np.testing.assert_allclose(l2, l2d, atol=2e-5, rtol=2e-6)
        dec = oracle.forward(sq, sk, v, iq, ik, hard, lut, reset=reset, dense=0)
        np.testing.assert_allclose(got, dec[0], rtol=1e-5, atol=1e-6)
        np.testing.assert_array_equal(lmax, dec[2])
