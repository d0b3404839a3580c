"""CPU pins of the level-row definition (oracle/dism_cpu_model.c: levels_build,
level_forward_row, level_backward_row; row mode 3) -- no GPU.

A dense row over a small alphabet (d_qk = 2: four labels) has about log4 N distinct match
lengths but N/4 valid keys per query, so its sums are taken per match length: with
c_l = p(l) - p(l - 1), sum_j p(L_ij) x_j = sum_l c_l * (sum of x_j over the keys with
L_ij >= l).  These tests pin:
  * the level count (the lists stop at the first level without a kept group) against the
    longest match of the textbook recurrence (dism_v3/tests/test_hard_chunk.py:24-36);
  * the level definition against the direct pairwise one (dense=1, the reference's quadratic
    loop) to fp32 association, lmax / argmax exactly, and against the FP64 dense restatement
    (oracle/dense.py), forward and backward, tau of both signs;
  * the eligibility limits (labels < 256, R * DV <= 512, at most 32 levels)."""
import numpy as np
import pytest

import oracle
from oracle import dense
from tests._data import vectors
from tests.test_oracle import _brute_L


def _alpha(n, a, b=1, h=2, seed=0):
    rng = np.random.default_rng(seed)
    return (rng.integers(0, a, (b, h, n)).astype(np.int32),
            rng.integers(0, a, (b, h, n)).astype(np.int32))


@pytest.mark.parametrize("a,n", [(4, 200), (3, 150), (2, 120)])
def test_level_count_is_the_longest_match(a, n):
    q, k = _alpha(n, a, seed=a)
    for h in range(2):
        L = _brute_L(q[0, h], k[0, h])
        cnt = oracle.level_count(q[0, h], k[0, h], 8, 64)
        longest = int(L.max())
        assert cnt == (longest if longest <= 32 else 0)


@pytest.mark.parametrize("r,dv,tau", [(2, 64, (0.5, -0.3)), (8, 64, (1.0, 0.0)),
                                      (4, 128, (-1.0, 0.2)), (16, 32, (0.7, -0.7))])
def test_level_rows_against_direct_and_fp64(r, dv, tau):
    n = 256
    q, k = _alpha(n, 4, seed=r + dv)
    assert (oracle.row_modes(q, k, r, dv) == 3).all()
    sq, sk, v = vectors(n, b=1, h=2, r=r, dv=dv, seed=r)
    hard = np.ones((1, 2), bool)
    tau = np.array(tau, np.float32)
    lut = oracle.log_weights(tau, n)
    dl = oracle.dlog_weights(tau, n)
    o3 = oracle.forward(sq, sk, v, q, k, hard, lut)
    o1 = oracle.forward(sq, sk, v, q, k, hard, lut, dense=1)
    np.testing.assert_allclose(o3[0], o1[0], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(o3[1], o1[1], rtol=5e-6, atol=1e-6)
    np.testing.assert_array_equal(o3[2], o1[2])
    np.testing.assert_array_equal(o3[3], o1[3])
    od, _ = dense.dense_forward(sq, sk, v, q, k, hard, tau)
    np.testing.assert_allclose(o3[0], od, rtol=1e-4, atol=1e-5)
    do = oracle.bf16_round(np.random.default_rng(r).standard_normal(v.shape))
    g3 = oracle.backward(sq, sk, v, do, q, k, hard, lut, dl, o1[1])
    g1 = oracle.backward(sq, sk, v, do, q, k, hard, lut, dl, o1[1], dense=1)
    for x, y in zip(g3[:3], g1[:3]):
        assert np.abs(x - y).max() <= 1e-5 * max(np.abs(y).max(), 1e-30)
    # row tau terms cancel internally (w - u * mean): compared on the scale of the row terms
    assert np.abs(g3[4] - g1[4]).max() <= 1e-3 * np.abs(g1[4]).max()
    gd = dense.dense_backward(sq, sk, v, do, q, k, hard, tau)
    for x, y in zip(g3[:3], gd[:3]):
        assert np.abs(x - y).max() <= 1e-3 * max(np.abs(y).max(), 1e-30)
    np.testing.assert_allclose(g3[3], gd[3], rtol=1e-3, atol=1e-4)


def test_level_eligibility_limits():
    q, k = _alpha(256, 4, seed=9)
    assert (oracle.row_modes(q, k, 8, 64) == 3).all()          # R * DV = 512
    assert (oracle.row_modes(q, k, 16, 64) == 1).all()         # R * DV = 1024: direct
    q2, k2 = q + 300, k + 300                                   # labels >= 256: direct
    assert (oracle.row_modes(q2, k2, 8, 64) == 1).all()
    qq = q.copy()
    kk = k.copy()
    qq[0, 0, 100:160] = 2                                       # a 60-long run: > 32 levels
    kk[0, 0, 20:80] = 2
    m = oracle.row_modes(qq, kk, 8, 64)
    assert m[0, 0] == 1 and m[0, 1] == 3
