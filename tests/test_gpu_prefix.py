"""Prefix rows on the MI355X (dism_amd/csrc/dism_prefix.hip): dense rows in which every label
has one predecessor label, so every valid pair's match runs to the key's row start
(L[i,j] = j + 1) and the sums over valid keys are prefix sums over label groups.  Every test
compares the HIP path bit for bit with the CPU model (oracle.forward / oracle.backward route
these rows to the prefix definition, oracle.row_modes 4) and checks the row modes.

The reference times identical labels at B16 H6 N2048 R32 DV64
(dism_v3/docs/HARD_FORWARD_PLAN.md:245-246); the cases below hold that row shape, the
headline length T = 16384, periods of distinct labels (queries and keys shifted against each
other), every (R, DV) and both dtypes, and rows of every mode in one call.
"""
import numpy as np
import pytest
import torch

import oracle
from oracle import dense
from tests._data import labels, taus, vectors
from tests.test_gpu_dense import _check, _inputs
from tests.test_gpu_parity import dev, host, max_rel

pytestmark = pytest.mark.gpu


def _modes(x):
    import dism_amd
    from dism_amd.hard_forward import row_modes
    sq, sk, v, q, k, hard, tau = x
    t = [dev(a, torch.bfloat16) for a in (sq, sk, v)]
    _, _, state = dism_amd.forward_hard(t[0], t[1], t[2], dev(q), dev(k), dev(hard), dev(tau),
                                        save_state=True)
    m = host(row_modes(state["workspace"], t[0], t[2]))
    return np.where(m == 2, 0, m)  # mode 2: sparse with strip-bounded walks, the same bits


def _shifted(n, b, h, period, shifts, seed=0):
    rng = np.random.default_rng(seed)
    base = rng.permutation(1000)[:period].astype(np.int32) - 500
    q = np.empty((b, h, n), np.int32)
    k = np.empty((b, h, n), np.int32)
    for x in range(h):
        q[:, x] = base[np.arange(n) % period]
        k[:, x] = base[(np.arange(n) + shifts[x % len(shifts)]) % period]
    return q, k


def test_identical_reference_shape_modes_and_fp64():
    """Identical labels, N2048 R32 DV64: mode 4, bit for bit, and close to FP64."""
    x, do = _inputs(2048, "equal", b=1, h=3, r=32, dv=64, seed=11)
    assert (oracle.row_modes(x[3], x[4], 32, 64) == 4).all()
    print("prefix identical N=2048 R=32 DV=64", flush=True)
    assert (_modes(x) == 4).all()
    o, g = _check(x, do, threads=3, what="prefix identical 2048")
    sq, sk, v, q, k, hard, tau = x
    od, _ = dense.dense_forward(sq[:, :512], sk[:, :512], v[:, :512], q[..., :512],
                                k[..., :512], hard, tau)
    np.testing.assert_allclose(o[:, :512], od, rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("period,shifts", [(7, [0, 1, 3]), (64, [0, 5]), (200, [1])])
def test_periods_of_distinct_labels(period, shifts):
    """Periods of distinct labels with queries and keys shifted against each other: the label
    groups hold keys and queries at different positions, groups end inside segments."""
    n = 1536
    q, k = _shifted(n, 2, 3, period, shifts, seed=period)
    sq, sk, v = vectors(n, b=2, h=3, r=8, dv=64, seed=7)
    hard = np.ones((2, 3), bool)
    do = oracle.bf16_round(np.random.default_rng(3).standard_normal(v.shape))
    x = (sq, sk, v, q, k, hard, np.array([0.9, -0.4, 0.05], np.float32))
    want = oracle.row_modes(q, k, 8, 64)
    print(f"prefix periods period={period} shifts={shifts} modes={want.tolist()}", flush=True)
    assert (_modes(x) == want).all()
    _check(x, do, threads=6, what=f"prefix period {period}")


@pytest.mark.parametrize("r,dv,dtype", [(2, 32, torch.bfloat16), (4, 128, torch.float32),
                                        (8, 64, torch.bfloat16), (16, 128, torch.bfloat16),
                                        (32, 128, torch.float32), (32, 32, torch.bfloat16)])
def test_prefix_dims_and_dtypes(r, dv, dtype):
    x, do = _inputs(768, "equal", b=1, h=2, r=r, dv=dv, seed=r + dv)
    print(f"prefix dims r={r} dv={dv} dtype={dtype}", flush=True)
    _check(x, do, dtype=dtype, what=f"prefix r{r} dv{dv}")


def test_identical_headline_length():
    """Identical labels at T = 16384: 512 segments per row, the chains run through them all."""
    x, do = _inputs(16384, "equal", b=1, h=2, r=8, dv=64, seed=12)
    print("prefix identical N=16384 R=8 DV=64", flush=True)
    o, g = _check(x, do, threads=2, what="prefix identical 16384")
    assert np.isfinite(o).all() and all(np.isfinite(t).all() for t in g[:3])


def test_rows_of_every_mode_in_one_call():
    """Prefix, level, direct, sparse and soft rows side by side."""
    n, b, h = 1024, 2, 5
    rng = np.random.default_rng(21)
    q = rng.integers(0, 256, (b, h, n)).astype(np.int32)
    k = rng.integers(0, 256, (b, h, n)).astype(np.int32)
    q[:, 1] = 5
    k[:, 1] = 5                                     # prefix (identical)
    q[:, 2] = rng.integers(0, 4, (b, n))
    k[:, 2] = rng.integers(0, 4, (b, n))            # level (alphabet 4)
    q[:, 3] = 1
    k[:, 3] = 1
    q[:, 3, ::97] = 2                               # dense, two predecessors of label 1
    k[:, 3, ::89] = 2
    qq, kk = _shifted(n, b, 1, 11, [4], seed=2)
    q[:, 4], k[:, 4] = qq[:, 0], kk[:, 0]           # prefix (period 11, shifted)
    sq, sk, v = vectors(n, b=b, h=h, r=4, dv=64, seed=8)
    hard = np.ones((b, h), bool)
    hard[1, 1] = False                              # a soft prefix row
    do = oracle.bf16_round(rng.standard_normal(v.shape))
    x = (sq, sk, v, q, k, hard, np.linspace(-0.6, 0.8, h).astype(np.float32))
    want = oracle.row_modes(q, k, 4, 64)
    assert want[0].tolist() == [0, 4, 3, 1, 4], want
    print("prefix mixed modes", flush=True)
    assert (_modes(x) == want).all()
    _check(x, do, threads=4, what="prefix mixed")


def test_bucket_sharing_labels_stay_direct():
    """Two labels in one classification bucket: the check keeps one slot per bucket, so such a
    row stays a direct dense row (mode 1) even when its predecessors are unique."""
    n = 512
    from oracle import lib
    import ctypes
    # find two labels with the same top-12-bit hash
    seen, pair = {}, None
    for x in range(1, 200000):
        bkt = ((x * 0x9E3779B1) & 0xFFFFFFFF) >> 20
        if bkt in seen:
            pair = (seen[bkt], x)
            break
        seen[bkt] = x
    a0, a1 = pair
    q = np.where(np.arange(n) % 2 == 0, a0, a1).astype(np.int32)[None, None]
    k = q.copy()
    sq, sk, v = vectors(n, b=1, h=1, r=8, dv=32, seed=1)
    x = (sq, sk, v, q, k, np.ones((1, 1), bool), np.array([0.3], np.float32))
    assert oracle.row_modes(q, k, 8, 32)[0, 0] == 1
    assert (_modes(x) == 1).all()
    do = oracle.bf16_round(np.random.default_rng(4).standard_normal(v.shape))
    _check(x, do, what="bucket pair")
