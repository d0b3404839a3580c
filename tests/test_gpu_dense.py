"""Dense rows on the MI355X (dism_amd/csrc/dism_dense.hip): rows whose labels collide often
(identical labels, tiny alphabets, short periods) are computed with the direct definition
over query-key tiles, their match lengths from the diagonal recurrence.  Every test compares
the HIP path bit for bit with the CPU model (oracle.forward / oracle.backward, which route each
row by the same classification, oracle.dense_rows) and checks the classification it expects.

The reference times identical labels against random ones at B16 H6 N2048 R32 DV64
(dism_v3/docs/HARD_FORWARD_PLAN.md:245-246); the identical-label cases below are that shape
and the headline length T = 16384.
"""
import numpy as np
import pytest
import torch

import oracle
from oracle import dense
from tests._data import labels, taus, vectors
from tests.test_gpu_parity import assert_bits, dev, host, max_rel

pytestmark = pytest.mark.gpu


def _fwd_bwd(sq, sk, v, do, q, k, hard, tau, dtype=torch.bfloat16):
    import dism_amd
    t = [dev(a, dtype) for a in (sq, sk, v, do)]
    out, lse2, state, m = dism_amd.forward_hard(t[0], t[1], t[2], dev(q), dev(k), dev(hard),
                                                dev(tau), save_state=True, return_matches=True,
                                                out_dtype=torch.float32)
    grads = dism_amd.backward_hard(t[0], t[1], t[2], t[3], dev(q), dev(k), dev(hard), lse2,
                                   state)
    return out, lse2, m, grads


def _check(x, do, threads=0, dtype=torch.bfloat16, what=""):
    sq, sk, v, q, k, hard, tau = x
    n = q.shape[-1]
    out, lse2, m, grads = _fwd_bwd(sq, sk, v, do, q, k, hard, tau, dtype)
    lut = oracle.log_weights(tau, n)
    dl = oracle.dlog_weights(tau, n)
    o, l2, lm, ja = oracle.forward(sq, sk, v, q, k, hard, lut, threads=threads)
    assert_bits(host(out), o, f"{what} out")
    assert_bits(host(lse2), l2, f"{what} lse2")
    assert_bits(host(m["length"]), lm, f"{what} lmax")
    assert_bits(host(m["index"]), ja, f"{what} argmax")
    g = oracle.backward(sq, sk, v, do, q, k, hard, lut, dl, l2, threads=threads)
    for got, want, name in zip(grads, g[:4], ("dsq", "dsk", "dv", "dtau")):
        assert_bits(host(got), want, f"{what} {name}")
    return o, g


def _inputs(n, pattern, b=2, h=3, r=8, dv=64, seed=0):
    q, k = labels(n, pattern, b=b, h=h, seed=20261014 + seed)
    sq, sk, v = vectors(n, b=b, h=h, r=r, dv=dv, seed=417 + seed)
    hard = np.ones((b, h), bool)
    do = oracle.bf16_round(np.random.default_rng(31 + seed).standard_normal(v.shape))
    return (sq, sk, v, q, k, hard, taus(h)), do


@pytest.mark.parametrize("pattern", ["equal", "alphabet4", "periodic", "boundary", "collide"])
@pytest.mark.parametrize("n", [256, 1280])
def test_dense_patterns_fwd_bwd(pattern, n):
    """Dense label patterns, bit for bit, and within the FP64 dense restatement's
    tolerances."""
    x, do = _inputs(n, pattern)
    flags = oracle.dense_rows(x[3], x[4], x[5])
    assert flags.all(), flags
    print(f"dense pattern={pattern} n={n}", flush=True)
    o, g = _check(x, do, what=pattern)
    if n <= 512:
        sq, sk, v, q, k, hard, tau = x
        od, _ = dense.dense_forward(sq, sk, v, q, k, hard, tau)
        np.testing.assert_allclose(o, od, rtol=1e-4, atol=2e-6)
        gd = dense.dense_backward(sq, sk, v, do, q, k, hard, tau)
        for got, want in zip(g[:3], gd[:3]):
            assert max_rel(got, want) < 1e-3


@pytest.mark.parametrize("r,dv,dtype", [(2, 64, torch.bfloat16), (4, 32, torch.float32),
                                        (16, 128, torch.bfloat16), (32, 64, torch.float32),
                                        (32, 128, torch.bfloat16), (8, 32, torch.bfloat16)])
def test_dense_dims_and_dtypes(r, dv, dtype):
    x, do = _inputs(512, "alphabet4", r=r, dv=dv, seed=2)
    print(f"dense dims r={r} dv={dv} dtype={dtype}", flush=True)
    _check(x, do, dtype=dtype, what=f"r{r} dv{dv}")


def test_mixed_dense_sparse_and_soft_rows():
    """One call holding dense rows, sparse rows and soft rows of both kinds."""
    n, b, h = 1024, 2, 4
    rng = np.random.default_rng(17)
    q = rng.integers(0, 256, (b, h, n)).astype(np.int32)
    k = rng.integers(0, 256, (b, h, n)).astype(np.int32)
    q[:, 1] = 9                                   # identical labels
    k[:, 1] = 9
    q[:, 2] = rng.integers(0, 3, (b, n))           # alphabet 3
    k[:, 2] = rng.integers(0, 3, (b, n))
    sq, sk, v = vectors(n, b=b, h=h, r=8, dv=64, seed=5)
    hard = np.ones((b, h), bool)
    hard[0, 1] = False                             # a soft dense row
    hard[1, 0] = False                             # a soft sparse row
    do = oracle.bf16_round(rng.standard_normal(v.shape))
    x = (sq, sk, v, q, k, hard, np.array([0.5, -0.3, 0.0, 1.0], np.float32))
    fl = oracle.dense_rows(q, k, np.ones((b, h), bool))
    assert fl[:, 1].all() and fl[:, 2].all() and not fl[:, [0, 3]].any()
    _check(x, do, what="mixed")


def test_identical_labels_reference_shape():
    """Identical labels at the reference's benchmark shape per row (N2048, R32, DV64): every
    causal pair matches, L[i,j] = j + 1."""
    n = 2048
    x, do = _inputs(n, "equal", b=2, h=3, r=32, dv=64, seed=4)
    print("identical labels N=2048 R=32 DV=64", flush=True)
    _check(x, do, threads=6, what="identical 2048")


def test_identical_labels_headline_length():
    """Identical labels at T = 16384 (two rows): O(N^2) work with O(1) length per cell."""
    n = 16384
    x, do = _inputs(n, "equal", b=1, h=2, r=4, dv=32, seed=6)
    print("identical labels N=16384 R=4 DV=32", flush=True)
    o, g = _check(x, do, threads=2, what="identical 16384")
    assert np.isfinite(o).all() and all(np.isfinite(t).all() for t in g[:3])


def test_dense_rows_with_non_finite_vectors():
    """A non-finite value in a key's vectors reaches exactly the outputs of the queries that
    match that key (the tile kernels skip invalid cells explicitly then)."""
    n = 512
    x, do = _inputs(n, "alphabet4", b=1, h=2, seed=8)
    sq, sk, v, q, k, hard, tau = x
    v = v.copy()
    sk = sk.copy()
    do = do.copy()
    v[0, 100, 0, 3] = np.inf
    sk[0, 200, 1, 1] = np.nan
    do[0, 300, 0, 5] = -np.inf
    x = (sq, sk, v, q, k, hard, tau)
    o, g = _check(x, do, what="non-finite")
    assert np.isnan(o).any() or np.isinf(o).any()


def test_phase1_counts_rows_past_65535():
    """A row of N > 65535 whose keys share one (predecessor, label) bigram: 65792 keys, more
    than a 16-bit count holds; the fused forward's phase-1 histogram counts them in 32 bits."""
    n = 65792
    q = np.ones((1, 1, n), np.int32)
    k = np.full((1, 1, n), 7, np.int32)
    q[0, 0, -2:] = 7
    sq, sk, v = vectors(n, b=1, h=1, r=8, dv=64, seed=12)
    hard = np.ones((1, 1), bool)
    tau = np.array([0.5], np.float32)
    assert not oracle.dense_rows(q, k, hard).any()
    import dism_amd
    out, lse2, m = dism_amd.forward_hard(dev(sq, torch.bfloat16), dev(sk, torch.bfloat16),
                                         dev(v, torch.bfloat16), dev(q), dev(k), dev(hard),
                                         dev(tau), return_matches=True,
                                         out_dtype=torch.float32)
    lut = oracle.log_weights(tau, n)
    o, l2, lm, ja = oracle.forward(sq, sk, v, q, k, hard, lut)
    assert_bits(host(out), o, "out")
    assert_bits(host(lse2), l2, "lse2")
    assert_bits(host(m["length"]), lm, "lmax")
    assert_bits(host(m["index"]), ja, "argmax")
    assert lm[0, 0, -1] == 2 and ja[0, 0, -1] == n - 1


def _periodic_row(n, period, rng):
    base = rng.integers(0, 256, period).astype(np.int32)
    return base[np.arange(n) % period]


def test_long_repeats_take_strip_bounded_walks():
    """Rows with few label collisions but long repeats are not dense.  A random 256-symbol
    pattern of period 200 (every run as long as the row allows: walk cost far above N^2)
    gets strip boundaries from the walk probe (mode 2), so its bigram walks stop within 64
    rows; the same pattern broken once per period (runs of at most 233 labels, cost below
    N^2) stays mode 0 and its walks past RUN_MIN labels take their lengths from the probe's
    list of run ends.  Lengths stay exact: bit for bit against the CPU model's walks."""
    import dism_amd
    from dism_amd.hard_forward import row_modes
    n, b, h = 4096, 1, 4
    rng = np.random.default_rng(23)
    q = rng.integers(0, 256, (b, h, n)).astype(np.int32)
    k = rng.integers(0, 256, (b, h, n)).astype(np.int32)
    q[0, 1] = _periodic_row(n, 200, rng)
    k[0, 1] = q[0, 1]
    q[0, 2] = _periodic_row(n, 233, rng)
    k[0, 2] = np.roll(q[0, 2], 5)
    k[0, 2, ::233] = 999                       # runs broken once per period
    sq, sk, v = vectors(n, b=b, h=h, r=8, dv=64, seed=9)
    hard = np.ones((b, h), bool)
    do = oracle.bf16_round(rng.standard_normal(v.shape))
    tau = np.array([0.5, 0.1, -0.2, 1.0], np.float32)
    assert not oracle.dense_rows(q, k, hard).any()
    x = (sq, sk, v, q, k, hard, tau)
    print("long repeats n=4096", flush=True)
    _check(x, do, threads=4, what="long repeats")
    t = [dev(a, torch.bfloat16) for a in (sq, sk, v)]
    _, _, state = dism_amd.forward_hard(*t, dev(q), dev(k), dev(hard), dev(tau),
                                        save_state=True)
    modes = host(row_modes(state["workspace"], t[0], t[2]))
    assert modes.tolist() == [[0, 2, 0, 0]], modes
