"""CPU pins of the oracle (oracle/dism_cpu_model.c, oracle/dense.py) -- no GPU.

Each oracle function is checked against something it does not restate: closed forms, FP64
evaluation, brute force on tiny inputs, finite differences, special cases with exact answers,
and the two independent fp32 formulations (decomposed vs pairwise) against each other.
The reference ships no golden vectors (its tests build inputs from seeds); the label patterns,
tau lists and special cases below are the ones its tests use (file:line in each docstring).
"""
import math

import numpy as np
import pytest

import oracle
from oracle import dense
from tests import _data

PATTERNS = ["random", "equal", "disjoint", "periodic", "boundary"]


def _ulp_err(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    ulp = np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64)
    return np.abs(got - ref) / ulp


# ---------------------------------------------------------------- elementary functions
def test_exp2_log2_accuracy():
    """Software exp2/log2 (used bit-identically on the GPU) against float64."""
    xs = np.concatenate([np.linspace(-126, 127, 4001), np.linspace(-1, 1, 2001),
                         [0.0, 0.5, -0.5, 1e-8, -1e-8]]).astype(np.float32)
    got = np.array([oracle.exp2f(x) for x in xs], np.float64)
    ref = np.exp2(xs.astype(np.float64))
    assert _ulp_err(got, ref).max() <= 2.0
    ys = np.exp2(np.linspace(-120, 120, 4001)).astype(np.float32)
    ys = np.concatenate([ys, np.linspace(0.5, 2.0, 2001, dtype=np.float32)])
    got = np.array([oracle.log2f(y) for y in ys], np.float64)
    ref = np.log2(ys.astype(np.float64))
    err = np.abs(got - ref)
    # absolute error near log2(1) = 0, relative elsewhere
    assert (err <= np.maximum(2.0 * np.spacing(np.abs(ref).astype(np.float32)), 2e-7)).all()
    assert oracle.exp2f(-1e6) == 0.0


# ---------------------------------------------------------------- log2 weight table
TAU_LIST = [-4.0, -1.0, -1e-4, -1e-6, 0.0, 1e-6, 1e-4, 0.1, 0.5, 1.0, 4.0]


def _lnW64(tau, L):
    """ln sum_{s=1..L} e^{s tau} in float64 by factoring the largest term (exact closed form
    of the geometric sum; dism_v3/tests/test_hard_forward.py:60-71 uses the same table)."""
    s = np.arange(1, L + 1, dtype=np.float64)
    x = s * tau
    m = x.max()
    return m + math.log(np.exp(x - m).sum())


@pytest.mark.parametrize("tau", TAU_LIST)
def test_log_weights_closed_form(tau):
    lut = oracle.log_weights(np.array([tau], np.float32), 600)[0]
    assert lut[0] == np.float32(-1e6)
    t32 = float(np.float32(tau))
    ref = np.array([_lnW64(t32, L) / math.log(2.0) for L in range(1, 601)])
    err = np.abs(lut[1:].astype(np.float64) - ref)
    assert (err <= 2.0 * np.spacing(np.abs(ref).astype(np.float32)) + 1e-7).all()
    if tau == 0.0:
        np.testing.assert_array_equal(lut[1:], np.log2(np.arange(1, 601)).astype(np.float32))


@pytest.mark.parametrize("tau", TAU_LIST)
def test_dlog_weights_finite_difference(tau):
    """g_L = d ln W_L / d tau (dism_v3/src/hard_backward.cu:8-23) against a central
    difference of the float64 closed form and the exact mean sum s e^{s tau}/sum e^{s tau}."""
    g = oracle.dlog_weights(np.array([tau], np.float32), 300)[0]
    assert g[0] == 0.0
    t = float(np.float32(tau))
    for L in (1, 2, 3, 7, 64, 299):
        s = np.arange(1, L + 1, dtype=np.float64)
        x = s * t
        w = np.exp(x - x.max())
        exact = (s * w).sum() / w.sum()
        assert abs(g[L] - exact) <= 4e-7 * max(1.0, abs(exact)), (L, g[L], exact)
        h = 1e-5
        fd = (_lnW64(t + h, L) - _lnW64(t - h, L)) / (2 * h)
        assert abs(g[L] - fd) <= 1e-5 * max(1.0, abs(fd))


# ---------------------------------------------------------------- labels
def test_sign_labels_bits():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((2, 33, 3, 8)).astype(np.float32)
    x[0, 0, 0, :] = 0.0
    x[0, 1, 0, 2] = -0.0
    x[0, 2, 0, 3] = np.nan
    got = oracle.sign_labels(x)
    bits = (x > 0).astype(np.int64) * (1 << np.arange(8))
    ref = bits.sum(-1).transpose(0, 2, 1).astype(np.int32)
    np.testing.assert_array_equal(got, ref)
    assert got[0, 0, 0] == 0


# ---------------------------------------------------------------- match lengths / boundaries
def _brute_L(q, k):
    n = q.shape[0]
    L = np.zeros((n, n), np.int64)
    for i in range(n):
        for j in range(i + 1):
            c = 0
            while i - c >= 0 and j - c >= 0 and q[i - c] == k[j - c]:
                c += 1
            L[i, j] = c
    return L


@pytest.mark.parametrize("pattern", PATTERNS)
def test_lengths_and_walk_brute_force(pattern):
    q, k = _data.labels(97, pattern, b=1, h=1)
    L = _brute_L(q[0, 0], k[0, 0])
    np.testing.assert_array_equal(dense.dense_lengths(q[0, 0], k[0, 0]), L)
    for i, j in [(0, 0), (5, 3), (96, 96), (96, 0), (60, 30)]:
        assert oracle.suffix_walk(q[0, 0], k[0, 0], i, j) == L[i, j]


@pytest.mark.parametrize("pattern", PATTERNS)
@pytest.mark.parametrize("strip", [32, 64])
def test_boundary_definitions(pattern, strip):
    """Strip summaries R[c,j] (dism_v3/tests/test_hard_summary.py:37-49) and composed
    boundaries j - L[r,j] (test_hard_chunk.py:24-36) by brute force."""
    n = 200
    q, k = _data.labels(n, pattern, b=1, h=2)
    hard = np.array([[True, False]])
    summ = oracle.boundary(q, k, hard, strip=strip, composed=False)
    comp = oracle.boundary(q, k, hard, strip=strip, composed=True)
    C = (n - 1) // strip
    L = _brute_L(q[0, 0], k[0, 0])
    for c in range(C):
        r = c * strip + strip - 1
        for j in range(n):
            if j > r:
                assert summ[0, 0, c, j] == -1 and comp[0, 0, c, j] == -1
                continue
            assert comp[0, 0, c, j] == j - L[r, j]
            seg = min(strip, j + 1)
            cnt = min(L[r, j], seg)
            assert summ[0, 0, c, j] == (-1 if cnt == seg else j - cnt)
    assert (summ[0, 1] == -1).all() and (comp[0, 1] == -1).all()
    if strip == 32:  # the chunk pass composes the strip-32 summaries into the boundary
        np.testing.assert_array_equal(oracle.chunk(summ), comp)


# ---------------------------------------------------------------- forward
def _inputs(n, pattern, b=2, h=3, r=8, dv=64, seed=11):
    q, k = _data.labels(n, pattern, b=b, h=h)
    sq, sk, v = _data.vectors(n, b=b, h=h, r=r, dv=dv, seed=seed)
    hard = _data.flags(b, h)
    tau = _data.taus(h)
    return sq, sk, v, q, k, hard, tau


@pytest.mark.parametrize("pattern", PATTERNS)
def test_forward_matches_dense_fp64(pattern):
    sq, sk, v, q, k, hard, tau = _inputs(160, pattern)
    lut = oracle.log_weights(tau, 160)
    out, l2, lmax, jarg = oracle.forward(sq, sk, v, q, k, hard, lut)
    ref, rl2 = dense.dense_forward(sq, sk, v, q, k, hard, tau)
    np.testing.assert_allclose(out, ref, rtol=1e-4, atol=2e-6)
    np.testing.assert_allclose(l2, rl2, rtol=1e-5, atol=1e-5)
    # decomposed vs pairwise fp32 formulation: same mathematics, other association
    out2, l22, lmax2, jarg2 = oracle.forward(sq, sk, v, q, k, hard, lut, direct=True)
    np.testing.assert_allclose(out, out2, rtol=1e-5, atol=1e-6)
    np.testing.assert_array_equal(lmax, lmax2)
    np.testing.assert_array_equal(jarg, jarg2)


@pytest.mark.parametrize("pattern", ["random", "periodic", "equal"])
def test_longest_match_brute_force(pattern):
    sq, sk, v, q, k, hard, tau = _inputs(90, pattern, b=1, h=1)
    hard = np.ones((1, 1), bool)
    lut = oracle.log_weights(tau, 90)
    _, _, lmax, jarg = oracle.forward(sq, sk, v, q, k, hard, lut)
    L = _brute_L(q[0, 0], k[0, 0])
    for i in range(90):
        best = L[i, :i + 1].max()
        assert lmax[0, 0, i] == best
        exp_j = -1 if best == 0 else int(np.nonzero(L[i, :i + 1] == best)[0].max())
        assert jarg[0, 0, i] == exp_j


def test_forward_special_cases():
    """dism_v3/tests/test_hard_forward.py:104-115: disjoint labels -> O = 0, lse2 = 0;
    sq -> -sq negates O exactly and keeps lse2; sq = 0 -> O = 0; a single match gives
    O = W s v / (1 + W) with W = e^tau."""
    sq, sk, v, q, k, hard, tau = _inputs(64, "disjoint")
    lut = oracle.log_weights(tau, 64)
    out, l2, _, _ = oracle.forward(sq, sk, v, q, k, hard, lut)
    assert not out.any() and not l2.any()
    sq, sk, v, q, k, hard, tau = _inputs(64, "random")
    lut = oracle.log_weights(tau, 64)
    o1, l1, _, _ = oracle.forward(sq, sk, v, q, k, hard, lut)
    o2, l2_, _, _ = oracle.forward(-sq, sk, v, q, k, hard, lut)
    np.testing.assert_array_equal(o2, -o1)
    np.testing.assert_array_equal(l2_, l1)
    o3, _, _, _ = oracle.forward(np.zeros_like(sq), sk, v, q, k, hard, lut)
    assert not o3.any()
    # single match: query 5 sees exactly key 3
    n = 16
    qq = np.full((1, 1, n), 1000, np.int32)
    kk = np.arange(n, dtype=np.int32).reshape(1, 1, n)
    qq[0, 0, 5] = 3
    rng = np.random.default_rng(0)
    sq1 = oracle.bf16_round(rng.standard_normal((1, n, 1, 8)).astype(np.float32))
    sk1 = oracle.bf16_round(rng.standard_normal((1, n, 1, 8)).astype(np.float32))
    v1 = oracle.bf16_round(rng.standard_normal((1, n, 1, 64)).astype(np.float32))
    t = np.array([0.3], np.float32)
    lut = oracle.log_weights(t, n)
    out, l2, lmax, jarg = oracle.forward(sq1, sk1, v1, qq, kk, np.ones((1, 1), bool), lut)
    W = math.exp(float(t[0]))
    s = float(np.dot(sq1[0, 5, 0].astype(np.float64), sk1[0, 3, 0].astype(np.float64)))
    np.testing.assert_allclose(out[0, 5, 0], W * s * v1[0, 3, 0] / (1 + W), rtol=2e-6,
                               atol=1e-7)
    assert lmax[0, 0, 5] == 1 and jarg[0, 0, 5] == 3
    assert abs(l2[0, 0, 5] - math.log2(1 + W)) < 1e-6


def test_forward_causality():
    """Changing v at positions >= t leaves O[< t] bit-identical (test_hard_forward.py:164-169)."""
    sq, sk, v, q, k, hard, tau = _inputs(128, "periodic")
    lut = oracle.log_weights(tau, 128)
    o1, _, _, _ = oracle.forward(sq, sk, v, q, k, hard, lut)
    v2 = v.copy()
    v2[:, 70:] = 7.0
    o2, _, _, _ = oracle.forward(sq, sk, v2, q, k, hard, lut)
    np.testing.assert_array_equal(o1[:, :70], o2[:, :70])


# ---------------------------------------------------------------- backward
@pytest.mark.parametrize("pattern", ["random", "periodic", "equal", "boundary"])
def test_backward_matches_dense_fp64(pattern):
    sq, sk, v, q, k, hard, tau = _inputs(150, pattern)
    rng = np.random.default_rng(5)
    do = oracle.bf16_round(rng.standard_normal(v.shape).astype(np.float32))
    lut = oracle.log_weights(tau, 150)
    dl = oracle.dlog_weights(tau, 150)
    _, l2, _, _ = oracle.forward(sq, sk, v, q, k, hard, lut)
    dsq, dsk, dv, dtau, _ = oracle.backward(sq, sk, v, do, q, k, hard, lut, dl, l2)
    rsq, rsk, rv, rtau = dense.dense_backward(sq, sk, v, do, q, k, hard, tau)
    for got, ref in ((dsq, rsq), (dsk, rsk), (dv, rv)):
        scale = max(np.abs(ref).max(), 1e-30)
        assert np.abs(got - ref).max() <= 1e-4 * scale
    assert np.abs(dtau - rtau).max() <= 1e-3 * max(np.abs(rtau).max(), 1e-6)
    g2 = oracle.backward(sq, sk, v, do, q, k, hard, lut, dl, l2, direct=True)
    for a_, b_ in zip((dsq, dsk, dv), g2[:3]):
        assert np.abs(a_ - b_).max() <= 1e-5 * max(np.abs(b_).max(), 1e-30)


def test_backward_finite_differences():
    """Gradients of L = sum(dO * O) by central differences of the FP64 dense forward
    (the reference checks its oracle with gradcheck, test_dism_v3_ref.py:85-94)."""
    sq, sk, v, q, k, hard, tau = _inputs(24, "periodic", b=1, h=2, r=4, dv=32)
    hard = np.ones((1, 2), bool)
    rng = np.random.default_rng(9)
    do = rng.standard_normal(v.shape)
    lut = oracle.log_weights(tau, 24)
    dl = oracle.dlog_weights(tau, 24)
    _, l2, _, _ = oracle.forward(sq, sk, v, q, k, hard, lut)
    dsq, dsk, dv, dtau, _ = oracle.backward(sq, sk, v, do.astype(np.float32), q, k, hard, lut,
                                            dl, l2)

    def loss(a, b_, c, t):
        o, _ = dense.dense_forward(a, b_, c, q, k, hard, t)
        return float((o * do).sum())

    h = 1e-6
    base = [x.astype(np.float64) for x in (sq, sk, v)]
    for which, grad in ((0, dsq), (1, dsk), (2, dv)):
        for idx in [(0, 3, 0, 1), (0, 20, 1, 0), (0, 11, 1, 2)]:
            xs = [b_.copy() for b_ in base]
            xs[which][idx] += h
            up = loss(*xs, tau.astype(np.float64))
            xs[which][idx] -= 2 * h
            dn = loss(*xs, tau.astype(np.float64))
            fd = (up - dn) / (2 * h)
            assert abs(grad[idx] - fd) <= 2e-4 * max(1.0, abs(fd)), (which, idx, grad[idx], fd)
    for hh in range(2):
        tp = tau.astype(np.float64).copy()
        tp[hh] += 1e-5
        tm = tau.astype(np.float64).copy()
        tm[hh] -= 1e-5
        fd = (loss(*base, tp) - loss(*base, tm)) / 2e-5
        assert abs(dtau[hh] - fd) <= 1e-3 * max(1.0, abs(fd)), (hh, dtau[hh], fd)


def test_tau_reduce_order():
    """orc_tau_reduce against an explicit three-level loop (blocks of 64 rows, groups of 32
    blocks) and the exact sum; lengths on and off the block and group grid."""
    rng = np.random.default_rng(1)
    for B, H, N in ((3, 4, 700), (2, 2, 4096), (1, 3, 64 * 32 * 3 + 5)):
        rowtau = rng.standard_normal((B, H, N)).astype(np.float32)
        out = oracle.tau_reduce(rowtau)
        for h in range(H):
            flat = rowtau[:, h, :].reshape(-1).astype(np.float64)
            outer = 0.0
            for g in range(0, flat.size, 64 * 32):
                mid = 0.0
                for s in range(g, min(g + 64 * 32, flat.size), 64):
                    inner = 0.0
                    for x in flat[s:s + 64]:
                        inner += x
                    mid += inner
                outer += mid
            assert out[h] == np.float32(outer)
            assert abs(float(out[h]) - float(np.sum(flat, dtype=np.longdouble))) <= \
                2e-7 * max(1.0, float(np.abs(flat).sum()))


def test_forward_with_query_resets_pinned_by_fp64():
    """orc_forward_reset (inference resets) against the FP64 restatement of the reference's
    inference oracle (dism_v3/tests/test_sam_inference.py:9-29, predecessor score -inf at a
    reset query); without resets it is orc_forward exactly, and resets do change the result."""
    from oracle import dense
    rng = np.random.default_rng(83)
    b, h, n, r, dv = 2, 2, 79, 16, 32
    for alphabet in (1, 4):
        iq = rng.integers(0, alphabet, (b, h, n)).astype(np.int32)
        ik = rng.integers(0, alphabet, (b, h, n)).astype(np.int32)
        sq, sk, v = (oracle.bf16_round(rng.standard_normal((b, n, h, c)) * 0.2)
                     for c in (r, r, dv))
        tau = np.array([0.0, 0.35], dtype=np.float32)
        hard = np.ones((b, h), bool)
        lut = oracle.log_weights(tau, n)
        reset = np.zeros((b, h, n), bool)
        reset[..., 17::19] = True
        got, l2, _, _ = oracle.forward(sq, sk, v, iq, ik, hard, lut, reset=reset)
        ref, l2d = dense.dense_forward(sq, sk, v, iq, ik, hard, tau, reset=reset)
        np.testing.assert_allclose(got, ref, atol=2e-6, rtol=2e-4)
        np.testing.assert_allclose(l2, l2d, atol=2e-5, rtol=2e-6)
        # (calls with resets never take the level path, so the plain call is given the
        # same row modes: direct for the dense rows)
        plain = oracle.forward(sq, sk, v, iq, ik, hard, lut,
                               dense=oracle.dense_rows(iq, ik, hard))[0]
        none = oracle.forward(sq, sk, v, iq, ik, hard, lut, reset=np.zeros_like(reset))[0]
        assert np.array_equal(plain.view(np.uint32), none.view(np.uint32))
        assert np.abs(plain - got).max() > 1e-3
    starts = oracle.reset_starts(np.array([[[0, 1, 0, 0, 1, 0]]], bool))
    assert starts.tolist() == [[[0, 1, 1, 1, 4, 4]]]


# ---------------------------------------------------------------- codebook argmax labels
def _exact_vocab_labels(x, vocab):
    """Argmax over v of sum_d x[d] * e[v, d] in exact rational arithmetic (every bf16 value is
    a dyadic rational, so the scaled products are Python integers), first index on ties."""
    from fractions import Fraction
    B, N, H, D = x.shape
    shared = vocab.ndim == 2
    V = vocab.shape[-2]
    xs = [[[[Fraction(float(t)) for t in x[b_, n_, h_]] for h_ in range(H)] for n_ in range(N)]
          for b_ in range(B)]
    es = [[[Fraction(float(t)) for t in (vocab[v_] if shared else vocab[h_, v_])]
           for v_ in range(V)] for h_ in range(1 if shared else H)]
    out = np.empty((B, H, N), np.int32)
    for b_ in range(B):
        for n_ in range(N):
            for h_ in range(H):
                tok = xs[b_][n_][h_]
                table = es[0 if shared else h_]
                best, bi = None, 0
                for v_ in range(V):
                    sc = sum(a * e for a, e in zip(tok, table[v_]))
                    if best is None or sc > best:
                        best, bi = sc, v_
                out[b_, h_, n_] = bi
    return out


def test_vocab_labels_exact_argmax():
    """orc_vocab_labels (fp64 sums in d order, first index on ties) against exact rational
    arithmetic: random rows, duplicated codebook rows (exact ties: the first index wins) and
    rows one bf16 ulp apart (near ties: the larger exact score wins, asserted explicitly).
    The fp64 sum of D bf16 products is exact while the products' exponents span less than
    about 53 - 16 - log2(D) bits, which holds for these inputs."""
    rng = np.random.default_rng(29)
    B, N, H, D, V = 1, 24, 2, 32, 40
    vocab = oracle.bf16_round(rng.standard_normal((H, V, D)))
    vocab[:, 5] = oracle.bf16_round(vocab[:, 5] * 3.0)   # long rows: tokens along them
    vocab[:, 8] = oracle.bf16_round(vocab[:, 8] * 3.0)   # pick them over every other row
    vocab[:, 17] = vocab[:, 5]                      # exact duplicate of row 5
    vocab[:, 30] = vocab[:, 8]
    bits = vocab.view(np.uint32)
    bits[:, 30, 3] += 1 << 16                       # row 30 = row 8 with one coordinate +1 ulp
    x = oracle.bf16_round(rng.standard_normal((B, N, H, D)))
    x[0, :6] = vocab[:, 5][None] * 2.0              # tokens aimed at the duplicated rows
    x[0, 6:12] = vocab[:, 8][None]                  # near tie between rows 8 and 30: the
    # bump raised |e[30,3]|, and x[3] has e[8,3]'s sign, so row 30 is larger by one ulp term
    got = oracle.vocab_labels(x, vocab)
    want = _exact_vocab_labels(x, vocab)
    np.testing.assert_array_equal(got, want)
    assert (got[0, :, :6] == 5).all()               # first index of the exact tie
    assert (got[0, :, 6:12] == 30).all()            # the one-ulp larger row
    shared = oracle.bf16_round(rng.standard_normal((V, D)))
    np.testing.assert_array_equal(oracle.vocab_labels(x, shared), _exact_vocab_labels(x, shared))
