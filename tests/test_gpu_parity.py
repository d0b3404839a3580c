"""HIP path vs the CPU oracle on identical seeded inputs (run on the MI355X).

Integers (summaries, boundaries, lengths, argmax) and the documented fp32 operation
sequences (LUT, dLUT, outputs, normalizer, gradients) are compared bit for bit against the
CPU model (oracle/dism_cpu_model.c); outputs and gradients are also compared against the
FP64 dense restatement of the reference oracle within the reference's own tolerances
(dism_v3/tests/test_hard_forward.py:54-57, test_hard_backward.py:248-254) and the north-star
gradient bound (max relative error 1e-3).
"""
import numpy as np
import pytest
import torch

import oracle
from oracle import dense
from tests._data import flags, labels, taus, vectors

pytestmark = pytest.mark.gpu

DEV = "cuda"


def dev(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    return t if dtype is None else t.to(dtype)


def host(t):
    return t.detach().float().cpu().numpy() if t.dtype.is_floating_point else t.cpu().numpy()


def assert_bits(actual, expected, what):
    a = np.ascontiguousarray(actual)
    e = np.ascontiguousarray(expected)
    assert a.shape == e.shape, (what, a.shape, e.shape)
    if a.dtype.kind == "f":
        bad = a.view(np.uint32) != e.astype(np.float32).view(np.uint32)
        bad &= ~(np.isnan(a) & np.isnan(e))
    else:
        bad = a != e
    assert not bad.any(), f"{what}: {int(bad.sum())} of {bad.size} differ; first at " \
                          f"{np.argwhere(bad)[:3].tolist()}"


def max_rel(actual, expected):
    return float(np.abs(actual - expected).max() / max(np.abs(expected).max(), 1e-30))


# ---------------------------------------------------------------- tables
TAU_SWEEP = [-4.0, -1.0, -0.5, -1e-4, -1e-6, -1e-12, 0.0, 1e-12, 1e-6, 1e-4, 0.1, 0.5, 4.0]


@pytest.mark.parametrize("n", [256, 2048])
def test_log_weight_tables_bit_exact(n):
    import dism_amd
    tau = np.array(TAU_SWEEP, dtype=np.float32)
    lut = host(dism_amd.hard_log_weights(dev(tau), n))
    assert_bits(lut, oracle.log_weights(tau, n), "lut")
    g = host(dism_amd.hard_dlog_weights(dev(tau), n + 1))
    assert_bits(g, oracle.dlog_weights(tau, n), "dlut")
    # closed form (dism_v3/tests/test_hard_forward.py:60-71)
    length = np.arange(1, n + 1, dtype=np.float64)
    t = tau.astype(np.float64)[:, None]
    a = np.abs(t)
    with np.errstate(divide="ignore", invalid="ignore"):
        exp = (np.where(t > 0, length * t, t) + np.log(-np.expm1(-length * a)) -
               np.log(-np.expm1(-a))) / np.log(2.0)
    exp[tau == 0] = np.log2(length)
    assert (lut[:, 0] == -1e6).all()
    np.testing.assert_allclose(lut[:, 1:], exp, atol=2e-5, rtol=2e-6)


# ---------------------------------------------------------------- integer core
PATTERNS = ["random", "equal", "disjoint", "periodic", "boundary", "alphabet4", "collide"]


@pytest.mark.parametrize("n", [256, 1024])
@pytest.mark.parametrize("pattern", PATTERNS)
def test_summary_chunk_boundary_exact(n, pattern):
    import dism_amd
    q, k = labels(n, pattern)
    hard = np.array([[True, False, True], [False, True, True]])
    iq, ik, hd = dev(q), dev(k), dev(hard)
    summ = dism_amd.summarize_hard(iq, ik, hd)
    assert_bits(host(summ), oracle.boundary(q, k, hard, 32, composed=False), "summary")
    chained = dism_amd.hard_chunk_scan(summ)
    expected = oracle.boundary(q, k, hard, 32, composed=True)
    assert_bits(host(chained), expected, "chunk")
    assert_bits(host(dism_amd.hard_boundary(iq, ik, hd, strip=32)), expected, "boundary32")
    assert_bits(host(dism_amd.hard_boundary(iq, ik, hd, strip=256)),
                oracle.boundary(q, k, hard, 256, composed=True), "boundary256")
    inplace = summ.clone()
    out = dism_amd.hard_chunk_scan(inplace, inplace=True)
    assert out.data_ptr() == inplace.data_ptr()
    assert_bits(host(out), expected, "chunk inplace")


def test_chunk_random_summaries_with_poison():
    """dism_v3/tests/test_hard_chunk.py:39-58: poisoned non-causal entries never leak."""
    import dism_amd
    n = 512
    rng = np.random.default_rng(63)
    s = rng.integers(-1, n, (2, 3, (n - 1) // 32, n), dtype=np.int32)
    for cp in range(s.shape[2]):
        s[:, :, cp, cp * 32 + 32:] = np.iinfo(np.int32).max
    got = host(dism_amd.hard_chunk_scan(dev(s)))
    assert_bits(got, oracle.chunk(s), "chunk poison")


def test_sign_labels_exact():
    import dism_amd
    rng = np.random.default_rng(5)
    x = rng.standard_normal((2, 512, 3, 8)).astype(np.float32)
    x[0, 0, 0, :] = 0.0
    x[0, 1, 0, :] = -0.0
    x[0, 2, 0, 3] = np.nan
    expected = oracle.sign_labels(x)
    assert_bits(host(dism_amd.sign_labels(dev(x))), expected, "labels f32")
    xb = oracle.bf16_round(x)
    assert_bits(host(dism_amd.sign_labels(dev(xb, torch.bfloat16))), oracle.sign_labels(xb),
                "labels bf16")


@pytest.mark.parametrize("b,n,h", [(1, 1, 1), (3, 100, 16), (2, 130, 64), (1, 70, 65)])
def test_sign_labels_tiled_shapes(b, n, h):
    """bf16 d = 8 rows take the tiled kernel (64 positions x all heads per workgroup) for
    H <= 64; ragged position counts, one position, and H = 65 (the per-token kernel)."""
    import dism_amd
    rng = np.random.default_rng(b * 1000 + n + h)
    x = oracle.bf16_round(rng.standard_normal((b, n, h, 8)).astype(np.float32))
    x[0, 0, 0, :] = 0.0
    assert_bits(host(dism_amd.sign_labels(dev(x, torch.bfloat16))), oracle.sign_labels(x),
                f"labels bf16 {b}x{n}x{h}")


# ---------------------------------------------------------------- forward
def _inputs(n, pattern, b=2, h=3, r=8, dv=64):
    q, k = labels(n, pattern, b, h)
    sq, sk, v = vectors(n, b, h, r, dv)
    return sq, sk, v, q, k, flags(b, h), taus(h)


def _run_forward(x, dtype, carry_strip, out_dtype=torch.float32):
    import dism_amd
    sq, sk, v, q, k, hard, tau = x
    return dism_amd.forward_hard(dev(sq, dtype), dev(sk, dtype), dev(v, dtype), dev(q), dev(k),
                                 dev(hard), dev(tau), carry_strip=carry_strip,
                                 return_matches=True, out_dtype=out_dtype)


@pytest.mark.parametrize("pattern", PATTERNS + ["alphabet256"])
@pytest.mark.parametrize("n,carry", [(256, 0), (512, 256), (1024, 32), (1024, 0)])
def test_forward_bit_exact(n, pattern, carry):
    x = _inputs(n, pattern)
    sq, sk, v, q, k, hard, tau = x
    lut = oracle.log_weights(tau, n)
    o, l2, lm, ja = oracle.forward(sq, sk, v, q, k, hard, lut)
    out, lse2, m = _run_forward(x, torch.bfloat16, carry)
    assert_bits(host(out), o, "out f32")
    assert_bits(host(lse2), l2, "lse2")
    assert_bits(host(m["length"]), lm, "lmax")
    assert_bits(host(m["index"]), ja, "argmax")
    out16, lse16, _ = _run_forward(x, torch.bfloat16, carry, torch.bfloat16)
    assert_bits(host(out16), oracle.bf16_round(o), "out bf16")
    assert_bits(host(lse16), l2, "lse2 (bf16 run)")
    # FP64 dense restatement of the reference oracle, reference tolerances
    od, l2d = dense.dense_forward(sq, sk, v, q, k, hard, tau)
    np.testing.assert_allclose(host(out16), od, atol=0.008, rtol=0.025)
    assert np.linalg.norm(host(out16) - od) / max(np.linalg.norm(od), 1e-8) < 0.01
    np.testing.assert_allclose(host(lse2), l2d, atol=2e-5, rtol=2e-6)


@pytest.mark.parametrize("r,dv", [(2, 64), (4, 32), (16, 64), (32, 128), (8, 128)])
def test_forward_dims_and_fp32(r, dv):
    x = _inputs(512, "alphabet4", r=r, dv=dv)
    sq, sk, v, q, k, hard, tau = x
    lut = oracle.log_weights(tau, 512)
    o, l2, lm, ja = oracle.forward(sq, sk, v, q, k, hard, lut)
    for dt in (torch.bfloat16, torch.float32):
        out, lse2, m = _run_forward(x, dt, 256)
        assert_bits(host(out), o, f"out {dt}")
        assert_bits(host(lse2), l2, "lse2")


def test_forward_fp32_inputs_not_bf16_representable():
    rng = np.random.default_rng(11)
    n, b, h = 256, 1, 4
    sq, sk, v = (rng.standard_normal((b, n, h, d)).astype(np.float32) for d in (8, 8, 64))
    q = oracle.sign_labels(sq)
    k = oracle.sign_labels(sk)
    hard = np.ones((b, h), bool)
    tau = taus(h)
    o, l2, lm, ja = oracle.forward(sq, sk, v, q, k, hard, oracle.log_weights(tau, n))
    out, lse2, m = _run_forward((sq, sk, v, q, k, hard, tau), torch.float32, 256)
    assert_bits(host(out), o, "out")
    assert_bits(host(m["index"]), ja, "argmax")


@pytest.mark.parametrize("tau", [-1.0, -1e-6, 0.0, 1e-6, 0.1, 0.5, 4.0])
def test_forward_long_all_match(tau):
    """dism_v3/tests/test_hard_forward.py:84-90 (1024-long all-equal chains)."""
    x = list(_inputs(1024, "equal", b=1, h=1))
    x[-1] = np.array([tau], dtype=np.float32)
    sq, sk, v, q, k, hard, t = x
    o, l2, _, _ = oracle.forward(sq, sk, v, q, k, hard, oracle.log_weights(t, 1024))
    out, lse2, _ = _run_forward(x, torch.bfloat16, 256)
    assert_bits(host(out), o, "out")
    assert_bits(host(lse2), l2, "lse2")
    od, l2d = dense.dense_forward(sq, sk, v, q, k, hard, t)
    np.testing.assert_allclose(host(out), od, atol=0.008, rtol=0.025)
    np.testing.assert_allclose(host(lse2), l2d, atol=2e-5, rtol=2e-6)


def test_forward_signed_readout_fallback_and_skip():
    """dism_v3/tests/test_hard_forward.py:101-119."""
    import dism_amd
    sq, sk, v, q, k, hard, tau = _inputs(512, "boundary")
    args = [dev(sq, torch.bfloat16), dev(sk, torch.bfloat16), dev(v, torch.bfloat16), dev(q),
            dev(k), dev(hard), dev(tau)]
    out, norm = dism_amd.forward_hard(*args)
    args[0] = -args[0]
    neg, neg_norm = dism_amd.forward_hard(*args)
    assert torch.equal(neg, -out) and torch.equal(neg_norm, norm)
    args[0].zero_()
    zero, zero_norm = dism_amd.forward_hard(*args)
    assert not zero.count_nonzero() and torch.equal(zero_norm, norm)
    args[3].fill_(1)
    args[4].fill_(2)
    zero, zero_norm = dism_amd.forward_hard(*args)
    assert not zero.count_nonzero() and not zero_norm.count_nonzero()
    args[5].fill_(False)
    for t in args[:3]:
        t.fill_(float("nan"))
    zero, zero_norm = dism_amd.forward_hard(*args)
    assert not zero.count_nonzero() and not zero_norm.count_nonzero()


def test_forward_causality():
    """dism_v3/tests/test_hard_forward.py:164-169: v at positions >= t never reaches O[<t]."""
    import dism_amd
    sq, sk, v, q, k, hard, tau = _inputs(512, "equal")
    args = [dev(sq, torch.bfloat16), dev(sk, torch.bfloat16), dev(v, torch.bfloat16), dev(q),
            dev(k), dev(hard), dev(tau)]
    original, _ = dism_amd.forward_hard(*args)
    args[2][:, 127:] = 20
    changed, _ = dism_amd.forward_hard(*args)
    assert torch.equal(original[:, :127], changed[:, :127])


def test_hard_readout_reference_boundary_and_validation():
    import dism_amd
    sq, sk, v, q, k, hard, tau = _inputs(256, "boundary")
    x = [dev(sq, torch.bfloat16), dev(sk, torch.bfloat16), dev(v, torch.bfloat16), dev(q),
         dev(k), dev(hard), dev(tau)]
    out, norm, state = dism_amd.forward_hard(*x, save_state=True)
    again, again_norm = dism_amd.hard_readout(*x[:6], state["boundary"], state["log_weights"])
    assert torch.equal(out, again) and torch.equal(norm, again_norm)
    none, none_norm = dism_amd.hard_readout(*x[:6], None, state["log_weights"])
    assert torch.equal(out, none) and torch.equal(norm, none_norm)
    with pytest.raises(RuntimeError, match="too short"):
        dism_amd.hard_readout(*x[:6], state["boundary"],
                              state["log_weights"][:, :128].contiguous())
    with pytest.raises(RuntimeError, match="boundary"):
        dism_amd.hard_readout(*x[:6], state["boundary"].float(), state["log_weights"])
    bad = list(x)
    bad[5] = x[5][:, :, None].expand(2, 3, 256)
    with pytest.raises(RuntimeError, match="token-level"):
        dism_amd.forward_hard(*bad)
    with pytest.raises(RuntimeError, match="CTA"):
        dism_amd.forward_hard(*x, ctas=-1)


# ---------------------------------------------------------------- backward
def _run_backward(x, dout, dtype, carry):
    import dism_amd
    sq, sk, v, q, k, hard, tau = x
    t = [dev(sq, dtype), dev(sk, dtype), dev(v, dtype), dev(q), dev(k), dev(hard), dev(tau)]
    out, norm, state = dism_amd.forward_hard(*t, save_state=True, carry_strip=carry)
    return dism_amd.backward_hard(*t[:3], dev(dout, dtype), *t[3:6], norm, state), norm


@pytest.mark.parametrize("pattern", PATTERNS + ["alphabet256"])
@pytest.mark.parametrize("n,carry", [(256, 0), (512, 256), (512, 32)])
def test_backward_bit_exact(n, pattern, carry):
    x = _inputs(n, pattern)
    sq, sk, v, q, k, hard, tau = x
    dout = oracle.bf16_round(np.random.default_rng(7).standard_normal(v.shape))
    (dsq, dsk, dvv, dtau), norm = _run_backward(x, dout, torch.bfloat16, carry)
    lut = oracle.log_weights(tau, n)
    dl = oracle.dlog_weights(tau, n)
    _, l2, _, _ = oracle.forward(sq, sk, v, q, k, hard, lut)
    assert_bits(host(norm), l2, "lse2")
    esq, esk, ev, etau, _ = oracle.backward(sq, sk, v, dout, q, k, hard, lut, dl, l2)
    assert_bits(host(dsq), esq, "dsq")
    assert_bits(host(dsk), esk, "dsk")
    assert_bits(host(dvv), ev, "dv")
    assert_bits(host(dtau), etau, "dtau")
    # FP64 dense restatement: reference tolerances and the 1e-3 north-star bound
    gd = dense.dense_backward(sq, sk, v, dout, q, k, hard, tau)
    for got, want, name in zip((dsq, dsk, dvv), gd[:3], ("dsq", "dsk", "dv")):
        got = host(got)
        np.testing.assert_allclose(got, want, atol=0.008, rtol=0.025, err_msg=name)
        assert max_rel(got, want) < 1e-3, (name, max_rel(got, want))
        assert not got[~np.broadcast_to(hard[:, None, :, None], got.shape)].any()
    np.testing.assert_allclose(host(dtau), gd[3], atol=0.003, rtol=0.01)


@pytest.mark.parametrize("tau", [-4.0, -1e-4, -1e-6, 0.0, 1e-6, 1e-4, 0.1, 0.5, 4.0])
def test_backward_tau_long_chain(tau):
    """dism_v3/tests/test_hard_backward.py:257-265 (1024-long all-equal chains)."""
    x = list(_inputs(1024, "equal", b=1, h=1))
    x[-1] = np.array([tau], dtype=np.float32)
    dout = oracle.bf16_round(np.random.default_rng(9).standard_normal(x[2].shape))
    (dsq, dsk, dvv, dtau), _ = _run_backward(x, dout, torch.bfloat16, 256)
    sq, sk, v, q, k, hard, t = x
    gd = dense.dense_backward(sq, sk, v, dout, q, k, hard, t)
    np.testing.assert_allclose(host(dtau), gd[3], atol=0.003, rtol=0.01)
    for got, want in zip((dsq, dsk, dvv), gd[:3]):
        assert max_rel(host(got), want) < 1e-3


def test_backward_recompute_and_autograd_match():
    import dism_amd
    x = _inputs(512, "alphabet4")
    sq, sk, v, q, k, hard, tau = x
    dout = oracle.bf16_round(np.random.default_rng(3).standard_normal(v.shape))
    (dsq, dsk, dvv, dtau), _ = _run_backward(x, dout, torch.bfloat16, 256)
    t = [dev(sq, torch.bfloat16), dev(sk, torch.bfloat16), dev(v, torch.bfloat16)]
    rec = dism_amd.backward_hard_recompute(*t, dev(dout, torch.bfloat16), dev(q), dev(k),
                                           dev(hard), dev(tau))
    assert torch.equal(rec["sq_vec"], dsq) and torch.equal(rec["v"], dvv)
    assert torch.equal(rec["sk_vec"], dsk) and torch.equal(rec["rtau"], dtau)
    leaves = [dev(a, torch.float32).requires_grad_() for a in (sq, sk, v)]
    tau_t = dev(tau).requires_grad_()
    out = dism_amd.dism_core_hard(*leaves, dev(q), dev(k), dev(hard), tau_t)
    out.backward(dev(dout, torch.float32))
    (esq, esk, ev, etau), _ = _run_backward(x, dout, torch.float32, 256)
    assert torch.equal(leaves[0].grad, esq) and torch.equal(leaves[2].grad, ev)
    assert torch.equal(leaves[1].grad, esk) and torch.equal(tau_t.grad, etau)


def test_backward_all_soft_and_validation():
    import dism_amd
    x = list(_inputs(256, "random"))
    x[5] = np.zeros_like(x[5])
    dout = np.ones_like(x[2])
    (dsq, dsk, dvv, dtau), _ = _run_backward(x, dout, torch.bfloat16, 256)
    assert all(not t.count_nonzero() for t in (dsq, dsk, dvv, dtau))
    sq, sk, v, q, k, hard, tau = _inputs(256, "random")
    t = [dev(sq, torch.bfloat16), dev(sk, torch.bfloat16), dev(v, torch.bfloat16), dev(q),
         dev(k), dev(hard), dev(tau)]
    _, norm, state = dism_amd.forward_hard(*t, save_state=True)
    with pytest.raises(RuntimeError, match="sequence hard flags"):
        dism_amd.backward_hard(*t[:3], t[2], *t[3:5],
                               t[5][:, :, None].expand_as(t[3]).contiguous(), norm, state)
