"""Packed batch-1 (varlen) layouts on the MI355X: every document of a packed call must give
exactly what the CPU model gives for that document alone (the reference's own criterion,
dism_v3/tests/test_hard_forward.py:122-148: packed equals fixed per document), soft training
rows give zeros, and documents never see each other.

Layout of the reference fixture (test_hard_forward.py:123-127, test_hard_summary.py:80-93):
offsets [0, 0, 256, 512, 1024, 1024, 2048] (two empty documents), two training rows of 1024
tokens with hard flags [[T, F], [F, T]].
"""
import numpy as np
import pytest
import torch

import oracle
from tests._data import labels, taus, vectors
from tests.test_gpu_parity import assert_bits, dev, host

pytestmark = pytest.mark.gpu

OFFSETS = [0, 0, 256, 512, 1024, 1024, 2048]
HARD = np.array([[True, False], [False, True]])


def _layout(offsets, n):
    import dism_amd
    return dism_amd.VarlenLayout.from_cu_seqlens(torch.tensor(offsets, dtype=torch.int32), n)


def _docs(offsets):
    return [(a, z) for a, z in zip(offsets, offsets[1:]) if z > a]


def _inputs(n, pattern, h=2, r=8, dv=64, seed=0):
    q, k = labels(n, pattern, b=1, h=h, seed=20261014 + seed)
    sq, sk, v = vectors(n, b=1, h=h, r=r, dv=dv, seed=417 + seed)
    rng = np.random.default_rng(99 + seed)
    do = oracle.bf16_round(rng.standard_normal(v.shape))
    return sq, sk, v, do, q, k, taus(h)


def _expected(x, offsets, hard, slots=None):
    """Per-document CPU model results assembled into packed tensors (soft rows as the model
    gives them for a soft row: zeros, lmax 0, argmax -1)."""
    sq, sk, v, do, q, k, tau = x
    n, h = sq.shape[1], sq.shape[2]
    row_n = n // hard.shape[0]
    o = np.zeros(v.shape, np.float32)
    l2 = np.zeros((1, h, n), np.float32)
    lm = np.zeros((1, h, n), np.int32)
    ja = np.full((1, h, n), -1, np.int32)
    g = [np.zeros(sq.shape, np.float32), np.zeros(sk.shape, np.float32),
         np.zeros(v.shape, np.float32)]
    rowtau = np.zeros((1, h, n), np.float32)
    # each head row of the packed call is computed with its own classification (dense rows:
    # the direct definition) for all of its documents
    dense = oracle.packed_dense_flags(q, k, offsets, slots)
    for a, z in _docs(offsets):
        flags = hard[a // row_n:a // row_n + 1]
        lut = oracle.log_weights(tau, z - a)
        dlut = oracle.dlog_weights(tau, z - a)
        args = (sq[:, a:z], sk[:, a:z], v[:, a:z])
        labs = (q[:, :, a:z], k[:, :, a:z])
        od, l2d, lmd, jad = oracle.forward(*args, *labs, flags, lut, dense=dense)
        o[:, a:z], l2[:, :, a:z], lm[:, :, a:z] = od, l2d, lmd
        ja[:, :, a:z] = np.where(jad >= 0, jad + a, -1)
        dsq, dsk, dv, _, rt = oracle.backward(*args, do[:, a:z], *labs, flags, lut, dlut, l2d,
                                              dense=dense)
        g[0][:, a:z], g[1][:, a:z], g[2][:, a:z] = dsq, dsk, dv
        rowtau[:, :, a:z] = rt
    dtau = oracle.tau_reduce(rowtau)
    return o, l2, lm, ja, g, dtau


def _run(x, layout, hard, dtype=torch.bfloat16):
    import dism_amd
    sq, sk, v, do, q, k, tau = x
    t = [dev(a, dtype) for a in (sq, sk, v, do)]
    iq, ik, th, tt = dev(q), dev(k), dev(hard), dev(tau)
    out, lse2, state, m = dism_amd.forward_hard(t[0], t[1], t[2], iq, ik, th, tt, layout=layout,
                                                save_state=True, return_matches=True,
                                                out_dtype=torch.float32)
    grads = dism_amd.backward_hard(t[0], t[1], t[2], t[3], iq, ik, th, lse2, state,
                                   layout=layout)
    return out, lse2, m, grads, state


@pytest.mark.parametrize("pattern", ["random", "equal", "periodic", "boundary", "alphabet4"])
def test_packed_matches_per_document_model(pattern):
    x = _inputs(2048, pattern)
    layout = _layout(OFFSETS, 2048)
    print(f"packed fwd+bwd pattern={pattern} offsets={OFFSETS}", flush=True)
    out, lse2, m, grads, _ = _run(x, layout, HARD)
    o, l2, lm, ja, g, dtau = _expected(x, OFFSETS, HARD)
    assert_bits(host(out), o, "out")
    assert_bits(host(lse2), l2, "lse2")
    assert_bits(host(m["length"]), lm, "lmax")
    assert_bits(host(m["index"]), ja, "argmax")
    for got, want, name in zip(grads[:3], g, ("dsq", "dsk", "dv")):
        assert_bits(host(got), want, name)
    assert_bits(host(grads[3]), dtau, "dtau")


def test_packed_long_documents_all_hard():
    """Documents of 512..4096 tokens with 256 symbols, R=8, DV=64; two training rows."""
    n = 8192
    offsets = [0, 512, 1536, 4096, 4352, 8192]
    hard = np.ones((2, 4), dtype=bool)
    x = _inputs(n, "alphabet256", h=4, seed=3)
    layout = _layout(offsets, n)
    print(f"packed long documents offsets={offsets}", flush=True)
    out, lse2, m, grads, _ = _run(x, layout, hard)
    o, l2, lm, ja, g, dtau = _expected(x, offsets, hard)
    assert_bits(host(out), o, "out")
    assert_bits(host(lse2), l2, "lse2")
    assert_bits(host(m["index"]), ja, "argmax")
    for got, want, name in zip(grads, g + [dtau], ("dsq", "dsk", "dv", "dtau")):
        assert_bits(host(got), want, name)


def test_packed_summaries_and_boundaries():
    import dism_amd
    n = 2048
    layout = _layout(OFFSETS, n)
    for pattern in ("random", "equal", "boundary"):
        q, k = labels(n, pattern, b=1, h=2)
        th = dev(HARD)
        summary = dism_amd.summarize_hard(dev(q), dev(k), th, layout=layout)
        assert summary.shape == (layout.forward_elements * 2,)
        boundary = dism_amd.hard_chunk_scan(summary, layout=layout, heads=2)
        want_s, want_b = [], []
        for a, z in _docs(OFFSETS):
            flags = HARD[a // 1024:a // 1024 + 1]
            want_s.append(oracle.boundary(q[:, :, a:z], k[:, :, a:z], flags,
                                          composed=False).ravel())
            want_b.append(oracle.boundary(q[:, :, a:z], k[:, :, a:z], flags).ravel())
        assert_bits(host(summary), np.concatenate(want_s), f"summary {pattern}")
        assert_bits(host(boundary), np.concatenate(want_b), f"boundary {pattern}")
        inplace = dism_amd.hard_chunk_scan(summary, layout=layout, heads=2, inplace=True)
        assert inplace.data_ptr() == summary.data_ptr()
        assert_bits(host(inplace), np.concatenate(want_b), f"boundary in place {pattern}")
    empty = _layout([0, 0, 0], 0)
    out = dism_amd.hard_chunk_scan(torch.empty(0, dtype=torch.int32, device="cuda"),
                                   layout=empty, heads=2)
    assert out.numel() == 0 and out.dtype == torch.int32


def test_packed_documents_are_independent_and_soft_rows_zero():
    x = list(_inputs(2048, "alphabet4"))
    layout = _layout(OFFSETS, 2048)
    out, lse2, _, grads, _ = _run(x, layout, HARD)
    # changing the values of the first document leaves every other document bit-identical
    x[2] = x[2].copy()
    x[2][:, :256] += 5.0
    out2, lse22, _, _, _ = _run(x, layout, HARD)
    assert torch.equal(out2[:, 256:], out[:, 256:]) and torch.equal(lse22, lse2)
    # NaN vectors on soft rows stay zero (reference test_hard_forward.py:100-120)
    sq, sk, v, do, q, k, tau = _inputs(2048, "random")
    for a in (sq, sk, v):
        a[:, :1024, 1] = np.nan
        a[:, 1024:, 0] = np.nan
    out3, l3, _, g3, _ = _run((sq, sk, v, do, q, k, tau), layout, HARD)
    assert not out3[:, :1024, 1].count_nonzero() and not out3[:, 1024:, 0].count_nonzero()
    assert torch.isfinite(out3).all() and torch.isfinite(l3).all()
    for t in g3:
        assert torch.isfinite(t).all()
    assert not g3[0][:, :1024, 1].count_nonzero() and not g3[2][:, 1024:, 0].count_nonzero()
    # all-soft pack: everything zero
    _, l4, _, g4, _ = _run(x, layout, np.zeros((2, 2), dtype=bool))
    assert not l4.count_nonzero() and all(not t.count_nonzero() for t in g4)


def test_packed_recompute_autograd_and_validation():
    import dism_amd
    x = _inputs(2048, "periodic")
    layout = _layout(OFFSETS, 2048)
    out, lse2, _, grads, _ = _run(x, layout, HARD)
    sq, sk, v, do, q, k, tau = x
    t = [dev(a, torch.bfloat16) for a in (sq, sk, v, do)]
    iq, ik, th, tt = dev(q), dev(k), dev(HARD), dev(tau)
    rec = dism_amd.backward_hard_recompute(*t, iq, ik, th, tt, layout=layout)
    for got, want in zip((rec["sq_vec"], rec["sk_vec"], rec["v"], rec["rtau"]), grads):
        assert torch.equal(got, want)
    _, _, _, grads32, _ = _run(x, layout, HARD, torch.float32)
    leaves = [dev(a_, torch.float32).requires_grad_() for a_ in (sq, sk, v)]
    tau_p = dev(tau).requires_grad_()
    o = dism_amd.dism_core_hard(*leaves, iq, ik, th, tau_p, layout=layout)
    o.backward(dev(do, torch.float32))
    for got, want in zip([l_.grad for l_ in leaves] + [tau_p.grad], grads32):
        assert torch.equal(got, want)
    # reference validation texts
    cross = _layout([0, 512], 512)
    q2, k2 = labels(512, "random", b=1, h=2)
    with pytest.raises(RuntimeError, match="cross a hard training-row"):
        dism_amd.summarize_hard(dev(q2), dev(k2), dev(np.ones((2, 2), dtype=bool)),
                                layout=cross)
    with pytest.raises(RuntimeError, match="evenly divide"):
        dism_amd.forward_hard(*t[:3], iq, ik, dev(np.ones((3, 2), dtype=bool)), tt,
                              layout=layout)
    with pytest.raises(RuntimeError, match="length mismatch"):
        dism_amd.forward_hard(*t[:3], iq, ik, th, tt, layout=_layout([0, 1024], 1024))
    with pytest.raises(RuntimeError, match="packed"):
        dism_amd.hard_chunk_scan(torch.zeros(7, dtype=torch.int32, device="cuda"),
                                 layout=layout, heads=2)
    with pytest.raises(ValueError, match="crosses original hard row"):
        dism_amd.backward_hard_recompute(*t, iq, ik, dev(np.ones((4, 2), dtype=bool)), tt,
                                         layout=_layout([0, 768, 2048], 2048))
