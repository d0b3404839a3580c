"""torch.library registration of the hard core (CPU: fake/meta shapes and argument checks;
GPU: eager vs torch.compile, reference-signature core)."""
import functools

import numpy as np
import pytest
import torch

import dism_amd


def _fake_inputs(b=2, n=512, h=3, r=8, dv=64, dtype=torch.bfloat16):
    sq = torch.empty(b, n, h, r, dtype=dtype)
    v = torch.empty(b, n, h, dv, dtype=dtype)
    lab = torch.empty(b, h, n, dtype=torch.int32)
    return sq, sq.clone(), v, lab, lab.clone(), torch.empty(b, h, dtype=torch.bool), torch.empty(h)


def test_fake_shapes():
    from torch._subclasses.fake_tensor import FakeTensorMode
    from dism_amd import _lib
    with FakeTensorMode():
        sq, sk, v, iq, ik, hard, tau = _fake_inputs()
        out, lse2, lut, ws = torch.ops.dism_amd.hard_core(sq, sk, v, iq, ik, hard, tau)
        assert out.shape == v.shape and out.dtype == torch.bfloat16
        assert lse2.shape == (2, 3, 512) and lse2.dtype == torch.float32
        assert lut.shape == (3, 513)
        assert ws.shape == (_lib.workspace_bytes(2, 512, 3, 8, 64, 0),) and ws.dtype == torch.uint8
        g = torch.ops.dism_amd.hard_core_backward(sq, sk, v, out, iq, ik, hard, tau, lse2, lut, ws)
        assert [t.shape for t in g] == [sq.shape, sk.shape, v.shape, tau.shape]
        assert all(t.dtype == torch.float32 for t in g)


def test_reference_signature_checks_cpu():
    sq, sk, v, iq, ik, _, tau = _fake_inputs(b=1, n=256, h=2)
    sq, sk, v = torch.zeros_like(sq), torch.zeros_like(sk), torch.zeros_like(v)
    q, k = sq.clone(), sk.clone()
    lse = torch.zeros(1, 2, 256)
    hard = torch.ones(1, 2, dtype=torch.bool)
    direction = torch.zeros(1, 2, dtype=torch.uint8)
    with pytest.raises(RuntimeError, match="q_lse/k_lse"):
        dism_amd.dism_core(q, k, sq, sk, v, lse[:, :1], lse, iq, ik, direction, hard, tau)
    with pytest.raises(NotImplementedError, match="soft rows"):
        dism_amd.dism_core(q, k, sq, sk, v, lse, lse, iq, ik, direction, ~hard, tau)
    with pytest.raises(RuntimeError, match="CUDA"):  # the product path never computes on the host
        dism_amd.dism_core(q, k, sq, sk, v, lse, lse, iq, ik, direction, hard, tau)


@pytest.mark.gpu
def test_compiled_matches_eager():
    from tests._data import labels, taus, vectors
    n, b, h = 512, 2, 3
    sq, sk, v = vectors(n, b, h)
    q, k = labels(n, "alphabet4", b, h)
    d = torch.device("cuda")
    dout = torch.from_numpy(np.random.default_rng(5).standard_normal(v.shape).astype(np.float32))
    dout = dout.to(d, torch.bfloat16)
    iq, ik = torch.from_numpy(q).to(d), torch.from_numpy(k).to(d)
    hard = torch.ones((b, h), dtype=torch.bool, device=d)

    def run(fn):
        leaves = [torch.from_numpy(a).to(d, torch.bfloat16).requires_grad_() for a in (sq, sk, v)]
        tau = torch.from_numpy(taus(h)).to(d).requires_grad_()
        qs = leaves[0].detach().clone().requires_grad_()
        lse = torch.zeros((b, h, n), device=d, requires_grad=True)
        direction = torch.zeros((b, h), dtype=torch.uint8, device=d)
        out = fn(qs, leaves[1].detach(), *leaves, lse, lse.detach(), iq, ik, direction, hard, tau)
        out.backward(dout)
        return out.detach(), [t.grad for t in leaves] + [tau.grad, qs.grad, lse.grad]

    eager = run(dism_amd.dism_core)
    compiled = run(torch.compile(functools.partial(dism_amd.dism_core, all_hard=True),
                                 backend="aot_eager", fullgraph=True))
    # without the assertion a compiled caller is refused (the flags cannot be read there)
    with pytest.raises(Exception, match="all_hard=True"):
        run(torch.compile(dism_amd.dism_core, backend="aot_eager", fullgraph=True))
    assert torch.equal(eager[0], compiled[0])
    for a, c in zip(eager[1], compiled[1]):
        assert torch.equal(a, c)
    assert not eager[1][4].any() and not eager[1][5].any()  # soft operands: zero gradients
    # the reference-signature core is the hard core on all-hard rows
    ref = dism_amd.dism_core_hard(*(torch.from_numpy(a).to(d, torch.bfloat16) for a in (sq, sk, v)),
                                  iq, ik, hard, torch.from_numpy(taus(h)).to(d))
    assert torch.equal(ref, eager[0])
    # an explicit planner object (the reference's hybrid route) gives the same result
    planned = run(functools.partial(dism_amd.dism_core, hard_planner=object()))
    assert torch.equal(planned[0], eager[0])


@pytest.mark.gpu
def test_forward_backward_graph_replay():
    """forward_hard + backward_hard (whose key chain forks onto the library's side stream)
    captured in a HIP graph: every replay, with eager work and synchronisations in between,
    equals the eager results bit for bit (reference test_hard_forward.py:160-172 replays its
    readout the same way)."""
    import numpy as np
    import torch
    import dism_amd
    from tests._data import labels, taus, vectors
    b, n, h = 2, 1024, 4
    q, k = labels(n, "alphabet4", b=b, h=h)
    sq, sk, v = vectors(n, b=b, h=h)
    do = np.random.default_rng(1).standard_normal(v.shape).astype(np.float32)
    dev = lambda a, dt=None: torch.from_numpy(np.ascontiguousarray(a)).cuda().to(  # noqa
        dt or torch.from_numpy(np.ascontiguousarray(a)).dtype)
    tq, tk, tv, tdo = (dev(a, torch.bfloat16) for a in (sq, sk, v, do))
    iq, ik = dev(q), dev(k)
    hard, tau = dev(np.ones((b, h), bool)), dev(taus(h))

    def run():
        out, lse2, state = dism_amd.forward_hard(tq, tk, tv, iq, ik, hard, tau, save_state=True)
        return (out, lse2) + tuple(dism_amd.backward_hard(tq, tk, tv, tdo, iq, ik, hard, lse2,
                                                          state))

    eager = [t.clone() for t in run()]  # also creates the side stream outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = run()
    for i in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for got, want in zip(captured, eager):
            assert torch.equal(got, want), i
        run()  # eager work between replays
        torch.cuda.synchronize()


def test_hybrid_core_checks_cpu():
    """dism_core_hybrid (the reference's _MixedCore with a caller-supplied soft core):
    argument checks before anything runs on a device; an empty hard side returns the soft
    output alone."""
    sq, sk, v, iq, ik, hard, tau = _fake_inputs(b=1, n=256, h=2)
    q, k = torch.zeros_like(sq), torch.zeros_like(sk)
    lse = torch.zeros(1, 2, 256)
    direction = torch.zeros(1, 2, dtype=torch.uint8)
    with pytest.raises(TypeError, match="soft_core"):
        dism_amd.dism_core_hybrid(q, k, sq, sk, v, lse, lse, iq, ik, direction, hard, tau,
                                  soft_core=None)
    with pytest.raises(ValueError, match="ctas"):
        dism_amd.dism_core_hybrid(q, k, sq, sk, v, lse, lse, iq, ik, direction, hard, tau,
                                  soft_core=lambda *a, **kw: None, layout=object(), ctas=4)
    soft = torch.ones(1, 256, 2, 64)
    empty = sq[:, :0]
    got = dism_amd.dism_core_hybrid(q, k, empty, empty, v[:, :0], lse, lse, iq, ik, direction,
                                    hard, tau, soft_core=lambda *a, **kw: soft)
    assert got is soft


@pytest.mark.gpu
def test_hybrid_core_sums_soft_and_hard():
    """O = soft + hard, gradients the sum of both parts' (hard rows mixed with soft rows: the
    hard core is zero on soft rows, the toy soft core zero on hard rows)."""
    from tests._data import labels, taus, vectors
    n, b, h = 512, 2, 3
    sq, sk, v = vectors(n, b, h)
    ql, kl = labels(n, "random", b, h)
    d = torch.device("cuda")
    iq, ik = torch.from_numpy(ql).to(d), torch.from_numpy(kl).to(d)
    hard = torch.tensor([[True, False, True], [False, True, True]], device=d)
    leaves = [torch.from_numpy(a).to(d, torch.bfloat16).requires_grad_() for a in (sq, sk, v)]
    tau = torch.from_numpy(taus(h)).to(d).requires_grad_()
    lse = torch.zeros((b, h, n), device=d)
    direction = torch.zeros((b, h), dtype=torch.uint8, device=d)
    soft_mask = (~hard).float().view(b, 1, h, 1)

    def soft_core(q, k, sq_, sk_, v_, lq, lk, iq_, ik_, dirn, hard_, tau_, **kw):
        return (v_.float() * 0.5 + sq_.float().sum(-1, keepdim=True)) * soft_mask

    out = dism_amd.dism_core_hybrid(leaves[0], leaves[1], *leaves, lse, lse, iq, ik, direction,
                                    hard, tau, soft_core=soft_core)
    dout = torch.randn(out.shape, device=d, generator=torch.Generator(d).manual_seed(3))
    out.backward(dout)
    got = [t.grad.clone() for t in leaves] + [tau.grad.clone()]
    for t in leaves + [tau]:
        t.grad = None
    hard_out = dism_amd.dism_core_hard(*leaves, iq, ik, hard, tau)
    soft_out = soft_core(None, None, *leaves, lse, lse, iq, ik, direction, hard, tau)
    torch.testing.assert_close(out, soft_out + hard_out.float(), rtol=0, atol=0)
    (soft_out + hard_out.float()).backward(dout)
    for a, c in zip(got, [t.grad for t in leaves] + [tau.grad]):
        torch.testing.assert_close(a, c, rtol=0, atol=0)
