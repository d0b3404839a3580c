"""voc_dism, the reference's vocabulary entry (flash_dism/__init__.py:43-56, voc.py:7-40), on
rows that are all hard: codebook argmax labels of q / k against their vocabularies, then the
hard core.  CPU: argument checks and the operator's fake shapes.  GPU: bit for bit against the
CPU model's exact argmax labels (orc_vocab_labels) and forward / backward (orc_forward /
orc_backward, every row by its own mode), zero gradients for q, k and the vocabularies, and
torch.compile against eager."""
import functools

import numpy as np
import pytest
import torch

import dism_amd
import oracle


def test_voc_checks_and_fake_shapes():
    from torch._subclasses.fake_tensor import FakeTensorMode
    with FakeTensorMode():
        x = torch.empty(2, 256, 3, 32, dtype=torch.bfloat16)
        voc = torch.empty(3, 16, 32, dtype=torch.bfloat16)
        lab = torch.ops.dism_amd.vocab_labels(x, voc)
        assert lab.shape == (2, 3, 256) and lab.dtype == torch.int32
    q = torch.zeros(1, 256, 2, 32, dtype=torch.bfloat16)
    sq = torch.zeros(1, 256, 2, 8, dtype=torch.bfloat16)
    v = torch.zeros(1, 256, 2, 64, dtype=torch.bfloat16)
    voc = torch.zeros(2, 16, 32, dtype=torch.bfloat16)
    hard = torch.ones(1, 2, dtype=torch.bool)
    direction = torch.zeros(1, 2, dtype=torch.uint8)
    with pytest.raises(RuntimeError, match="beta"):
        dism_amd.voc_dism(q, q, sq, sq, v, voc, voc, torch.zeros(2), direction=direction,
                          hard=hard, beta=0.0)


def _inputs(b, n, h, d, r, dv, vsize, seed):
    rng = np.random.default_rng(seed)
    bf = oracle.bf16_round
    q = bf(rng.standard_normal((b, n, h, d)))
    k = bf(rng.standard_normal((b, n, h, d)))
    qv = bf(rng.standard_normal((h, vsize, d)))
    kv = bf(rng.standard_normal((h, vsize, d)))
    sq = bf(rng.standard_normal((b, n, h, r)))
    sk = bf(rng.standard_normal((b, n, h, r)))
    v = bf(rng.standard_normal((b, n, h, dv)))
    do = bf(rng.standard_normal((b, n, h, dv)))
    tau = np.linspace(-0.3, 0.6, h).astype(np.float32)
    return q, k, qv, kv, sq, sk, v, do, tau


def _run(fn, x, dev):
    q, k, qv, kv, sq, sk, v, do, tau = x
    b, _, h, _ = q.shape
    t = lambda a: torch.from_numpy(a).to(dev, torch.bfloat16).requires_grad_()  # noqa: E731
    leaves = [t(a) for a in (q, k, sq, sk, v, qv, kv)]  # the reference's argument order
    rtau = torch.from_numpy(tau).to(dev).requires_grad_()
    hard = torch.ones((b, h), dtype=torch.bool, device=dev)
    direction = torch.zeros((b, h), dtype=torch.uint8, device=dev)
    out = fn(*leaves, rtau, direction=direction, hard=hard)
    out.backward(torch.from_numpy(do).to(dev, torch.bfloat16))
    return out.detach(), [a.grad for a in leaves] + [rtau.grad]


@pytest.mark.gpu
@pytest.mark.parametrize("vsize,d", [(16, 32), (256, 64)])
def test_voc_dism_matches_cpu_model_and_compile(vsize, d):
    dev = torch.device("cuda:0")
    b, n, h, r, dv = 2, 512, 3, 8, 64
    x = _inputs(b, n, h, d, r, dv, vsize, seed=vsize)
    print(f"voc_dism V={vsize} D={d}", flush=True)
    out, grads = _run(dism_amd.voc_dism, x, dev)
    q, k, qv, kv, sq, sk, v, do, tau = x
    lq, lk = oracle.vocab_labels(q, qv), oracle.vocab_labels(k, kv)
    hard = np.ones((b, h), bool)
    lut, dl = oracle.log_weights(tau, n), oracle.dlog_weights(tau, n)
    o, l2, _, _ = oracle.forward(sq, sk, v, lq, lk, hard, lut)
    esq, esk, ev, etau, _ = oracle.backward(sq, sk, v, do, lq, lk, hard, lut, dl, l2)
    bits = lambda a: np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)  # noqa: E731
    host = lambda t: t.float().cpu().numpy()  # noqa: E731
    assert np.array_equal(bits(host(out)), bits(oracle.bf16_round(o))), "out"
    for got, want, name in zip(grads[2:5], (esq, esk, ev), ("dsq", "dsk", "dv")):
        assert np.array_equal(bits(host(got)), bits(oracle.bf16_round(want))), name
    assert np.array_equal(bits(host(grads[7])), bits(etau)), "dtau"
    for gz in grads[:2] + grads[5:7]:  # q, k and the vocabularies: zero gradients
        assert gz is not None and not gz.any()
    compiled = torch.compile(functools.partial(dism_amd.voc_dism, all_hard=True),
                             backend="aot_eager", fullgraph=True)
    out_c, grads_c = _run(compiled, x, dev)
    assert torch.equal(out, out_c)
    for a, c in zip(grads, grads_c):
        assert torch.equal(a, c)
