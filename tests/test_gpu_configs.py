"""The HIP path at the shapes of BASELINE.json configs[3] and configs[4] (run on the MI355X).

one long sequence (B=1, H=16, T=65536, d_qk=8, d_v=128, bf16) whose queries copy
earlier key spans (long suffix matches); rows this long take the global-memory prepare path.
the nanochat-shaped layer (B=8, T=2048, H=10, d_qk=8, d_v=128, bf16): q, k, v from
random-init projections of x ~ N(0, 0.02), forward and backward through the autograd core.
Results are compared bit for bit with the CPU model (oracle/dism_cpu_model.c) on the same inputs.
"""
import numpy as np
import pytest
import torch

import oracle
from tests._data import copied_spans

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


def test_config3_long_sequence_copied_spans():
    import dism_amd
    B, T, H, D, DV = 1, 65536, 16, 8, 128
    rng = np.random.default_rng(20261201 + 3)
    q = rng.standard_normal((B, T, H, D), dtype=np.float32)
    k = rng.standard_normal((B, T, H, D), dtype=np.float32)
    assert copied_spans(q, k) >= 0.1 * T
    v = rng.standard_normal((B, T, H, DV), dtype=np.float32)
    sq, sk, vv = (oracle.bf16_round(x) for x in (q, k, v))
    tau = np.linspace(-0.5, 0.5, H).astype(np.float32)
    hard = np.ones((B, H), dtype=bool)
    tq, tk, tv = (dev(x, torch.bfloat16) for x in (sq, sk, vv))
    iq, ik = dism_amd.sign_labels(tq), dism_amd.sign_labels(tk)
    out, lse2, m = dism_amd.forward_hard(tq, tk, tv, iq, ik, dev(hard), dev(tau),
                                         return_matches=True, out_dtype=torch.float32)
    labels_q, labels_k = oracle.sign_labels(sq), oracle.sign_labels(sk)
    assert_bits(host(iq), labels_q, "labels q")
    assert_bits(host(ik), labels_k, "labels k")
    lut = oracle.log_weights(tau, T)
    o, l2, lm, ja = oracle.forward(sq, sk, vv, labels_q, labels_k, hard, lut)
    assert lm.max() >= 256  # the copied spans give long matches
    assert_bits(host(out), o, "out")
    assert_bits(host(lse2), l2, "lse2")
    assert_bits(host(m["length"]), lm, "lmax")
    assert_bits(host(m["index"]), ja, "argmax")


def test_config4_nanochat_layer_fwd_bwd():
    import dism_amd
    B, T, H, D, DV, DM = 8, 2048, 10, 8, 128, 1280
    rng = np.random.default_rng(20261201 + 4)
    x = (rng.standard_normal((B, T, DM), dtype=np.float32) * 0.02)
    wq, wk = (rng.standard_normal((DM, H * D), dtype=np.float32) / np.sqrt(DM) for _ in range(2))
    wv = rng.standard_normal((DM, H * DV), dtype=np.float32) / np.sqrt(DM)
    sq = oracle.bf16_round((x @ wq).reshape(B, T, H, D))
    sk = oracle.bf16_round((x @ wk).reshape(B, T, H, D))
    vv = oracle.bf16_round((x @ wv).reshape(B, T, H, DV))
    dout = oracle.bf16_round(rng.standard_normal((B, T, H, DV), dtype=np.float32))
    tau = np.linspace(-0.5, 0.5, H).astype(np.float32)
    hard = np.ones((B, H), dtype=bool)
    leaves = [dev(a, torch.bfloat16).requires_grad_() for a in (sq, sk, vv)]
    tau_t = dev(tau).requires_grad_()
    iq, ik = dism_amd.sign_labels(leaves[0].detach()), dism_amd.sign_labels(leaves[1].detach())
    out = dism_amd.dism_core_hard(*leaves, iq, ik, dev(hard), tau_t)
    out.backward(dev(dout, torch.bfloat16))

    labels_q, labels_k = oracle.sign_labels(sq), oracle.sign_labels(sk)
    lut = oracle.log_weights(tau, T)
    dl = oracle.dlog_weights(tau, T)
    o, l2, _, _ = oracle.forward(sq, sk, vv, labels_q, labels_k, hard, lut)
    esq, esk, ev, etau, _ = oracle.backward(sq, sk, vv, dout, labels_q, labels_k, hard, lut, dl,
                                            l2)
    assert_bits(host(out), oracle.bf16_round(o), "out (bf16)")
    # autograd hands bf16 leaves their gradients in bf16 (round to nearest even of the fp32)
    assert_bits(host(leaves[0].grad), oracle.bf16_round(esq), "dsq")
    assert_bits(host(leaves[1].grad), oracle.bf16_round(esk), "dsk")
    assert_bits(host(leaves[2].grad), oracle.bf16_round(ev), "dv")
    assert_bits(host(tau_t.grad), etau, "dtau")
