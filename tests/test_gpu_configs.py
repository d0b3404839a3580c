"""The HIP path at the shapes of BASELINE.json configs[1..4] (run on the MI355X).

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


def test_config1_low_entropy_fwd_bwd_and_fp64():
    """B=2, H=8, T=2048, d_qk=2 (alphabet 4, long matches), v bf16 N(0,1) d_v=64,
    fp32 q/k, a bf16 N(0,1) upstream gradient; fwd+bwd bit-exact to the CPU model and within the
    north-star gradient bound (max relative error 1e-3) of the FP64 dense oracle."""
    import dism_amd
    from oracle import dense
    B, T, H, D, DV = 2, 2048, 8, 2, 64
    rng = np.random.default_rng(20261201 + 1)
    q = rng.standard_normal((B, T, H, D), dtype=np.float32)
    k = rng.standard_normal((B, T, H, D), dtype=np.float32)
    vv = oracle.bf16_round(rng.standard_normal((B, T, H, DV), dtype=np.float32))
    dout = oracle.bf16_round(rng.standard_normal((B, T, H, DV), dtype=np.float32))
    tau = np.linspace(-0.5, 0.5, H).astype(np.float32)
    hard = np.ones((B, H), dtype=bool)
    tq, tk = dev(q), dev(k)
    tv, tdo = dev(vv), dev(dout)
    iq, ik = dism_amd.sign_labels(tq), dism_amd.sign_labels(tk)
    out, lse2, state, m = dism_amd.forward_hard(tq, tk, tv, iq, ik, dev(hard), dev(tau),
                                                save_state=True, return_matches=True)
    grads = dism_amd.backward_hard(tq, tk, tv, tdo, iq, ik, dev(hard), lse2, state)
    lq, lk = oracle.sign_labels(q), oracle.sign_labels(k)
    assert lq.max() <= 3
    lut, dl = oracle.log_weights(tau, T), oracle.dlog_weights(tau, T)
    o, l2, lm, ja = oracle.forward(q, k, vv, lq, lk, hard, lut)
    assert lm.max() >= 8
    assert_bits(host(out), o, "out")
    assert_bits(host(lse2), l2, "lse2")
    assert_bits(host(m["length"]), lm, "lmax")
    assert_bits(host(m["index"]), ja, "argmax")
    ref = oracle.backward(q, k, vv, dout, lq, lk, hard, lut, dl, l2)
    for got, want, name in zip(grads, ref[:4], ("dsq", "dsk", "dv", "dtau")):
        assert_bits(host(got), want, name)
    # FP64 dense oracle on two (b,h) rows of the first batch (O(T^2) each)
    sl = (slice(0, 1), slice(None), slice(0, 2))
    lsl = (slice(0, 1), slice(0, 2))
    args = (q[sl], k[sl], vv[sl])
    od, _ = dense.dense_forward(*args, lq[lsl], lk[lsl], hard[lsl], tau[:2])
    np.testing.assert_allclose(host(out)[sl], od, atol=1e-5, rtol=1e-4)
    dsq, dsk, dvd, _ = dense.dense_backward(*args, dout[sl], lq[lsl], lk[lsl], hard[lsl],
                                            tau[:2])
    for got, want, name in zip(grads[:3], (dsq, dsk, dvd), ("dsq", "dsk", "dv")):
        err = np.abs(host(got)[sl] - want).max() / max(np.abs(want).max(), 1e-30)
        assert err < 1e-3, (name, err)


def test_config2_headline_fwd_bwd_full_size():
    """configs[2], the headline workload at full size (B=4, H=16, T=16384, d_qk=8, d_v=64,
    bf16, period-97 component on heads h % 4 == 0 -- the bench's own generator and seed):
    every output, index, normalizer and gradient bit-exact to the CPU model."""
    import dism_amd
    from bench import make_inputs
    B, T, H, D, DV = 4, 16384, 16, 8, 64
    q, k, v, do = make_inputs(B, T, H, D, DV, seed=20261203)
    sq, sk, vv, dout = (oracle.bf16_round(x) for x in (q, k, v, do))
    tau = np.full(H, 0.5, dtype=np.float32)
    hard = np.ones((B, H), dtype=bool)
    tq, tk, tv, tdo = (dev(x, torch.bfloat16) for x in (sq, sk, vv, dout))
    iq, ik = dism_amd.sign_labels(tq), dism_amd.sign_labels(tk)
    out, lse2, m = dism_amd.forward_hard(tq, tk, tv, iq, ik, dev(hard), dev(tau),
                                         return_matches=True, out_dtype=torch.float32)
    state = dict(log_weights=dism_amd.hard_log_weights(dev(tau), T), tau=dev(tau))
    grads = dism_amd.backward_hard(tq, tk, tv, tdo, iq, ik, dev(hard), lse2, state)
    lq, lk = oracle.sign_labels(sq), oracle.sign_labels(sk)
    assert_bits(host(iq), lq, "labels q")
    lut, dl = oracle.log_weights(tau, T), oracle.dlog_weights(tau, T)
    o, l2, lm, ja = oracle.forward(sq, sk, vv, lq, lk, hard, lut, threads=16)
    assert_bits(host(out), o, "out")
    assert_bits(host(lse2), l2, "lse2")
    assert_bits(host(m["length"]), lm, "lmax")
    assert_bits(host(m["index"]), ja, "argmax")
    ref = oracle.backward(sq, sk, vv, dout, lq, lk, hard, lut, dl, l2, threads=16)
    for got, want, name in zip(grads, ref[:4], ("dsq", "dsk", "dv", "dtau")):
        assert_bits(host(got), want, name)
