"""dism_hard_forward (prepare + readout in one call, the bigram half of the prepare on a side
stream overlapping the length-1 label scan) against the two-call sequence dism_hard_prepare ->
dism_hard_readout and against the CPU model, bit for bit.  One batch mixes every kind of row
the fused call must split between its two scan phases: one-byte labels in the low byte and in a
higher byte (prepared in LDS, pair counts from the scan's own predecessor histogram),
multi-byte labels (global-memory prepare, pair counts from the plan), constant rows and soft
rows; then rows longer than the LDS prepare takes, and a composed carry boundary."""
import numpy as np
import pytest
import torch

import oracle
from tests._data import flags, taus, vectors
from tests.test_gpu_parity import assert_bits, dev, host

pytestmark = pytest.mark.gpu


def _mixed_labels(n, b=2, h=4, seed=5):
    rng = np.random.default_rng(seed)
    q = np.empty((b, h, n), dtype=np.int32)
    k = np.empty_like(q)
    per = np.arange(n, dtype=np.int32)
    kinds = ["byte0", "byte2", "multi", "const", "period", "alpha4", "multi_rep", "byte1"]
    for r in range(b * h):
        kind = kinds[r % len(kinds)]
        bi, hi = divmod(r, h)
        if kind == "byte0":
            q[bi, hi] = rng.integers(0, 256, n)
            k[bi, hi] = rng.integers(0, 256, n)
        elif kind == "byte2":  # one byte, but not the low one
            q[bi, hi] = rng.integers(0, 8, n) << 16
            k[bi, hi] = rng.integers(0, 8, n) << 16
        elif kind == "multi":  # two label bytes: the global-memory prepare
            q[bi, hi] = rng.integers(0, 3, n) * 257
            k[bi, hi] = rng.integers(0, 3, n) * 257
        elif kind == "const":
            q[bi, hi] = 5
            k[bi, hi] = 5
        elif kind == "period":
            q[bi, hi] = per % 7
            k[bi, hi] = (per + 2) % 7
        elif kind == "alpha4":
            q[bi, hi] = rng.integers(0, 4, n)
            k[bi, hi] = rng.integers(0, 4, n)
        elif kind == "multi_rep":  # repeats with negative (all-byte) labels
            base = rng.integers(-2, 2, 64).astype(np.int32)
            q[bi, hi] = np.resize(base, n)
            k[bi, hi] = np.resize(base, n)
        else:
            q[bi, hi] = (rng.integers(0, 4, n) << 8)
            k[bi, hi] = (rng.integers(0, 4, n) << 8)
    return q, k


def _fused_and_staged(sq, sk, v, q, k, hard, tau, carry=0):
    import dism_amd
    from dism_amd import hard_forward as hf
    x = [dev(sq, torch.bfloat16), dev(sk, torch.bfloat16), dev(v, torch.bfloat16), dev(q),
         dev(k), dev(hard), dev(tau)]
    fused = dism_amd.forward_hard(*x, carry_strip=carry, return_matches=True,
                                  out_dtype=torch.float32)
    n = q.shape[-1]
    lut = dism_amd.hard_log_weights(x[6], n)
    boundary = dism_amd.hard_boundary(x[3], x[4], x[5], strip=carry, fill_all=False) \
        if carry else None
    ws = hf.prepare_workspace(*x[:5])
    o, l2, lm, ja, _ = hf._readout(*x[:6], boundary, carry, lut, torch.float32, True,
                                   workspace=ws)
    return fused, (o, l2, lm, ja)


@pytest.mark.parametrize("n,carry", [(1024, 0), (4096, 0), (4096, 256), (20480, 0)])
def test_fused_forward_mixed_rows(n, carry):
    print(f"fused forward mixed rows n={n} carry={carry}", flush=True)
    q, k = _mixed_labels(n)
    b, h = q.shape[:2]
    sq, sk, v = vectors(n, b, h, 8, 64)
    hard = flags(b, h)
    tau = taus(h)
    (out, lse2, m), (o, l2, lm, ja) = _fused_and_staged(sq, sk, v, q, k, hard, tau, carry)
    assert_bits(host(out), host(o), "out (fused vs staged)")
    assert_bits(host(lse2), host(l2), "lse2 (fused vs staged)")
    assert_bits(host(m["length"]), host(lm), "lmax (fused vs staged)")
    assert_bits(host(m["index"]), host(ja), "argmax (fused vs staged)")
    if n <= 4096:  # the CPU model at sizes it finishes in seconds
        lut = oracle.log_weights(tau, n)
        eo, el2, elm, eja = oracle.forward(sq, sk, v, q, k, hard, lut)
        assert_bits(host(out), eo, "out")
        assert_bits(host(lse2), el2, "lse2")
        assert_bits(host(m["length"]), elm, "lmax")
        assert_bits(host(m["index"]), eja, "argmax")


def test_fused_forward_then_backward_and_repeat():
    """The workspace the fused call leaves serves the backward, and repeated fused calls on
    one stream (side stream and events reused) give identical results."""
    import dism_amd
    n = 2048
    q, k = _mixed_labels(n, seed=9)
    b, h = q.shape[:2]
    sq, sk, v = vectors(n, b, h, 8, 64)
    hard, tau = flags(b, h), taus(h)
    x = [dev(sq, torch.bfloat16), dev(sk, torch.bfloat16), dev(v, torch.bfloat16), dev(q),
         dev(k), dev(hard), dev(tau)]
    first = dism_amd.forward_hard(*x, out_dtype=torch.float32)
    for _ in range(3):
        again = dism_amd.forward_hard(*x, out_dtype=torch.float32)
        assert torch.equal(first[0], again[0]) and torch.equal(first[1], again[1])
    rng = np.random.default_rng(1)
    dout = oracle.bf16_round(rng.standard_normal(v.shape))
    leaves = [t.clone().requires_grad_(True) for t in x[:3]]
    taut = x[6].clone().requires_grad_(True)
    y = dism_amd.dism_core_hard(*leaves, x[3], x[4], x[5], taut)
    y.backward(dev(dout, torch.bfloat16))
    lut = oracle.log_weights(tau, n)
    dl = oracle.dlog_weights(tau, n)
    eo, el2, _, _ = oracle.forward(sq, sk, v, q, k, hard, lut)
    esq, esk, ev, etau, _ = oracle.backward(sq, sk, v, dout, q, k, hard, lut, dl, el2)
    assert_bits(host(y), oracle.bf16_round(eo), "out (bf16)")
    assert_bits(host(leaves[0].grad), oracle.bf16_round(esq), "dsq")
    assert_bits(host(leaves[1].grad), oracle.bf16_round(esk), "dsk")
    assert_bits(host(leaves[2].grad), oracle.bf16_round(ev), "dv")
    assert_bits(host(taut.grad), etau, "dtau")
