"""Inference on the MI355X: prefill (with query resets, any length) and the incremental decoder
against the CPU model (oracle.forward, with resets: orc_forward_reset) bit for bit, against
the FP64 dense restatement of the reference's inference oracle
(dism_v3/tests/test_sam_inference.py:9-29), and against each other and the training forward.

Prefill is the training forward, so rows the classifier marks dense use the direct definition;
the decoder always computes the decomposed one (it cannot classify a row before its end), so
its reference is the CPU model with dense=0.  On sparse rows the two are the same bits; on
dense rows they agree to fp32 association.

Inputs follow the reference's SAM tests (test_sam_inference.py:32-45): B=2, H=2, N=79,
R=16, DV=32, alphabet 4, patterns random / repeat (all labels 0) / mismatch (q 0, k 1),
tau [0, .35], vectors N(0,1)*.2 in bf16.
"""
import numpy as np
import pytest
import torch

import oracle
from oracle import dense
from tests.test_gpu_parity import assert_bits, dev, host

pytestmark = pytest.mark.gpu

TAU = np.array([0.0, 0.35], dtype=np.float32)


def sam_inputs(pattern, b=2, h=2, n=79, r=16, dv=32, alphabet=4, seed=83):
    rng = np.random.default_rng(seed)
    iq = rng.integers(0, alphabet, (b, h, n)).astype(np.int32)
    ik = rng.integers(0, alphabet, (b, h, n)).astype(np.int32)
    if pattern == "repeat":
        iq[:] = 0
        ik[:] = 0
    elif pattern == "mismatch":
        iq[:] = 0
        ik[:] = 1
    sq, sk, v = (oracle.bf16_round(rng.standard_normal((b, n, h, c)) * 0.2) for c in (r, r, dv))
    return iq, ik, sq, sk, v


def cpu_model(iq, ik, sq, sk, v, tau, reset=None, dense=None):
    b, h, n = iq.shape
    lut = oracle.log_weights(tau, n)
    out, lse2, _, _ = oracle.forward(sq, sk, v, iq, ik, np.ones((b, h), bool), lut,
                                     reset=reset, dense=dense)
    return out, lse2


def to_dev(iq, ik, sq, sk, v, dtype=torch.bfloat16):
    return dev(iq), dev(ik), dev(sq, dtype), dev(sk, dtype), dev(v, dtype)


@pytest.mark.parametrize("pattern", ["random", "repeat", "mismatch"])
def test_prefill_matches_cpu_model_and_fp64(pattern):
    from dism_amd.inference import HardDismPrefill
    x = sam_inputs(pattern)
    print(f"prefill pattern={pattern}", flush=True)
    with HardDismPrefill(workers=4) as engine:
        out = engine(*to_dev(*x), list(TAU))
    want, _ = cpu_model(*x, TAU)
    assert out.shape == (2, 79, 2, 32) and out.dtype == torch.float32
    assert_bits(host(out), want, "prefill")
    ref, _ = dense.dense_forward(*x[2:], *x[:2], np.ones((2, 2), bool), TAU)
    np.testing.assert_allclose(host(out), ref, atol=2e-6, rtol=2e-4)


def test_prefill_and_decode_with_query_resets():
    from dism_amd.inference import HardDismDecoder, HardDismPrefill
    x = sam_inputs("repeat")
    reset = np.zeros((2, 2, 79), dtype=bool)
    reset[..., 17::19] = True
    want, _ = cpu_model(*x, TAU, reset)
    ref, _ = dense.dense_forward(*x[2:], *x[:2], np.ones((2, 2), bool), TAU, reset=reset)
    np.testing.assert_allclose(want, ref, atol=2e-6, rtol=2e-4)
    with HardDismPrefill(mma_precision="tf32x3") as engine:
        out = engine(*to_dev(*x), TAU, reset=dev(reset))
    assert_bits(host(out), want, "prefill with resets")
    decoder = HardDismDecoder(2, 2, 16, 32, 79, list(TAU), planner_backend="gpu")
    got = decoder.append(*to_dev(*x), reset=dev(reset))
    want_dec, _ = cpu_model(*x, TAU, reset, dense=0)
    assert_bits(host(got), want_dec, "decode with resets")
    np.testing.assert_allclose(host(got), host(out), atol=1e-6, rtol=1e-5)


@pytest.mark.parametrize("pattern", ["random", "repeat", "mismatch"])
@pytest.mark.parametrize("prime", [False, True])
def test_decode_matches_prefill_bit_for_bit(pattern, prime):
    from dism_amd.inference import HardDismDecoder
    x = sam_inputs(pattern)
    want, _ = cpu_model(*x, TAU, dense=0)
    iq, ik, sq, sk, v = to_dev(*x)
    decoder = HardDismDecoder(2, 2, 16, 32, 79, torch.tensor(TAU), label_slots=64)
    start = 31 if prime else 0
    print(f"decode pattern={pattern} prime={prime}", flush=True)
    if prime:
        decoder.prime(iq[..., :start], ik[..., :start], sk[:, :start], v[:, :start])
    outs, t = [], start
    for step in (1, 5, 1, 11):  # mixed chunk sizes, then the rest
        outs.append(decoder.append(iq[..., t:t + step], ik[..., t:t + step], sq[:, t:t + step],
                                   sk[:, t:t + step], v[:, t:t + step]))
        t += step
    outs.append(decoder.append(iq[..., t:], ik[..., t:], sq[:, t:], sk[:, t:], v[:, t:]))
    got = torch.cat(outs, dim=1)
    assert decoder.position == 79
    assert_bits(host(got), want[:, start:], "decode")


def test_decode_equals_training_forward_long():
    """1024 tokens per row, 256 symbols and periodic rows, R=8, DV=64: the decoder's tokens
    equal the training forward's fp32 output (one GPU path against the other)."""
    import dism_amd
    from dism_amd.inference import HardDismDecoder
    b, h, n, r, dv = 2, 4, 1024, 8, 64
    rng = np.random.default_rng(5)
    iq = rng.integers(0, 256, (b, h, n)).astype(np.int32)
    ik = rng.integers(0, 256, (b, h, n)).astype(np.int32)
    iq[:, 1] = np.arange(n) % 13          # long repeats on one head
    ik[:, 1] = (np.arange(n) + 4) % 13
    sq, sk, v = (oracle.bf16_round(rng.standard_normal((b, n, h, c))) for c in (r, r, dv))
    tau = np.array([0.5, 0.1, 0.0, 1.0], dtype=np.float32)
    t_iq, t_ik, t_sq, t_sk, t_v = to_dev(iq, ik, sq, sk, v)
    out, _ = dism_amd.forward_hard(t_sq, t_sk, t_v, t_iq, t_ik, dev(np.ones((b, h), bool)),
                                   dev(tau), out_dtype=torch.float32)
    decoder = HardDismDecoder(b, h, r, dv, n, list(tau), label_slots=512)
    decoder.prime(t_iq[..., :300], t_ik[..., :300], t_sk[:, :300], t_v[:, :300])
    pieces = []
    for t0 in range(300, n, 181):
        t1 = min(n, t0 + 181)
        pieces.append(decoder.append(t_iq[..., t0:t1], t_ik[..., t0:t1], t_sq[:, t0:t1],
                                     t_sk[:, t0:t1], t_v[:, t0:t1]))
    got = torch.cat(pieces, dim=1)
    # head 1 (period 13) is a dense row: the training forward takes the direct definition
    dense = oracle.dense_rows(iq, ik, np.ones((b, h), bool))
    assert dense[:, 1].all() and not dense[:, [0, 2, 3]].any()
    sparse_heads = [0, 2, 3]
    assert torch.equal(got[:, :, sparse_heads], out[:, 300:, sparse_heads])
    np.testing.assert_allclose(host(got[:, :, 1]), host(out[:, 300:, 1]), atol=1e-5, rtol=1e-4)
    want, _ = cpu_model(iq, ik, sq, sk, v, tau, dense=0)
    assert_bits(host(got), want[:, 300:], "decode vs CPU model")
    stats = decoder.memory_stats()
    assert stats["position"] == n and stats["list_blocks_used"] > 0


def test_decoder_validation_and_overflow():
    from dism_amd.inference import HardDismDecoder, HardDismPrefill
    x = sam_inputs("random")
    iq, ik, sq, sk, v = to_dev(*x)
    with pytest.raises(ValueError, match="one fixed tau per head"):
        HardDismDecoder(2, 2, 16, 32, 79, [0.0])
    with pytest.raises(ValueError, match="planner_backend"):
        HardDismDecoder(2, 2, 16, 32, 79, list(TAU), planner_backend="tpu")
    with pytest.raises(ValueError, match="nonnegative"):
        HardDismDecoder(2, 2, 16, 32, 79, [0.0, -1.0])
    decoder = HardDismDecoder(2, 2, 16, 32, 40, list(TAU))
    with pytest.raises(ValueError, match="capacity exceeded"):
        decoder.append(iq, ik, sq, sk, v)
    decoder.prime(iq[..., :8], ik[..., :8], sk[:, :8], v[:, :8])
    with pytest.raises(ValueError, match="prime requires empty cache"):
        decoder.prime(iq[..., :8], ik[..., :8], sk[:, :8], v[:, :8])
    with pytest.raises(ValueError, match="labels must be int32"):
        decoder.append(iq[..., 8:9].long(), ik[..., 8:9], sq[:, 8:9], sk[:, 8:9], v[:, 8:9])
    with pytest.raises(ValueError, match="sq must match sk"):
        decoder.append(iq[..., 8:9], ik[..., 8:9], sq[:, 8:9].float(), sk[:, 8:9].float(),
                       v[:, 8:9].float())
    # more distinct key labels than the table holds -> reported, not silently wrong
    many = HardDismDecoder(1, 1, 16, 32, 200, [0.5], label_slots=64)
    labels = torch.arange(200, dtype=torch.int32, device="cuda").view(1, 1, 200)
    vec = lambda c: torch.zeros((1, 200, 1, c), dtype=torch.bfloat16, device="cuda")  # noqa
    with pytest.raises(RuntimeError, match="label table overflow"):
        many.append(labels, labels, vec(16), vec(16), vec(32))
    with HardDismPrefill() as engine:
        with pytest.raises(ValueError, match="labels must be int32"):
            engine(iq.long(), ik, sq, sk, v, TAU)
    with pytest.raises(ValueError, match="chunk_size"):
        HardDismPrefill(chunk_size=7)


@pytest.mark.parametrize("pattern", ["random", "repeat", "wide"])
def test_parallel_prime_equals_serial_prime(pattern):
    """The parallel prime (label order -> per-label running matrices and key lists) decodes
    exactly like the token-by-token key steps: odd prompt length, a query reset inside the
    prompt, labels spanning the int32 range ('wide', where padding label 0 is also real)."""
    from dism_amd.inference import HardDismDecoder
    b, h, n, r, dv, start = 2, 3, 700, 8, 64, 333
    rng = np.random.default_rng(21)
    if pattern == "wide":
        pool = np.array([np.iinfo(np.int32).min, -7, 0, 5, np.iinfo(np.int32).max], np.int32)
        iq, ik = (pool[rng.integers(0, 5, (b, h, n))] for _ in range(2))
    else:
        iq, ik, *_ = sam_inputs(pattern, b=b, h=h, n=n, alphabet=16)
    sq, sk, v = (oracle.bf16_round(rng.standard_normal((b, n, h, c)) * 0.3) for c in (r, r, dv))
    reset = np.zeros((b, h, n), dtype=bool)
    reset[..., 100] = True
    tau = np.array([0.5, 0.0, 1.5], dtype=np.float32)
    want, _ = cpu_model(iq, ik, sq, sk, v, tau, reset, dense=0)
    t = to_dev(iq, ik, sq, sk, v)
    rs = dev(reset)
    outs = []
    for serial in (False, True):
        dec = HardDismDecoder(b, h, r, dv, n, list(tau), label_slots=64)
        dec.prime(t[0][..., :start], t[1][..., :start], t[3][:, :start], t[4][:, :start],
                  reset=rs[..., :start], serial=serial)
        outs.append(dec.append(t[0][..., start:], t[1][..., start:], t[2][:, start:],
                               t[3][:, start:], t[4][:, start:], reset=rs[..., start:]))
    assert torch.equal(outs[0], outs[1])
    assert_bits(host(outs[0]), want[:, start:], "decode after parallel prime")
