"""Codebook argmax labels on the MI355X matrix cores against the exact CPU oracle
(oracle.vocab_labels: fp64 scores, first index on ties -- the argmax of
dism_v3/python/flash_dism/reference/dism_v3_ref.py:159-162).  Covers ragged token and vocabulary
counts, per-head and shared tables, D in {32, 64, 128}, exact ties (duplicated codebook rows),
near ties one bf16 ulp apart (the fp64 rescoring path) and subnormal inputs."""
import numpy as np
import pytest
import torch

import oracle
from tests.test_gpu_parity import assert_bits, dev, host

pytestmark = pytest.mark.gpu


def _run(x, vocab):
    import dism_amd
    labels, count = dism_amd.vocab_labels(dev(x, torch.bfloat16), dev(vocab, torch.bfloat16),
                                          return_exact_count=True)
    return host(labels), int(count.item())


@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("shared", [False, True])
def test_vocab_labels_random(d, shared):
    rng = np.random.default_rng(d + shared)
    b, n, h, v = 2, 500, 3, 500
    x = oracle.bf16_round(rng.standard_normal((b, n, h, d)))
    vocab = oracle.bf16_round(rng.standard_normal((v, d) if shared else (h, v, d)))
    print(f"vocab labels d={d} shared={shared}", flush=True)
    got, count = _run(x, vocab)
    assert_bits(got, oracle.vocab_labels(x, vocab), "labels")
    assert count < b * n * h // 20  # almost every token is certified by the fp32 bound


def test_vocab_labels_ties_and_near_ties():
    rng = np.random.default_rng(7)
    b, n, h, d, v = 1, 256, 2, 64, 96
    vocab = oracle.bf16_round(rng.standard_normal((h, v, d)))
    vocab[:, 50] = vocab[:, 10]            # exact duplicate rows: first index must win
    vocab[:, 70] = vocab[:, 20]
    vocab[:, 80] = vocab[:, 30]            # the same row, one bf16 ulp apart in one coordinate
    bits = vocab.view(np.uint32)
    bits[:, 80, 0] += 1 << 16
    x = oracle.bf16_round(rng.standard_normal((b, n, h, d)) * 0.1)
    x[0, :64, :] = vocab[:, 10][None] * 2.0   # tokens pointing at the duplicated rows
    x[0, 64:128, :] = vocab[:, 20][None]
    x[0, 128:192, :] = vocab[:, 30][None]     # near tie between rows 30 and 80
    got, count = _run(x, vocab)
    want = oracle.vocab_labels(x, vocab)
    assert_bits(got, want, "labels")
    assert (want[0, :, :64] == 10).all() and (want[0, :, 64:128] == 20).all()
    assert count >= 128  # exact ties are always rescored


def test_vocab_labels_subnormal_inputs():
    rng = np.random.default_rng(11)
    b, n, h, d, v = 1, 64, 1, 32, 64
    x = oracle.bf16_round(rng.standard_normal((b, n, h, d)))
    x[0, :8, 0, 3] = np.float32(3e-39)        # subnormal in bf16
    vocab = oracle.bf16_round(rng.standard_normal((h, v, d)) * 1e30)
    got, count = _run(x, vocab)
    assert_bits(got, oracle.vocab_labels(x, vocab), "labels")
    assert count >= 8


def test_vocab_labels_nanochat_shape_and_sign_codebook():
    """nanochat-shaped layer (B=2 of 8, T=2048, H=10, D=64, V=512), and the hypercube codebook
    on which the sign binarizer is the argmax (+-1 rows; ties resolved to the first index)."""
    import dism_amd
    rng = np.random.default_rng(3)
    b, n, h, d, v = 2, 2048, 10, 64, 512
    x = oracle.bf16_round(rng.standard_normal((b, n, h, d)) * 0.02)
    vocab = oracle.bf16_round(rng.standard_normal((h, v, d)))
    got, _ = _run(x, vocab)
    assert_bits(got, oracle.vocab_labels(x, vocab), "labels")
    # 8-bit hypercube codebook padded to D=32 with zero columns: argmax == sign labels
    cube = np.array([[2.0 * ((c >> k) & 1) - 1.0 for k in range(8)] + [0.0] * 24
                     for c in range(256)], dtype=np.float32)
    xs = oracle.bf16_round(rng.standard_normal((1, 512, 2, 32)))
    got, _ = _run(xs, cube)
    signs = host(dism_amd.sign_labels(dev(xs[..., :8], torch.bfloat16)))
    assert_bits(got, signs, "hypercube argmax vs sign labels")
