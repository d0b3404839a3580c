"""bench.py's algorithmic counts (the roofline's work figures) against brute force."""
import numpy as np

from bench import bigram_pair_counts, causal_counts, valid_pairs


def test_causal_counts_brute_force():
    rng = np.random.default_rng(5)
    for alphabet in (1, 2, 4, 9):
        q = rng.integers(0, alphabet, 61)
        k = rng.integers(0, alphabet, 61)
        qn, kn = causal_counts(q, k)
        assert qn.tolist() == [int(sum(k[j] == q[i] for j in range(i + 1))) for i in range(61)]
        assert kn.tolist() == [int(sum(q[i] == k[j] for i in range(j, 61))) for j in range(61)]


def test_bigram_pairs_and_owners_brute_force():
    rng = np.random.default_rng(6)
    for alphabet in (2, 3, 256):
        iq = rng.integers(0, alphabet, (2, 2, 45)).astype(np.int32)
        ik = rng.integers(0, alphabet, (2, 2, 45)).astype(np.int32)
        iq[1, 1] = 7    # one all-equal row: every pair with j >= 1 is a bigram pair
        ik[1, 1] = 7
        want = [0, 0, 0]
        for b in range(2):
            for h in range(2):
                a, c = iq[b, h], ik[b, h]
                m = np.array([[1 <= j <= i and a[i] == c[j] and a[i - 1] == c[j - 1]
                               for j in range(45)] for i in range(45)])
                want[0] += int(m.sum())
                want[1] += int(m.any(1).sum())
                want[2] += int(m.any(0).sum())
        assert list(bigram_pair_counts(iq, ik)) == want


def test_valid_pairs_brute_force():
    rng = np.random.default_rng(7)
    iq = rng.integers(0, 3, (1, 3, 33)).astype(np.int32)
    ik = rng.integers(0, 3, (1, 3, 33)).astype(np.int32)
    want = [sum(int(ik[0, r, j] == iq[0, r, i]) for i in range(33) for j in range(i + 1))
            for r in range(3)]
    assert valid_pairs(iq, ik).tolist() == want
