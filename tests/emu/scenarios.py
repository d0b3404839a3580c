"""Scenarios run against the CPU-emulated library (tests/emu/build.py): each feeds the
C ABI with seeded inputs and compares with the CPU model (oracle/) bit for bit.  Run as
``python tests/emu/scenarios.py NAME...`` with DISM_EMU_LIB set (build.asan_env); prints
``OK NAME`` per scenario.  Test infrastructure only."""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import drv  # noqa: E402
import oracle  # noqa: E402


def same_bits(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def _inputs(B, N, H, R, DV, seed, labels=None):
    rng = np.random.default_rng(seed)
    q = oracle.bf16_round(rng.standard_normal((B, N, H, R)))
    k = oracle.bf16_round(rng.standard_normal((B, N, H, R)))
    v = oracle.bf16_round(rng.standard_normal((B, N, H, DV)))
    do = oracle.bf16_round(rng.standard_normal((B, N, H, DV)))
    if labels is None:
        iq, ik = oracle.sign_labels(q), oracle.sign_labels(k)
    else:
        iq, ik = labels(rng)
    return q, k, v, do, iq, ik


def check_fwd_bwd(q, k, v, do, iq, ik, tau, fused=True):
    B, N, H, _ = q.shape
    hard = np.ones((B, H), bool)
    lut = oracle.log_weights(tau, N)
    fwd = drv.forward if fused else drv.staged
    out, l2, lm, ja, st = fwd(q, k, v, iq, ik, hard, lut)
    o, l2o, lmo, jao = oracle.forward(q, k, v, iq, ik, hard, lut)
    assert same_bits(out, o), "forward output"
    assert same_bits(l2, l2o), "normalizer"
    assert np.array_equal(lm, lmo) and np.array_equal(ja, jao), "match lengths / argmax"
    dl = oracle.dlog_weights(tau, N)
    got = drv.backward(st, do, dl, l2)
    ref = oracle.backward(q, k, v, do, iq, ik, hard, lut, dl, l2o)
    for g, r, name in zip(got, ref, ("dsq", "dsk", "dv", "dtau", "rowtau")):
        assert same_bits(g, r), name


def fused_fwd_bwd():
    """one-call forward (side-stream halves serialised) + backward, random 256-symbol rows"""
    x = _inputs(1, 256, 2, 8, 64, 20261201)
    check_fwd_bwd(*x, np.linspace(-0.5, 0.5, 2).astype(np.float32))


def staged_fwd_bwd():
    """prepare + readout, then the backward on the prepared workspace"""
    x = _inputs(1, 256, 2, 8, 64, 7)
    check_fwd_bwd(*x, np.array([0.3, -0.2], np.float32), fused=False)


def mixed_modes():
    """rows of every mode in one call: sparse, identical labels (prefix row), a period of
    distinct labels (prefix row), alphabet 4 (level row), 3 labels in blocks (dense)"""
    N = 256

    def labels(rng):
        iq = rng.integers(0, 256, (1, 5, N)).astype(np.int32)
        ik = rng.integers(0, 256, (1, 5, N)).astype(np.int32)
        iq[0, 1] = ik[0, 1] = 9
        per = rng.permutation(200)[:13]
        iq[0, 2] = per[np.arange(N) % 13]
        ik[0, 2] = per[(np.arange(N) + 5) % 13]
        iq[0, 3] = rng.integers(0, 4, N)
        ik[0, 3] = rng.integers(0, 4, N)
        iq[0, 4] = np.repeat(rng.integers(0, 3, N // 16), 16)
        ik[0, 4] = np.repeat(rng.integers(0, 3, N // 16), 16)
        return iq, ik
    x = _inputs(1, N, 5, 8, 32, 11, labels)
    modes = oracle.row_modes(x[4], x[5], 8, 32)
    assert set(modes.reshape(-1).tolist()) >= {0, 3, 4}, modes
    check_fwd_bwd(*x, np.linspace(-0.4, 0.4, 5).astype(np.float32))


def prefill_padded():
    """prefill rows padded from 79 to 256 tokens (the inference tests' shapes): random,
    identical (prefix rows over the real positions) and disjoint labels"""
    tau = np.array([0.0, 0.35], np.float32)
    for pattern in ("repeat", "random", "mismatch"):
        rng = np.random.default_rng(83)
        n, pad = 79, 256
        iq = rng.integers(0, 4, (2, 2, n)).astype(np.int32)
        ik = rng.integers(0, 4, (2, 2, n)).astype(np.int32)
        if pattern == "repeat":
            iq[:] = 0
            ik[:] = 0
        elif pattern == "mismatch":
            iq[:] = 0
            ik[:] = 1
        sq, sk, v = (oracle.bf16_round(rng.standard_normal((2, n, 2, c)) * 0.2)
                     for c in (16, 16, 32))
        padl = lambda x: np.concatenate([x, np.zeros((2, 2, pad - n), np.int32)], 2)  # noqa
        padv = lambda x: np.concatenate([x, np.zeros((2, pad - n) + x.shape[2:],  # noqa
                                                     np.float32)], 1)
        out, l2 = drv.prefill(padv(sq), padv(sk), padv(v), padl(iq), padl(ik),
                              oracle.log_weights(tau, pad), n)
        want, wl2, _, _ = oracle.forward(sq, sk, v, iq, ik, np.ones((2, 2), bool),
                                         oracle.log_weights(tau, n))
        assert same_bits(out[:, :n], want), pattern
        assert same_bits(l2[:, :, :n], wl2), pattern
        if pattern == "repeat":
            break  # the suite runs the prefix-row case; the others by name below


def prefill_other():
    """prefill of the random and disjoint patterns (see prefill_padded)"""
    tau = np.array([0.0, 0.35], np.float32)
    for pattern in ("random", "mismatch"):
        rng = np.random.default_rng(83)
        n, pad = 79, 256
        iq = rng.integers(0, 4, (2, 2, n)).astype(np.int32)
        ik = rng.integers(0, 4, (2, 2, n)).astype(np.int32)
        if pattern == "mismatch":
            iq[:] = 0
            ik[:] = 1
        sq, sk, v = (oracle.bf16_round(rng.standard_normal((2, n, 2, c)) * 0.2)
                     for c in (16, 16, 32))
        padl = lambda x: np.concatenate([x, np.zeros((2, 2, pad - n), np.int32)], 2)  # noqa
        padv = lambda x: np.concatenate([x, np.zeros((2, pad - n) + x.shape[2:],  # noqa
                                                     np.float32)], 1)
        out, l2 = drv.prefill(padv(sq), padv(sk), padv(v), padl(iq), padl(ik),
                              oracle.log_weights(tau, pad), n)
        want, wl2, _, _ = oracle.forward(sq, sk, v, iq, ik, np.ones((2, 2), bool),
                                         oracle.log_weights(tau, n))
        assert same_bits(out[:, :n], want), pattern
        assert same_bits(l2[:, :, :n], wl2), pattern



def packed_docs(size="512"):
    """a packed batch-1 call of two documents of N/2 tokens in two training rows (hard flags
    [[T, F], [F, T]]): every hard document equals the CPU model on that document alone, soft
    documents give zeros; dtau over the hard documents.  N = 4096 with two-byte labels takes
    the multi-block sort through two chunks per segment and two digits per key"""
    N, H, R, DV = int(size), 2, 8, 64
    half = N // 2
    if N > 512:
        def labels(rng):
            return (rng.integers(0, 3000, (1, H, N)).astype(np.int32),
                    rng.integers(0, 3000, (1, H, N)).astype(np.int32))
        q, k, v, do, iq, ik = _inputs(1, N, H, R, DV, 31, labels)
    else:
        q, k, v, do, iq, ik = _inputs(1, N, H, R, DV, 31)
    hard_rows = np.array([[True, False], [False, True]])
    tau = np.array([0.4, -0.3], np.float32)
    offsets = [0, half, N]
    lut = oracle.log_weights(tau, half)
    dlut = oracle.dlog_weights(tau, half)
    out, l2, lm, ja, dsq, dsk, dv, dtau, rowtau = drv.packed(q, k, v, do, iq, ik, hard_rows,
                                                            lut, dlut, offsets, half)
    want_rt = np.zeros((1, H, N), np.float32)
    dense = oracle.packed_dense_flags(iq, ik, offsets)
    for d, (a, z) in enumerate(((0, half), (half, N))):
        flags = hard_rows[d:d + 1]
        args = (q[:, a:z], k[:, a:z], v[:, a:z])
        labs = (iq[:, :, a:z], ik[:, :, a:z])
        o, l2o, lmo, jao = oracle.forward(*args, *labs, flags, lut, dense=dense)
        assert same_bits(out[:, a:z], o), ("packed output", d)
        assert same_bits(l2[:, :, a:z], l2o), ("packed normalizer", d)
        assert np.array_equal(lm[:, :, a:z], lmo), ("packed lmax", d)
        assert np.array_equal(ja[:, :, a:z], np.where(jao >= 0, jao + a, -1)), ("jarg", d)
        g = oracle.backward(*args, do[:, a:z], *labs, flags, lut, dlut, l2o, dense=dense)
        for x, y, name in zip((dsq[:, a:z], dsk[:, a:z], dv[:, a:z]), g[:3], ("dsq", "dsk", "dv")):
            assert same_bits(x, y), (name, d)
        want_rt[:, :, a:z] = g[4]
    assert same_bits(rowtau, want_rt), "rowtau"
    assert same_bits(dtau, oracle.tau_reduce(want_rt)), "dtau"


def decode_chunks():
    """incremental decoding (prime 31 tokens, then chunks of 1, 5, 1, 11 and the rest) of the
    inference tests' random and identical-label rows: equal to the CPU model's decomposed
    forward bit for bit"""
    tau = np.array([0.0, 0.35], np.float32)
    for pattern in ("random", "repeat"):
        rng = np.random.default_rng(83)
        n = 79
        iq = rng.integers(0, 4, (2, 2, n)).astype(np.int32)
        ik = rng.integers(0, 4, (2, 2, n)).astype(np.int32)
        if pattern == "repeat":
            iq[:] = 0
            ik[:] = 0
        sq, sk, v = (oracle.bf16_round(rng.standard_normal((2, n, 2, c)) * 0.2)
                     for c in (16, 16, 32))
        want, _, _, _ = oracle.forward(sq, sk, v, iq, ik, np.ones((2, 2), bool),
                                       oracle.log_weights(tau, n), dense=0)
        dec = drv.Decoder(2, 2, 16, 32, 79, oracle.log_weights(tau, 256), slots=64)
        dec.prime(iq[..., :31], ik[..., :31], sk[:, :31], v[:, :31])
        outs, t = [], 31
        for step in (1, 5, 1, 11, n - 49):
            outs.append(dec.append(iq[..., t:t + step], ik[..., t:t + step], sq[:, t:t + step],
                                   sk[:, t:t + step], v[:, t:t + step]))
            t += step
        assert same_bits(np.concatenate(outs, axis=1), want[:, 31:]), pattern


def noalloc_forward():
    """the allocation-free forward (library scratch) equals the CPU model"""
    q, k, v, do, iq, ik = _inputs(1, 256, 2, 8, 64, 5)
    tau = np.array([0.5, -0.1], np.float32)
    hard = np.ones((1, 2), bool)
    lut = oracle.log_weights(tau, 256)
    out, l2, lm, ja = drv.noalloc(q, k, v, iq, ik, hard, lut)
    o, l2o, lmo, jao = oracle.forward(q, k, v, iq, ik, hard, lut)
    assert same_bits(out, o) and same_bits(l2, l2o)
    assert np.array_equal(lm, lmo) and np.array_equal(ja, jao)


def grid(spec):
    """one fwd+bwd case "pattern:R:DV:dtype:N[:staged]" over the five label patterns of the
    reference (tests/_data.labels) with soft rows (tests/_data.flags), B=2, H=2"""
    from tests._data import flags, labels, taus, vectors
    parts = spec.split(":")
    pattern, R, DV, dtype, N = parts[0], int(parts[1]), int(parts[2]), parts[3], int(parts[4])
    fused = not (len(parts) > 5 and parts[5] == "staged")
    B, H = 2, 2
    iq, ik = labels(N, pattern, b=B, h=H)
    sq, sk, v = vectors(N, b=B, h=H, r=R, dv=DV)
    rng = np.random.default_rng(R * 1000 + DV)
    do = oracle.bf16_round(rng.standard_normal(v.shape))
    if dtype == "f32":
        sq = sq + np.float32(1e-3) * rng.standard_normal(sq.shape).astype(np.float32)
    code = 0 if dtype == "bf16" else 1
    hard = flags(B, H)
    tau = taus(H)
    lut = oracle.log_weights(tau, N)
    fwd = drv.forward if fused else drv.staged
    out, l2, lm, ja, st = fwd(sq, sk, v, iq, ik, hard, lut, dtype=code)
    o, l2o, lmo, jao = oracle.forward(sq, sk, v, iq, ik, hard, lut)
    assert same_bits(out, o), "forward output"
    assert same_bits(l2, l2o), "normalizer"
    assert np.array_equal(lm, lmo) and np.array_equal(ja, jao), "lmax/argmax"
    dl = oracle.dlog_weights(tau, N)
    got = drv.backward(st, do, dl, l2, dtype=code)
    ref = oracle.backward(sq, sk, v, do, iq, ik, hard, lut, dl, l2o)
    for g, r, name in zip(got, ref, ("dsq", "dsk", "dv", "dtau", "rowtau")):
        assert same_bits(g, r), name


def long_runs(alphabet="1024"):
    """copied spans longer than RUN_MIN (the run list) in rows planned in global memory
    (labels of two bytes) or in LDS (one byte), N = 1024; fwd+bwd bit-exact"""
    A = int(alphabet)
    N = 1024

    def labels(rng):
        iq = rng.integers(0, A, (1, 2, N)).astype(np.int32)
        ik = rng.integers(0, A, (1, 2, N)).astype(np.int32)
        iq[0, :, 600:720] = ik[0, :, 100:220]
        iq[0, 1, 900:1000] = ik[0, 1, 300:400]
        return iq, ik
    x = _inputs(1, N, 2, 8, 32, 13, labels)
    check_fwd_bwd(*x, np.array([0.5, -0.2], np.float32))


def prefill_resets():
    """prefill of identical-label rows with query resets every 19 tokens (the inference
    tests' case): the CPU model with resets"""
    tau = np.array([0.0, 0.35], np.float32)
    rng = np.random.default_rng(83)
    n, pad = 79, 256
    iq = np.zeros((2, 2, n), np.int32)
    ik = np.zeros((2, 2, n), np.int32)
    sq, sk, v = (oracle.bf16_round(rng.standard_normal((2, n, 2, c)) * 0.2)
                 for c in (16, 16, 32))
    reset = np.zeros((2, 2, n), bool)
    reset[..., 17::19] = True
    padl = lambda x: np.concatenate([x, np.zeros((2, 2, pad - n), x.dtype)], 2)  # noqa
    padv = lambda x: np.concatenate([x, np.zeros((2, pad - n) + x.shape[2:], np.float32)], 1)  # noqa
    out, l2 = drv.prefill(padv(sq), padv(sk), padv(v), padl(iq), padl(ik),
                          oracle.log_weights(tau, pad), n, reset=padl(reset.astype(np.uint8)))
    want, wl2, _, _ = oracle.forward(sq, sk, v, iq, ik, np.ones((2, 2), bool),
                                     oracle.log_weights(tau, n), reset=reset)
    assert same_bits(out[:, :n], want) and same_bits(l2[:, :, :n], wl2)


def probe_modes():
    """the walk-cost probe: rows with a period of 80 distinct labels (sparse: M = N^2/80, but
    every diagonal d = 80 m is one long run, cost ~ N^3/480 > N^2) become strip-bounded rows
    (mode 2), planned in global memory (two-byte labels) or in LDS (one byte); random rows
    stay mode 0; fwd+bwd bit-exact"""
    N = 1024

    def labels(rng):
        iq = rng.integers(0, 256, (1, 4, N)).astype(np.int32)
        ik = rng.integers(0, 256, (1, 4, N)).astype(np.int32)
        per2 = rng.permutation(5000)[:80].astype(np.int32) + 300   # two-byte labels
        per1 = rng.permutation(256)[:80].astype(np.int32)          # one-byte labels
        iq[0, 0] = ik[0, 0] = per2[np.arange(N) % 80]
        iq[0, 1] = ik[0, 1] = per1[np.arange(N) % 80]
        iq[0, 3] = rng.integers(0, 3000, N)                         # random, two-byte
        ik[0, 3] = rng.integers(0, 3000, N)
        return iq, ik
    q, k, v, do, iq, ik = _inputs(1, N, 4, 8, 32, 17, labels)
    assert (oracle.row_modes(iq, ik, 8, 32) == 0).all()
    a, b, c = drv.vec(q, 0), drv.vec(k, 0), drv.vec(v, 0)
    nb = drv.lib.dism_hard_workspace_bytes(1, N, 4, 8, 32, 0)
    ws = drv.aligned(nb)
    ws[:] = 0xCD
    drv.call("dism_hard_prepare", drv.p(a), drv.p(b), drv.p(c), 0, drv.p(iq), drv.p(ik), 1, N,
             4, 8, 32, drv.p(ws), nb, None)
    modes = np.empty((1, 4), np.int32)
    drv.call("dism_hard_row_modes", drv.p(ws), nb, 1, N, 4, 8, 32, drv.p(modes), None)
    assert modes.tolist() == [[2, 2, 0, 0]], modes
    check_fwd_bwd(q, k, v, do, iq, ik, np.linspace(-0.3, 0.3, 4).astype(np.float32))


def vocab():
    """codebook argmax labels on the emulated matrix-core tiles: random, duplicated (exact
    ties: first index) and near-tie rows, per-head and shared vocabularies, a vocabulary that
    is not a multiple of 32 rows; equal to the exact CPU model"""
    rng = np.random.default_rng(21)
    B, N, H = 1, 64, 2
    for D, V, shared in ((32, 96, False), (64, 70, True), (128, 40, False)):
        x = oracle.bf16_round(rng.standard_normal((B, N, H, D)))
        voc = oracle.bf16_round(rng.standard_normal((V, D) if shared else (H, V, D)))
        if not shared:
            # duplicated rows: exact ties (first index wins), and tokens equal to them
            voc[:, V - 3] = voc[:, 7]
            x[0, :8, :, :] = voc[:, 7][None, :, :].transpose(0, 1, 2)
        got, rescored = drv.vocab_labels(x, voc)
        want = oracle.vocab_labels(x, voc)
        assert np.array_equal(got, want), (D, V, shared, int((got != want).sum()))
        assert shared or rescored > 0, "ties must be rescored in fp64"


def packed_graph_offsets():
    """a packed call with the fixed-capacity offsets of a graph layout: one slot per 256
    tokens, the padding slots repeating the token count (empty documents at the end), and
    the documents' labels tagged with that slot count (oracle.packed_dense_flags slots=)"""
    N, H, R, DV = 1024, 2, 8, 32
    q, k, v, do, iq, ik = _inputs(1, N, H, R, DV, 41)
    hard_rows = np.ones((1, H), bool)
    tau = np.array([0.2, -0.4], np.float32)
    docs = ((0, 256), (256, 1024))
    offsets = [0, 256, 1024, 1024, 1024]
    lut = oracle.log_weights(tau, N)
    dlut = oracle.dlog_weights(tau, N)
    out, l2, lm, ja, dsq, dsk, dv, dtau, rowtau = drv.packed(q, k, v, do, iq, ik, hard_rows,
                                                            lut, dlut, offsets, 768)
    dense = oracle.packed_dense_flags(iq, ik, offsets, slots=len(offsets) - 1)
    want_rt = np.zeros((1, H, N), np.float32)
    for a, z in docs:
        lt = oracle.log_weights(tau, z - a)
        dt = oracle.dlog_weights(tau, z - a)
        args = (q[:, a:z], k[:, a:z], v[:, a:z])
        labs = (iq[:, :, a:z], ik[:, :, a:z])
        o, l2o, lmo, jao = oracle.forward(*args, *labs, hard_rows, lt, dense=dense)
        assert same_bits(out[:, a:z], o), ("out", a)
        assert same_bits(l2[:, :, a:z], l2o), ("lse2", a)
        g = oracle.backward(*args, do[:, a:z], *labs, hard_rows, lt, dt, l2o, dense=dense)
        for x, y, name in zip((dsq[:, a:z], dsk[:, a:z], dv[:, a:z]), g[:3], ("dsq", "dsk", "dv")):
            assert same_bits(x, y), (name, a)
        want_rt[:, :, a:z] = g[4]
    assert same_bits(dtau, oracle.tau_reduce(want_rt)), "dtau"

if __name__ == "__main__":
    for name in sys.argv[1:]:
        fn, _, arg = name.partition("=")
        globals()[fn](*([arg] if arg else []))
        print("OK", name, flush=True)
