"""CPU oracle for the flash_dism hard core -- TEST INFRASTRUCTURE ONLY.

Two independent layers:
  * ``oracle.dense``: FP64 numpy restatement of the reference's dense torch oracle
    (dism_v3/python/flash_dism/reference/dism_v3_ref.py), feasible for N <= ~2048;
  * ``liboracle.so`` (built from ``dism_cpu_model.c``): the CPU model with the exact fp32
    operation order of the HIP kernels, used for bit-exact checks and as the timed CPU
    baseline (``cpu_baseline.kind = "port"``).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this package.
The product path (dism_amd) must never import it.

Parity pinning status of every function is asserted in tests/test_oracle.py.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
SOURCE = os.path.join(HERE, "dism_cpu_model.c")
CFLAGS = ["-O3", "-fPIC", "-shared", "-fopenmp", "-ffp-contract=off", "-mfma", "-mavx2",
          "-fno-fast-math", "-Wall"]

_lib = None


def build(force=False):
    """Compile dism_cpu_model.c -> liboracle.so with gcc (recipe also in oracle/Makefile)."""
    if force or not os.path.exists(LIB_PATH) or \
            os.path.getmtime(LIB_PATH) < os.path.getmtime(SOURCE):
        subprocess.check_call(["gcc", *CFLAGS, "-o", LIB_PATH, SOURCE, "-lm"])
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.c_void_p
        i32, i64 = ctypes.c_int, ctypes.c_long
        L.orc_exp2f.restype = ctypes.c_float
        L.orc_exp2f.argtypes = [ctypes.c_float]
        L.orc_log2f.restype = ctypes.c_float
        L.orc_log2f.argtypes = [ctypes.c_float]
        L.orc_logd.restype = ctypes.c_double
        L.orc_logd.argtypes = [ctypes.c_double]
        L.orc_expd.restype = ctypes.c_double
        L.orc_expd.argtypes = [ctypes.c_double]
        L.orc_log_weight.restype = ctypes.c_float
        L.orc_log_weight.argtypes = [ctypes.c_float, i64]
        L.orc_dlog_weight.restype = ctypes.c_float
        L.orc_dlog_weight.argtypes = [ctypes.c_float, i64]
        L.orc_lut.argtypes = [P, i32, i64, P]
        L.orc_dlut.argtypes = [P, i32, i64, P]
        L.orc_sign_labels.argtypes = [P, i64, i32, P]
        L.orc_boundary.argtypes = [P, P, P, i32, i32, i64, i32, i32, P]
        L.orc_chunk.argtypes = [P, i64, i64, i64, P]
        L.orc_suffix_walk.restype = i64
        L.orc_suffix_walk.argtypes = [P, P, i64, i64]
        L.orc_forward.argtypes = [P, P, P, P, P, P, P, i64, i32, i64, i32, i32, i32, P, P, P,
                                  P, i32]
        L.orc_backward.argtypes = [P, P, P, P, P, P, P, P, P, i64, P, i32, i64, i32, i32, i32,
                                   P, P, P, P, i32]
        L.orc_forward_direct.argtypes = L.orc_forward.argtypes
        L.orc_forward_reset.argtypes = L.orc_forward.argtypes + [P]
        L.orc_vocab_labels.argtypes = [P, P, i64, i32, i64, i32, i64, i32, P]
        L.orc_suffix_walk_from.restype = i64
        L.orc_suffix_walk_from.argtypes = [P, P, i64, i64, i64]
        L.orc_backward_direct.argtypes = L.orc_backward.argtypes
        L.orc_tau_reduce.argtypes = [P, i32, i32, i64, i64, i64, P]
        L.orc_forward_flags.argtypes = L.orc_forward.argtypes + [P, P]
        L.orc_backward_flags.argtypes = L.orc_backward.argtypes + [P]
        L.orc_bucket_collisions.restype = ctypes.c_uint64
        L.orc_bucket_collisions.argtypes = [P, P, i64]
        L.orc_dense_rows.argtypes = [P, P, P, i32, i64, P]
        L.orc_row_modes.argtypes = [P, P, i32, i64, i32, i32, P]
        L.orc_level_row.restype = i32
        L.orc_level_row.argtypes = [P, P, i64, i32, i32]
        L.orc_prefix_row.restype = i32
        L.orc_prefix_row.argtypes = [P, P, i64]
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _f32(x):
    return np.ascontiguousarray(np.asarray(x, dtype=np.float32))


def _i32(x):
    return np.ascontiguousarray(np.asarray(x, dtype=np.int32))


def _flags(hard):
    return np.ascontiguousarray(np.asarray(hard, dtype=np.uint8).reshape(-1))


def bf16_round(x):
    """Round float32 -> bfloat16 (round to nearest even), returned as float32 values."""
    x = _f32(x)
    b = x.view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32)
    return np.where(np.isnan(x), x, out)


def exp2f(x):
    return lib().orc_exp2f(float(x))


def log2f(x):
    return lib().orc_log2f(float(x))


def sign_labels(x):
    """x [B,N,H,d] -> int32 labels [B,H,N], bit d set iff x[...,d] > 0."""
    x = _f32(x)
    B, N, H, d = x.shape
    out = np.empty((B, N, H), dtype=np.int32)
    lib().orc_sign_labels(_p(x), B * N * H, d, _p(out))
    return np.ascontiguousarray(out.transpose(0, 2, 1))


def log_weights(tau, max_length):
    tau = _f32(tau)
    out = np.empty((tau.shape[0], max_length + 1), dtype=np.float32)
    lib().orc_lut(_p(tau), tau.shape[0], max_length + 1, _p(out))
    return out


def dlog_weights(tau, max_length):
    tau = _f32(tau)
    out = np.empty((tau.shape[0], max_length + 1), dtype=np.float32)
    lib().orc_dlut(_p(tau), tau.shape[0], max_length + 1, _p(out))
    return out


def boundary(iq, ik, hard, strip=32, composed=True):
    """Strip summaries (composed=False) or composed boundaries, int32 [B,H,(N-1)//S,N]."""
    iq, ik = _i32(iq), _i32(ik)
    B, H, N = iq.shape
    out = np.empty((B, H, (N - 1) // strip, N), dtype=np.int32)
    lib().orc_boundary(_p(iq), _p(ik), _p(_flags(hard)), B, H, N, strip, int(composed), _p(out))
    return out


def chunk(summary):
    s = _i32(summary)
    B, H, C, N = s.shape
    out = np.empty_like(s)
    lib().orc_chunk(_p(s), B * H, C, N, _p(out))
    return out


def suffix_walk(q, k, i, j):
    q, k = _i32(q), _i32(k)
    return lib().orc_suffix_walk(_p(q), _p(k), i, j)


def reset_starts(reset):
    """[B,H,N] bool query resets -> int32 [B,H,N]: last reset position at or before each
    query (0 where none)."""
    reset = np.asarray(reset, dtype=bool)
    pos = np.where(reset, np.arange(reset.shape[-1], dtype=np.int64), 0)
    return np.ascontiguousarray(np.maximum.accumulate(pos, axis=-1).astype(np.int32))


def dense_rows(iq, ik, hard):
    """Row classification of the HIP path: uint8 [B,H], 1 where a hard row's bucketed label
    collisions M (bucket_collisions) exceed N^2/64 (and N <= 65536)."""
    iq, ik = _i32(iq), _i32(ik)
    B, H, N = iq.shape
    out = np.empty(B * H, dtype=np.uint8)
    lib().orc_dense_rows(_p(iq), _p(ik), _p(_flags(hard)), B * H, N, _p(out))
    return out.reshape(B, H)


def row_modes(iq, ik, R, DV):
    """Row modes of a fixed-length call without resets as the HIP path chooses them (every row
    taken as hard): uint8 [B,H], 0 decomposed, 1 direct (dense), 3 levels (dense rows with
    labels below 256, N <= 4096, R * DV <= 512 and at most 32 levels: level_count), 4 prefix
    (dense rows whose every label has one predecessor label: prefix_row)."""
    iq, ik = _i32(iq), _i32(ik)
    B, H, N = iq.shape
    out = np.empty(B * H, dtype=np.uint8)
    lib().orc_row_modes(_p(iq), _p(ik), B * H, N, R, DV, _p(out))
    return out.reshape(B, H)


def prefix_row(q, k):
    """1 when one row (q, k [N]) is a prefix row: dense, and every label has one predecessor
    label over both sides (so every valid pair's match runs to the key's row start)."""
    q, k = _i32(q), _i32(k)
    return int(lib().orc_prefix_row(_p(q), _p(k), q.shape[-1]))


def level_count(q, k, R, DV):
    """Levels of one row (its longest match) when it is a level row, else 0."""
    q, k = _i32(q), _i32(k)
    return int(lib().orc_level_row(_p(q), _p(k), q.shape[-1], R, DV))


def packed_dense_flags(iq, ik, offsets, slots=None):
    """Row classification of a packed call (B = 1): the HIP path classifies each head row of
    its document-tagged labels tag = rank * slots + d (rank: dense rank of the raw label among
    the row's distinct labels in unsigned order; d: index among the non-empty documents;
    slots: the document count the library receives, by default the non-empty documents, for
    a fixed-capacity graph layout tokens / 256).  Returns uint8 [1, H]."""
    iq, ik = _i32(iq), _i32(ik)
    _, H, N = iq.shape
    offs = [int(x) for x in offsets]
    docs = [(a, z) for a, z in zip(offs, offs[1:]) if z > a]
    slots = len(docs) if slots is None else int(slots)
    dindex = np.empty(N, np.uint64)
    for d, (a, z) in enumerate(docs):
        dindex[a:z] = d
    tq = np.empty_like(iq)
    tk = np.empty_like(ik)
    for h in range(H):
        uq, uk = iq[0, h].view(np.uint32), ik[0, h].view(np.uint32)
        uniq = np.unique(np.concatenate([uq, uk]))
        for src, dst in ((uq, tq), (uk, tk)):
            rank = np.searchsorted(uniq, src).astype(np.uint64)
            tag = (rank * np.uint64(slots) + dindex) & np.uint64(0xFFFFFFFF)
            dst[0, h] = tag.astype(np.uint32).view(np.int32)
    return dense_rows(tq, tk, np.ones((1, H), bool))


def bucket_collisions(q, k):
    """M of one row: sum over the 4096 label buckets (top 12 bits of label * 0x9E3779B1) of
    (#queries in the bucket) x (#keys in the bucket)."""
    q, k = _i32(q), _i32(k)
    return int(lib().orc_bucket_collisions(_p(q), _p(k), q.shape[-1]))


def _dense_arg(dense, B, H):
    if dense is None:
        return None
    d = np.ascontiguousarray(np.broadcast_to(np.asarray(dense, dtype=np.uint8), (B, H)))
    return d.reshape(-1)


def forward(sq, sk, v, iq, ik, hard, lut, threads=0, direct=False, reset=None, dense=None):
    """CPU model forward.  Returns (O fp32 [B,N,H,DV], lse2 [B,H,N], Lmax, argmax).

    direct=False: the sequence the HIP kernels reproduce bit for bit -- per row, the prefix
    definition for prefix rows (row_modes 4), the level definition for level rows (3), the direct (pairwise) definition for the other
    rows classified dense (dense_rows) and the decomposed one for the rest;  direct=True: the
    pairwise definition for every row.
    dense: optional [B,H] (or scalar) override of the row modes (0 decomposed, 1 direct,
    3 levels where the row qualifies, else direct, 4 the prefix definition, which assumes a
    prefix row).
    reset: optional [B,H,N] bool query resets (inference semantics: a reset query's match
    starts afresh at that query; keys stay)."""
    sq, sk, v, lut = _f32(sq), _f32(sk), _f32(v), _f32(lut)
    iq, ik = _i32(iq), _i32(ik)
    B, N, H, R = sq.shape
    DV = v.shape[-1]
    out = np.empty((B, N, H, DV), dtype=np.float32)
    lse2 = np.empty((B, H, N), dtype=np.float32)
    lmax = np.empty((B, H, N), dtype=np.int32)
    jarg = np.empty((B, H, N), dtype=np.int32)
    args = (_p(sq), _p(sk), _p(v), _p(iq), _p(ik), _p(_flags(hard)), _p(lut), lut.shape[1], B,
            N, H, R, DV, _p(out), _p(lse2), _p(lmax), _p(jarg), threads)
    dflags = _dense_arg(dense, B, H)
    if reset is not None or dflags is not None:
        assert not direct
        wlo = reset_starts(reset) if reset is not None else None
        lib().orc_forward_flags(*args, None if wlo is None else _p(wlo),
                                None if dflags is None else _p(dflags))
    else:
        (lib().orc_forward_direct if direct else lib().orc_forward)(*args)
    return out, lse2, lmax, jarg


def tau_reduce(rowtau, block=64, group=32):
    """dtau [H] from rowtau [B,H,N] in the fixed order of the HIP reduction (orc_tau_reduce:
    blocks of `block` rows, groups of `group` blocks, each level summed sequentially in
    double, rounded to float)."""
    rowtau = _f32(rowtau)
    B, H, N = rowtau.shape
    dtau = np.empty(H, dtype=np.float32)
    lib().orc_tau_reduce(_p(rowtau), B, H, N, block, group, _p(dtau))
    return dtau


def backward(sq, sk, v, dout, iq, ik, hard, lut, dlut, lse2, threads=0, direct=False,
             dense=None):
    """CPU model backward.  Returns (dSQ, dSK, dV fp32, dtau [H], rowtau [B,H,N]).
    `direct` and `dense` as in forward()."""
    sq, sk, v, dout, lut, dlut, lse2 = map(_f32, (sq, sk, v, dout, lut, dlut, lse2))
    iq, ik = _i32(iq), _i32(ik)
    B, N, H, R = sq.shape
    DV = v.shape[-1]
    dsq = np.empty_like(sq)
    dsk = np.empty_like(sk)
    dv = np.empty_like(v)
    rowtau = np.empty((B, H, N), dtype=np.float32)
    args = (_p(sq), _p(sk), _p(v), _p(dout), _p(iq), _p(ik), _p(_flags(hard)), _p(lut),
            _p(dlut), lut.shape[1], _p(lse2), B, N, H, R, DV, _p(dsq), _p(dsk), _p(dv),
            _p(rowtau), threads)
    dflags = _dense_arg(dense, B, H)
    if dflags is not None:
        assert not direct
        lib().orc_backward_flags(*args, _p(dflags))
    else:
        (lib().orc_backward_direct if direct else lib().orc_backward)(*args)
    return dsq, dsk, dv, tau_reduce(rowtau), rowtau


def vocab_labels(x, vocab):
    """Exact codebook argmax labels [B,H,N] (first index on ties): x [B,N,H,D] floats (bf16
    values), vocab [H,V,D] or shared [V,D]."""
    x = _f32(x)
    vocab = _f32(vocab)
    B, N, H, D = x.shape
    V = vocab.shape[-2]
    vhs = 0 if vocab.ndim == 2 else V * D
    out = np.empty((B, H, N), dtype=np.int32)
    lib().orc_vocab_labels(_p(x), _p(vocab), vhs, B, N, H, V, D, _p(out))
    return out
