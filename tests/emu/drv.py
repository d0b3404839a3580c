"""ctypes driver of the CPU-emulated library (tests/emu/build.py): the C ABI of
include/dism_hard.h called with numpy host buffers.  Test infrastructure only."""
import ctypes
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from dism_amd import _lib as L  # noqa: E402  (argument types of the C ABI only)

LIB = os.environ["DISM_EMU_LIB"]
lib = ctypes.CDLL(LIB)
for name, args in L.SIGNATURES.items():
    f = getattr(lib, name); f.argtypes = args; f.restype = ctypes.c_int32
for name, args in L.SIZE_SIGNATURES.items():
    f = getattr(lib, name); f.argtypes = args; f.restype = ctypes.c_int64
lib.dism_last_error.restype = ctypes.c_char_p
lib.dism_layout_check.restype = ctypes.c_int32


def p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def call(name, *args):
    rc = getattr(lib, name)(*args)
    if rc != 0:
        raise RuntimeError(f"{name}: {lib.dism_last_error().decode()}")


def bf16_bits(x):
    x = np.ascontiguousarray(x, np.float32)
    return (x.view(np.uint32) >> 16).astype(np.uint16)


def vec(x, dtype):
    return bf16_bits(x) if dtype == 0 else np.ascontiguousarray(x, np.float32)


def aligned(nbytes):
    buf = np.empty(nbytes + 256, np.uint8)
    off = (-buf.ctypes.data) % 256
    return buf[off:off + nbytes]


def forward(sq, sk, v, iq, ik, hard, lut, dtype=0, out_dtype=1, prepared=None):
    B, N, H, R = sq.shape
    DV = v.shape[-1]
    a, b, c = vec(sq, dtype), vec(sk, dtype), vec(v, dtype)
    iq = np.ascontiguousarray(iq, np.int32); ik = np.ascontiguousarray(ik, np.int32)
    hd = np.ascontiguousarray(np.broadcast_to(hard, (B, H)), np.uint8)
    lut = np.ascontiguousarray(lut, np.float32)
    nb = lib.dism_hard_workspace_bytes(B, N, H, R, DV, dtype)
    ws = aligned(nb); ws[:] = 0xCD
    out = np.empty((B, N, H, DV), np.float32 if out_dtype == 1 else np.uint16)
    lse2 = np.empty((B, H, N), np.float32)
    lmax = np.empty((B, H, N), np.int32); jarg = np.empty((B, H, N), np.int32)
    call("dism_hard_forward", p(a), p(b), p(c), dtype, p(iq), p(ik), p(hd), None, 0, p(lut),
         lut.shape[1], B, N, H, R, DV, p(ws), nb, p(out), out_dtype, p(lse2), p(lmax), p(jarg), None)
    return out, lse2, lmax, jarg, (ws, nb, a, b, c, iq, ik, hd, lut)


def backward(st, dout, dlut, lse2, dtype=0):
    ws, nb, a, b, c, iq, ik, hd, lut = st
    B, H, N = iq.shape
    R = a.size // (B * N * H); DV = c.size // (B * N * H)
    d = vec(dout, dtype)
    dlut = np.ascontiguousarray(dlut, np.float32)
    dsq = np.empty((B, N, H, R), np.float32); dsk = np.empty_like(dsq)
    dv = np.empty((B, N, H, DV), np.float32); rowtau = np.empty((B, H, N), np.float32)
    dtau = np.empty(H, np.float32)
    call("dism_hard_backward", p(a), p(b), p(c), p(d), dtype, p(iq), p(ik), p(hd), None, 0,
         p(lut), p(dlut), lut.shape[1], p(lse2), B, N, H, R, DV, p(ws), nb, p(dsq), p(dsk),
         p(dv), p(rowtau), p(dtau), None)
    return dsq, dsk, dv, dtau, rowtau


def prefill(sq, sk, v, iq, ik, lut, n_valid, reset=None, dtype=0):
    B, N, H, R = sq.shape
    DV = v.shape[-1]
    a, b, c = vec(sq, dtype), vec(sk, dtype), vec(v, dtype)
    iq = np.ascontiguousarray(iq, np.int32); ik = np.ascontiguousarray(ik, np.int32)
    lut = np.ascontiguousarray(lut, np.float32)
    nb = lib.dism_hard_prefill_workspace_bytes(B, N, H, R, DV, dtype)
    ws = aligned(nb); ws[:] = 0xCD
    out = np.empty((B, N, H, DV), np.float32); lse2 = np.empty((B, H, N), np.float32)
    rs = None if reset is None else np.ascontiguousarray(reset, np.uint8)
    call("dism_hard_prefill", p(a), p(b), p(c), dtype, p(iq), p(ik), p(rs), p(lut), lut.shape[1],
         B, N, n_valid, H, R, DV, p(ws), nb, p(out), p(lse2), None)
    return out, lse2


def staged(sq, sk, v, iq, ik, hard, lut, dtype=0, out_dtype=1):
    B, N, H, R = sq.shape
    DV = v.shape[-1]
    a, b, c = vec(sq, dtype), vec(sk, dtype), vec(v, dtype)
    iq = np.ascontiguousarray(iq, np.int32); ik = np.ascontiguousarray(ik, np.int32)
    hd = np.ascontiguousarray(np.broadcast_to(hard, (B, H)), np.uint8)
    lut = np.ascontiguousarray(lut, np.float32)
    nb = lib.dism_hard_workspace_bytes(B, N, H, R, DV, dtype)
    ws = aligned(nb); ws[:] = 0xCD
    call("dism_hard_prepare", p(a), p(b), p(c), dtype, p(iq), p(ik), B, N, H, R, DV, p(ws), nb, None)
    out = np.empty((B, N, H, DV), np.float32)
    lse2 = np.empty((B, H, N), np.float32)
    lmax = np.empty((B, H, N), np.int32); jarg = np.empty((B, H, N), np.int32)
    call("dism_hard_readout", p(a), p(b), p(c), dtype, p(iq), p(ik), p(hd), None, 0, p(lut),
         lut.shape[1], B, N, H, R, DV, p(ws), nb, p(out), out_dtype, p(lse2), p(lmax), p(jarg), None)
    return out, lse2, lmax, jarg, (ws, nb, a, b, c, iq, ik, hd, lut)


def packed(sq, sk, v, do, iq, ik, hard_rows, lut, dlut, offsets, longest, dtype=0):
    """packed prepare + readout + backward; offsets are the non-empty documents' starts + N"""
    _, N, H, R = sq.shape
    DV = v.shape[-1]
    a, b, c, d = vec(sq, dtype), vec(sk, dtype), vec(v, dtype), vec(do, dtype)
    iq = np.ascontiguousarray(iq, np.int32); ik = np.ascontiguousarray(ik, np.int32)
    cu = np.ascontiguousarray(offsets, np.int32)
    hd = np.ascontiguousarray(hard_rows, np.uint8)
    lut = np.ascontiguousarray(lut, np.float32); dlut = np.ascontiguousarray(dlut, np.float32)
    nb = lib.dism_hard_packed_workspace_bytes(N, H, R, DV, dtype)
    ws = aligned(nb); ws[:] = 0xCD
    call("dism_hard_packed_prepare", p(a), p(b), p(c), dtype, p(iq), p(ik), p(cu), cu.size - 1,
         N, H, R, DV, p(ws), nb, None)
    out = np.empty((1, N, H, DV), np.float32); lse2 = np.empty((1, H, N), np.float32)
    lmax = np.empty((1, H, N), np.int32); jarg = np.empty((1, H, N), np.int32)
    call("dism_hard_packed_readout", p(a), p(b), p(c), dtype, p(hd), hd.shape[0], p(lut),
         lut.shape[1], longest, N, H, R, DV, p(ws), nb, p(out), 1, p(lse2), p(lmax), p(jarg), None)
    dsq = np.empty((1, N, H, R), np.float32); dsk = np.empty_like(dsq)
    dv = np.empty((1, N, H, DV), np.float32); rowtau = np.empty((1, H, N), np.float32)
    dtau = np.empty(H, np.float32)
    call("dism_hard_packed_backward", p(a), p(b), p(c), p(d), dtype, p(hd), hd.shape[0], p(lut),
         p(dlut), lut.shape[1], longest, p(lse2), N, H, R, DV, p(ws), nb, p(dsq), p(dsk), p(dv),
         p(rowtau), p(dtau), None)
    return out, lse2, lmax, jarg, dsq, dsk, dv, dtau, rowtau


class Decoder:
    def __init__(self, B, H, R, DV, capacity, lut, slots=64, dtype=0):
        self.B, self.H, self.R, self.DV, self.cap, self.slots, self.dtype = B, H, R, DV, capacity, slots, dtype
        self.lut = np.ascontiguousarray(lut, np.float32)
        self.nb = lib.dism_decoder_state_bytes(B * H, R, DV, capacity, slots, dtype)
        self.state = aligned(self.nb); self.state[:] = 0xCD
        call("dism_decoder_init", p(self.state), self.nb, B * H, R, DV, capacity, slots, dtype, None)

    def append(self, iq, ik, sq, sk, v, reset=None):
        n = iq.shape[-1]
        iq = np.ascontiguousarray(iq, np.int32); ik = np.ascontiguousarray(ik, np.int32)
        a, b, c = vec(sq, self.dtype), vec(sk, self.dtype), vec(v, self.dtype)
        out = np.empty((self.B, n, self.H, self.DV), np.float32)
        rs = None if reset is None else np.ascontiguousarray(reset, np.uint8)
        call("dism_decoder_step", p(self.state), self.nb, self.B, self.H, self.R, self.DV,
             self.cap, self.slots, self.dtype, n, p(iq), p(ik), p(rs), p(a), p(b), p(c),
             p(self.lut), self.lut.shape[1], p(out), None, None)
        return out

    def prime(self, iq, ik, sk, v):
        n = iq.shape[-1]
        iq = np.ascontiguousarray(iq, np.int32); ik = np.ascontiguousarray(ik, np.int32)
        b, c = vec(sk, self.dtype), vec(v, self.dtype)
        wb = lib.dism_decoder_prime_workspace_bytes(self.B, n, self.H, self.R, self.DV, self.dtype)
        ws = aligned(wb); ws[:] = 0xCD
        call("dism_decoder_prime", p(self.state), self.nb, self.B, self.H, self.R, self.DV,
             self.cap, self.slots, self.dtype, n, p(iq), p(ik), None, p(b), p(c), p(ws), wb, None)


def noalloc(sq, sk, v, iq, ik, hard, lut, dtype=0):
    B, N, H, R = sq.shape
    DV = v.shape[-1]
    a, b, c = vec(sq, dtype), vec(sk, dtype), vec(v, dtype)
    iq = np.ascontiguousarray(iq, np.int32); ik = np.ascontiguousarray(ik, np.int32)
    hd = np.ascontiguousarray(np.broadcast_to(hard, (B, H)), np.uint8)
    lut = np.ascontiguousarray(lut, np.float32)
    out = np.empty((B, N, H, DV), np.float32); lse2 = np.empty((B, H, N), np.float32)
    lmax = np.empty((B, H, N), np.int32); jarg = np.empty((B, H, N), np.int32)
    call("dism_hard_forward_noalloc", p(a), p(b), p(c), dtype, p(iq), p(ik), p(hd), p(lut),
         lut.shape[1], B, N, H, R, DV, p(out), 1, p(lse2), p(lmax), p(jarg), None)
    return out, lse2, lmax, jarg


def vocab_labels(x, vocab):
    """codebook argmax labels of x [B,N,H,D] (bf16 values) against vocab [H,V,D] or [V,D]"""
    B, N, H, D = x.shape
    V = vocab.shape[-2]
    a, b = bf16_bits(x), bf16_bits(vocab)
    out = np.empty((B, H, N), np.int32)
    scratch = np.empty(1 + 2 * H + B * H * N, np.int32)
    call("dism_vocab_labels", p(a), p(b), 0 if vocab.ndim == 2 else V * D, B, N, H, V, D,
         p(out), p(scratch), None)
    return out, int(scratch[0])
