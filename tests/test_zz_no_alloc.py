"""The allocation-free forward (dism_hard_forward_noalloc: workspace in the library's device
array, every launch on the caller's stream) against the existing one-call forward with a caller
workspace (dism_hard_forward), bit for bit: two calls in a row, the second smaller (the array
keeps the first call's contents), with sparse, dense and strip-bounded rows and soft rows;
the fp32 call also against the CPU model (oracle.forward), bit for bit.  Also the size
limit's error."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from tests._data import labels, taus, vectors

pytestmark = pytest.mark.gpu


def _inputs(b, h, n, r, dv, seed):
    rng = np.random.default_rng(seed)
    q, k = labels(n, "alphabet256", b=b, h=h, seed=seed)
    q[:, 0] = 3                                     # a dense row (identical labels)
    k[:, 0] = 3
    if h > 2:
        base = rng.integers(0, 256, 200)            # long repeats: strip-bounded walks
        q[:, 2] = base[np.arange(n) % 200]
        k[:, 2] = q[:, 2]
    sq, sk, v = vectors(n, b=b, h=h, r=r, dv=dv, seed=seed + 1)
    hard = np.ones((b, h), bool)
    if b > 1 and h > 1:
        hard[1, 1] = False
    return sq, sk, v, q, k, hard, taus(h)


def _call(entry, x, out_dtype):
    import dism_amd
    from dism_amd import _lib
    from dism_amd._checks import DTYPE_CODE
    sq, sk, v, q, k, hard, tau = x
    b, n, h, r = sq.shape
    dv = v.shape[-1]
    d = torch.device("cuda")
    t = [torch.from_numpy(a).to(d, torch.bfloat16) for a in (sq, sk, v)]
    iq, ik = torch.from_numpy(q).to(d), torch.from_numpy(k).to(d)
    th = torch.from_numpy(hard).to(d)
    lut = dism_amd.hard_log_weights(torch.from_numpy(tau).to(d), n)
    out = torch.empty((b, n, h, dv), dtype=out_dtype, device=d)
    lse2 = torch.empty((b, h, n), dtype=torch.float32, device=d)
    lmax = torch.empty((b, h, n), dtype=torch.int32, device=d)
    jarg = torch.empty((b, h, n), dtype=torch.int32, device=d)
    s = torch.cuda.current_stream(d).cuda_stream
    code = DTYPE_CODE[torch.bfloat16]
    common = (t[0].data_ptr(), t[1].data_ptr(), t[2].data_ptr(), code, iq.data_ptr(),
              ik.data_ptr(), th.data_ptr())
    if entry == "noalloc":
        _lib.call("dism_hard_forward_noalloc", *common, lut.data_ptr(), n + 1, b, n, h, r, dv,
                  out.data_ptr(), DTYPE_CODE[out_dtype], lse2.data_ptr(), lmax.data_ptr(),
                  jarg.data_ptr(), s)
    else:
        nbytes = _lib.workspace_bytes(b, n, h, r, dv, code)
        ws = torch.empty((nbytes,), dtype=torch.uint8, device=d)
        _lib.call("dism_hard_forward", *common, 0, 0, lut.data_ptr(), n + 1, b, n, h, r, dv,
                  ws.data_ptr(), nbytes, out.data_ptr(), DTYPE_CODE[out_dtype],
                  lse2.data_ptr(), lmax.data_ptr(), jarg.data_ptr(), s)
    torch.cuda.synchronize()
    return [a.cpu() for a in (out, lse2, lmax, jarg)]


def test_noalloc_forward_matches_workspace_forward():
    first = _inputs(2, 4, 2048, 8, 64, seed=5)
    second = _inputs(1, 3, 512, 16, 32, seed=9)     # smaller: the array holds stale data
    for x, od in ((first, torch.float32), (second, torch.bfloat16)):
        print(f"no-alloc forward {x[0].shape} {od}", flush=True)
        want = _call("workspace", x, od)
        got = _call("noalloc", x, od)
        for g, w, name in zip(got, want, ("out", "lse2", "lmax", "jarg")):
            assert torch.equal(g.view(torch.int16 if g.dtype == torch.bfloat16 else
                                      (torch.int32 if g.dtype.is_floating_point else g.dtype)),
                               w.view(torch.int16 if w.dtype == torch.bfloat16 else
                                      (torch.int32 if w.dtype.is_floating_point else w.dtype))), name
        if od == torch.float32:
            sq, sk, v, q, k, hard, tau = x
            ref = oracle.forward(sq, sk, v, q, k, hard, oracle.log_weights(tau, sq.shape[1]))
            for g, w, name in zip(got, ref, ("out", "lse2", "lmax", "jarg")):
                g = g.numpy()
                if g.dtype == np.float32:
                    assert np.array_equal(g.view(np.uint32),
                                          np.asarray(w, np.float32).view(np.uint32)), name
                else:
                    assert np.array_equal(g, w), name


def test_noalloc_forward_rejects_large_shapes():
    from dism_amd import _lib
    lib = _lib.load()
    limit = lib.dism_hard_forward_noalloc_max_bytes()
    assert limit == 256 << 20
    b, n, h, r, dv = 4, 16384, 16, 8, 64
    assert _lib.workspace_bytes(b, n, h, r, dv, 0) > limit
    null = ctypes.c_void_p(16)  # never dereferenced: the size check comes first
    status = lib.dism_hard_forward_noalloc(null, null, null, 0, null, null, null, null, n + 1, b,
                                           n, h, r, dv, null, 0, null, None, None, None)
    assert status != 0
    assert b"use dism_hard_forward with a caller workspace" in lib.dism_last_error()
