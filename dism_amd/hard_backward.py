"""Hard backward on the MI355X library.

Mirrors dism_v3/python/flash_dism/hard_backward.py:7-59 (backward_hard,
backward_hard_recompute): same names, argument meaning and RuntimeError texts.

Differences by design: all four gradients are returned in FP32 (the reference stores dSK/dV
as BF16, whose rounding alone is ~2e-3 relative), and the result is deterministic -- every
gradient element is accumulated by one lane in a fixed order and dtau is reduced in a fixed
order (the reference uses FP32 global atomics for dSQ and the tau moments).
"""
import math

import torch

from . import _lib
from ._checks import (DTYPE_CODE, check_ctas, check_graph_choice, check_labels, check_layout,
                      check_tensor, check_vectors, require)
from .hard_forward import (_forward_core, _packed_forward_core, hard_dlog_weights,
                           prepare_workspace)
from .varlen import packed_backward


def _stream(t):
    return torch.cuda.current_stream(t.device).cuda_stream


@torch.no_grad()
def backward_hard(sq, sk, v, dout, idx_q, idx_k, hard, normalizer, state, *, layout=None,
                  ctas=0, _graph_choice=None):
    """Return dSQ, dSK, dV, d(tau) (all FP32) for sequence-hard rows; soft rows get zeros.

    ``state`` comes from forward_hard(..., save_state=True) on the same inputs; ``normalizer``
    is that call's log2 normalizer.  tau is the natural-log coefficient.  ``layout`` selects
    packed batch-1 execution (hard [training_rows, H]); soft training rows get zeros and dtau
    sums the hard documents.
    """
    check_ctas(ctas)
    check_layout(layout)
    check_graph_choice(_graph_choice)
    if layout is not None:
        return _packed_backward_hard(sq, sk, v, dout, idx_q, idx_k, hard, normalizer, state,
                                     layout)
    b, n, h, r, dv, dt = check_vectors(sq, sk, v, extra=(("dO", dout),))
    check_labels(idx_q, idx_k, b, h, n, sq.device)
    check_tensor(hard, torch.bool, (b, h), "sequence hard flags", sq.device)
    check_tensor(normalizer, torch.float32, (b, h, n), "log2 normalizer", sq.device)
    require(isinstance(state, dict) and "log_weights" in state, "invalid hard forward state")
    lut = state["log_weights"]
    check_tensor(lut, torch.float32, (h, n + 1), "log weight LUT", sq.device)
    if state.get("carry") is not None:
        carry, strip = state["carry"], int(state["carry_strip"])
        check_tensor(carry, torch.int32, (b, h, (n - 1) // strip, n), "integer boundary",
                     sq.device)
    elif _given(state, "boundary"):
        # a boundary handed in by the caller (e.g. a reference-format state) bounds the walks;
        # a lazily offered one is not computed for this
        carry, strip = state["boundary"], 32
        check_tensor(carry, torch.int32, (b, h, (n - 1) // 32, n), "integer boundary", sq.device)
    else:
        carry, strip = None, 0
    tau = _state_tau(state, lut)
    dlut = hard_dlog_weights(tau, n + 1)
    ws = state.get("workspace")
    if ws is None or ws.numel() < _lib.workspace_bytes(b, n, h, r, dv, DTYPE_CODE[dt]):
        ws = prepare_workspace(sq, sk, v, idx_q, idx_k)
    dsq = torch.empty((b, n, h, r), dtype=torch.float32, device=sq.device)
    dsk = torch.empty((b, n, h, r), dtype=torch.float32, device=sq.device)
    dvv = torch.empty((b, n, h, dv), dtype=torch.float32, device=sq.device)
    rowtau = torch.empty((b, h, n), dtype=torch.float32, device=sq.device)
    dtau = torch.empty((h,), dtype=torch.float32, device=sq.device)
    with torch.cuda.device(sq.device):
        _lib.call("dism_hard_backward", sq.data_ptr(), sk.data_ptr(), v.data_ptr(),
                  dout.data_ptr(), DTYPE_CODE[dt], idx_q.data_ptr(), idx_k.data_ptr(),
                  hard.data_ptr(), 0 if carry is None else carry.data_ptr(), strip,
                  lut.data_ptr(), dlut.data_ptr(), n + 1, normalizer.data_ptr(), b, n, h, r,
                  dv, ws.data_ptr(), ws.numel(), dsq.data_ptr(), dsk.data_ptr(),
                  dvv.data_ptr(), rowtau.data_ptr(), dtau.data_ptr(), _stream(sq))
    return dsq, dsk, dvv, dtau


def _given(state, key):
    materialized = getattr(state, "materialized", None)
    if materialized is not None:
        return materialized(key) and state.get(key) is not None
    return state.get(key) is not None


def _state_tau(state, lut):
    tau = state.get("tau")
    if tau is None:  # reference state: recover tau from LUT[:,1] = tau / ln 2
        tau = (lut[:, 1].double() * math.log(2.0)).float().contiguous()
    return tau


def _packed_backward_hard(sq, sk, v, dout, idx_q, idx_k, hard, normalizer, state, layout):
    require(isinstance(state, dict) and "log_weights" in state, "invalid hard forward state")
    lut = state["log_weights"]
    require(isinstance(lut, torch.Tensor) and lut.dim() == 2,
            "log weight LUT: invalid device, dtype, shape or stride")
    dlut = hard_dlog_weights(_state_tau(state, lut), lut.shape[1])
    ws = state.get("workspace") if state.get("layout") is layout else None
    return packed_backward(sq, sk, v, dout, idx_q, idx_k, hard, normalizer, lut, dlut, layout,
                           workspace=ws)


@torch.no_grad()
def backward_hard_recompute(sq, sk, v, dout, iq, ik, hard, tau, *, layout=None, ctas=0,
                            _graph_choice=None):
    """Backward with no retained state: recompute the forward normalizer, then backward.
    Returns dict(sq_vec, sk_vec, v, rtau)."""
    check_layout(layout)
    a, b_, c, do = [x.contiguous() for x in (sq, sk, v, dout)]
    q, k = [x.to(torch.int32).contiguous() for x in (iq, ik)]
    check_ctas(ctas)
    check_graph_choice(_graph_choice)
    if layout is not None:
        # reference host checks of the packed fallback (hard_backward.py:41-51)
        n = sq.shape[1]
        if sq.shape[0] != 1 or hard.ndim != 2 or n % hard.shape[0] or layout.tokens != n:
            raise ValueError("invalid packed fallback rows")
        row_n = n // hard.shape[0]
        if any(start // row_n != (start + length - 1) // row_n
               for start, length in layout.spans()):
            raise ValueError("document crosses original hard row")
        flags, t = hard.contiguous(), tau.contiguous()
        _, norm, lut, _, _, ws = _packed_forward_core(a, b_, c, q, k, flags, t, layout, None,
                                                      False)
        dlut = hard_dlog_weights(t, lut.shape[1])
        result = packed_backward(a, b_, c, do, q, k, flags, norm, lut, dlut, layout,
                                 workspace=ws)
        return dict(zip(("sq_vec", "sk_vec", "v", "rtau"), result))
    _, norm, lut, carry, strip, _, _, ws = _forward_core(a, b_, c, q, k, hard.contiguous(),
                                                         tau.contiguous(), None, None, False)
    state = dict(log_weights=lut, tau=tau.contiguous(), carry=carry, carry_strip=strip,
                 workspace=ws)
    result = backward_hard(a, b_, c, do, q, k, hard.contiguous(), norm, state, ctas=ctas,
                           _graph_choice=_graph_choice)
    return dict(zip(("sq_vec", "sk_vec", "v", "rtau"), result))
