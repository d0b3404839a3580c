"""Hard-only forward on the MI355X library.

Mirrors dism_v3/python/flash_dism/hard_forward.py:9-47 (hard_log_weights, hard_readout,
forward_hard): same names, argument meaning, defaults and RuntimeError texts.

Differences by design (the reference's chain is summary -> chunk -> LUT -> readout with an
O(B*H*N^2/32) int32 boundary in between):
  * forward_hard computes the LUT and runs the readout directly; match lengths of the
    (rare) pairs with L >= 2 are recomputed from the labels by a suffix walk inside the
    readout.  ``carry_strip`` S > 0 (default 0 = off, env DISM_HARD_CARRY_STRIP) adds a
    composed boundary of strip height S (B*H*N^2/S int32) that bounds each walk by S steps,
    for inputs with very long repeats.  With save_state=True the state also offers the
    reference's strip-32 summary/boundary, computed when first read (callers that inspect
    them still work; the backward does not read them);
  * fp32 vectors are accepted besides bf16 (all vectors share one dtype);
  * ``return_matches=True`` additionally returns, per query, the longest match length and
    its key index (ties -> most recent key, -1 if none).
"""
import os

import torch

from . import _lib
from ._checks import (DTYPE_CODE, check_ctas, check_graph_choice, check_hard, check_labels,
                      check_layout, check_tensor, check_vectors, require)
from .summary import hard_boundary, hard_chunk_scan, summarize_hard
from .varlen import VarlenLayout, packed_readout

DEFAULT_CARRY_STRIP = int(os.environ.get("DISM_HARD_CARRY_STRIP", "0"))


def _stream(t):
    return torch.cuda.current_stream(t.device).cuda_stream


@torch.no_grad()
def hard_log_weights(tau, max_length, *, _graph_choice=None):
    """Fresh FP32 log2 geometric-sum table [H, max_length+1]; entry 0 is -1e6."""
    require(isinstance(tau, torch.Tensor) and tau.is_cuda and tau.dtype == torch.float32 and
            tau.dim() == 1 and tau.is_contiguous() and 0 < tau.numel() <= 65535,
            "tau must be contiguous CUDA FP32 [H]")
    require(isinstance(max_length, int) and max_length > 0 and max_length % 256 == 0,
            "LUT maximum length must be positive and 256-aligned")
    check_graph_choice(_graph_choice)
    out = torch.empty((tau.numel(), max_length + 1), dtype=torch.float32, device=tau.device)
    with torch.cuda.device(tau.device):
        _lib.call("dism_hard_log_weights", tau.data_ptr(), tau.numel(), max_length,
                  out.data_ptr(), _stream(tau))
    return out


@torch.no_grad()
def hard_dlog_weights(tau, stride):
    """FP32 [H, stride] natural-tau derivative of ln W_L (entry 0 is 0)."""
    require(isinstance(tau, torch.Tensor) and tau.is_cuda and tau.dtype == torch.float32 and
            tau.dim() == 1 and tau.is_contiguous() and 0 < tau.numel() <= 65535,
            "tau must be contiguous CUDA FP32 [H]")
    out = torch.empty((tau.numel(), stride), dtype=torch.float32, device=tau.device)
    with torch.cuda.device(tau.device):
        _lib.call("dism_hard_dlog_weights", tau.data_ptr(), tau.numel(), stride,
                  out.data_ptr(), _stream(tau))
    return out


def prepare_workspace(sq, sk, v, idx_q, idx_k):
    """Allocate the workspace and fill it for these labels: the combined label order of
    queries and keys, the bigram orders of each side and the bigram-pair plans.  Returns the
    uint8 workspace tensor."""
    b, n, h, r, dv, dt = check_vectors(sq, sk, v)
    nbytes = _lib.workspace_bytes(b, n, h, r, dv, DTYPE_CODE[dt])
    ws = torch.empty((nbytes,), dtype=torch.uint8, device=sq.device)
    with torch.cuda.device(sq.device):
        _lib.call("dism_hard_prepare", sq.data_ptr(), sk.data_ptr(), v.data_ptr(),
                  DTYPE_CODE[dt], idx_q.data_ptr(), idx_k.data_ptr(), b, n, h, r, dv,
                  ws.data_ptr(), nbytes, _stream(sq))
    return ws


def row_modes(workspace, sq, v):
    """Row modes [B,H] int32 of a workspace prepared for vectors shaped like sq/v: 0 sparse,
    1 dense (direct tile kernels), 2 sparse with strip-bounded walks, 3 dense level rows,
    4 dense prefix rows (every label with one predecessor label)."""
    b, n, h, r = sq.shape
    dv = v.shape[3]
    out = torch.empty((b, h), dtype=torch.int32, device=workspace.device)
    with torch.cuda.device(workspace.device):
        _lib.call("dism_hard_row_modes", workspace.data_ptr(), workspace.numel(), b, n, h, r,
                  dv, out.data_ptr(), _stream(workspace))
    return out


def _readout(sq, sk, v, idx_q, idx_k, hard, boundary, strip, log_weights, out_dtype,
             matches, workspace=None):
    b, n, h, r, dv, dt = check_vectors(sq, sk, v)
    check_labels(idx_q, idx_k, b, h, n, sq.device)
    check_hard(hard, b, h, sq.device)
    require(isinstance(log_weights, torch.Tensor) and log_weights.device == sq.device and
            log_weights.dtype == torch.float32 and log_weights.dim() == 2 and
            log_weights.shape[0] == h and log_weights.is_contiguous(),
            "invalid hard log-weight table")
    require(log_weights.shape[1] > n, "hard log-weight table is too short")
    if boundary is not None:
        check_tensor(boundary, torch.int32, (b, h, (n - 1) // strip, n), "hard boundary",
                     sq.device)
    entry = "dism_hard_readout"
    if workspace is None:  # prepare and read out in one call (the prepare's halves overlap)
        nbytes = _lib.workspace_bytes(b, n, h, r, dv, DTYPE_CODE[dt])
        workspace = torch.empty((nbytes,), dtype=torch.uint8, device=sq.device)
        entry = "dism_hard_forward"
    out = torch.empty((b, n, h, dv), dtype=out_dtype, device=sq.device)
    lse2 = torch.empty((b, h, n), dtype=torch.float32, device=sq.device)
    lmax = jarg = None
    if matches:
        lmax = torch.empty((b, h, n), dtype=torch.int32, device=sq.device)
        jarg = torch.empty((b, h, n), dtype=torch.int32, device=sq.device)
    ptr = lambda t: 0 if t is None else t.data_ptr()  # noqa: E731
    with torch.cuda.device(sq.device):
        _lib.call(entry, sq.data_ptr(), sk.data_ptr(), v.data_ptr(),
                  DTYPE_CODE[dt], idx_q.data_ptr(), idx_k.data_ptr(), hard.data_ptr(),
                  ptr(boundary), strip if boundary is not None else 0, log_weights.data_ptr(),
                  log_weights.shape[1], b, n, h, r, dv, workspace.data_ptr(),
                  workspace.numel(), out.data_ptr(), DTYPE_CODE[out_dtype], lse2.data_ptr(),
                  ptr(lmax), ptr(jarg), _stream(sq))
    return out, lse2, lmax, jarg, workspace


@torch.no_grad()
def hard_readout(sq, sk, v, idx_q, idx_k, hard, boundary, log_weights, *, layout=None, ctas=0,
                 _graph_choice=None):
    """Fused hard matching/normalization/readout with integer incoming boundaries.

    SQ/SK/V: contiguous BF16 (or FP32) BNHD; labels: int32 BHN; hard: sequence bool [B,H];
    boundary: the strip-32 composed boundary [B,H,(N-1)//32,N] of these labels (or None:
    lengths are then recomputed from the labels alone).  Returns output BNHD in the vectors'
    dtype and the FP32 log2 normalizer BHN.  Soft sequences give zero output/statistics.
    """
    check_ctas(ctas)
    check_layout(layout)
    check_graph_choice(_graph_choice)
    if layout is not None:
        # the packed readout recomputes lengths from the labels; the boundary is validated
        check_tensor(boundary, torch.int32, (layout.forward_elements * sq.shape[2],),
                     "packed hard boundary", sq.device)
        out, lse2, _, _, _ = packed_readout(sq, sk, v, idx_q, idx_k, hard, log_weights, layout,
                                            sq.dtype, False)
        return out, lse2
    out, lse2, _, _, _ = _readout(sq, sk, v, idx_q, idx_k, hard, boundary, 32, log_weights,
                                  sq.dtype, False)
    return out, lse2


def _packed_forward_core(sq, sk, v, idx_q, idx_k, hard, tau, layout, out_dtype, matches):
    """Packed LUT + readout; returns (out, lse2, lut, lmax, jarg, workspace)."""
    b, n, h, _, _, dt = check_vectors(sq, sk, v)
    require(isinstance(tau, torch.Tensor) and tau.is_cuda and tau.dtype == torch.float32 and
            tau.shape == (h,) and tau.is_contiguous(), "tau must be contiguous CUDA FP32 [H]")
    require(isinstance(layout, VarlenLayout), "layout must be a VarlenLayout")
    lut = hard_log_weights(tau, layout.longest)
    out, lse2, lmax, jarg, ws = packed_readout(sq, sk, v, idx_q, idx_k, hard, lut, layout,
                                               out_dtype or dt, matches)
    return out, lse2, lut, lmax, jarg, ws


def _forward_core(sq, sk, v, idx_q, idx_k, hard, tau, carry_strip, out_dtype, matches):
    """LUT + (optional carry boundary) + readout; returns (out, lse2, lut, carry, strip,
    lmax, jarg, workspace)."""
    b, n, h, _, _, dt = check_vectors(sq, sk, v)
    check_labels(idx_q, idx_k, b, h, n, sq.device)
    check_hard(hard, b, h, sq.device)
    require(isinstance(tau, torch.Tensor) and tau.is_cuda and tau.dtype == torch.float32 and
            tau.shape == (h,) and tau.is_contiguous(), "tau must be contiguous CUDA FP32 [H]")
    strip = DEFAULT_CARRY_STRIP if carry_strip is None else int(carry_strip)
    lut = hard_log_weights(tau, n)
    carry = None
    if strip > 0 and (n - 1) // strip > 0:
        carry = hard_boundary(idx_q, idx_k, hard, strip=strip, fill_all=False)
    out, lse2, lmax, jarg, ws = _readout(sq, sk, v, idx_q, idx_k, hard, carry, strip, lut,
                                         out_dtype or dt, matches)
    return out, lse2, lut, carry, strip, lmax, jarg, ws


class _LazyState(dict):
    """forward_hard's state: the reference-format strip-32 summary and boundary
    (O(B*H*N^2/32) int32 each) are computed on first access only; the backward here does not
    need them."""

    def __init__(self, lazy, **items):
        super().__init__(**items)
        self._lazy = dict(lazy)

    def _fill(self, key):
        if key in self._lazy and not dict.__contains__(self, key):
            dict.__setitem__(self, key, self._lazy.pop(key)())

    def __getitem__(self, key):
        self._fill(key)
        return dict.__getitem__(self, key)

    def get(self, key, default=None):
        self._fill(key)
        return dict.get(self, key, default)

    def __contains__(self, key):
        return key in self._lazy or dict.__contains__(self, key)

    def keys(self):
        return list(dict.keys(self)) + [k for k in self._lazy if not dict.__contains__(self, k)]

    def items(self):
        for k in self._lazy.copy():
            self._fill(k)
        return dict.items(self)

    def materialized(self, key):
        return dict.__contains__(self, key)


@torch.no_grad()
def forward_hard(sq, sk, v, idx_q, idx_k, hard, tau, *, layout=None, ctas=0, save_state=False,
                 _graph_choice=None, carry_strip=None, return_matches=False, out_dtype=None):
    """Complete standalone hard contribution: LUT and fused readout.

    Returns (O, lse2) or, with save_state, (O, lse2, dict(summary, boundary, log_weights,
    tau, strip, carry, carry_strip, workspace)); with return_matches a further
    dict(length, index).  ``layout`` (a VarlenLayout) selects packed batch-1 execution: B = 1,
    hard [training_rows, H], documents never matched against each other; the LUT then covers
    the longest document and the saved summary/boundary use the reference's flat packed
    format.
    O has the vectors' dtype unless out_dtype is given.
    """
    check_ctas(ctas)
    check_layout(layout)
    check_graph_choice(_graph_choice)
    if layout is not None:
        out, lse2, lut, lmax, jarg, ws = _packed_forward_core(
            sq, sk, v, idx_q, idx_k, hard, tau, layout, out_dtype, return_matches)
        result = [out, lse2]
        if save_state:
            result.append(_LazyState(
                {"summary": lambda: summarize_hard(idx_q, idx_k, hard, layout=layout),
                 "boundary": lambda: hard_chunk_scan(
                     summarize_hard(idx_q, idx_k, hard, layout=layout), layout=layout,
                     heads=sq.shape[2])},
                log_weights=lut, tau=tau, strip=32, carry=None, carry_strip=0, workspace=ws,
                layout=layout))
        if return_matches:
            result.append(dict(length=lmax, index=jarg))
        return tuple(result)
    out, lse2, lut, carry, strip, lmax, jarg, ws = _forward_core(
        sq, sk, v, idx_q, idx_k, hard, tau, carry_strip, out_dtype, return_matches)
    result = [out, lse2]
    if save_state:
        result.append(_LazyState(
            {"summary": lambda: summarize_hard(idx_q, idx_k, hard),
             "boundary": lambda: hard_chunk_scan(summarize_hard(idx_q, idx_k, hard))},
            log_weights=lut, tau=tau, strip=32, carry=carry, carry_strip=strip, workspace=ws))
    if return_matches:
        result.append(dict(length=lmax, index=jarg))
    return tuple(result)
