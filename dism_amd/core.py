"""Differentiable hard core (autograd, torch.compile) on the MI355X library.

The reference's training op is _MixedCore / dism_core_hybrid
(dism_v3/python/flash_dism/hard_training.py:343-409): the soft core's output plus the hard
output, and in backward the soft gradients plus backward_hard_recompute's FP32 gradients.  The
soft core skips hard rows (dism_v3/include/forward/producer.cuh:18), so on rows that are all
hard the op is exactly the hard core.  This build implements that part:

* ``hard_core`` / ``hard_core_backward`` -- torch.library custom operators (``dism_amd::``)
  with fake (meta) implementations and a registered autograd formula, so the op is opaque to
  torch.compile the way the reference registers its cores (flash_dism/compiler.py:143-181).
  Unlike the reference default (which re-runs the forward in backward), the forward's
  workspace and O(B*H*N) log2 normalizer are saved, so the backward does not recompute it.
* ``dism_core_hard(sq, sk, v, idx_q, idx_k, hard, tau)`` -- the hard core with autograd;
  soft rows give zero output and zero gradients.
* ``dism_core(q, k, sq, sk, v, q_lse, k_lse, idx_q, idx_k, direction, hard, rtau, *, ctas=0,
  _lse_preabsorbed=False)`` -- the reference's signature (flash_dism/backward.py:41); rows must
  all be hard (soft rows need the soft DISM core, which this build does not provide, and raise).
"""
import torch
from torch import Tensor

from . import _lib
from ._checks import DTYPE_CODE, check_ctas, require
from .hard_backward import backward_hard
from .hard_forward import _forward_core, _packed_forward_core, hard_dlog_weights
from .labels import vocab_labels_op
from .varlen import VarlenLayout, packed_backward


@torch.library.custom_op("dism_amd::hard_core", mutates_args=())
def hard_core(sq: Tensor, sk: Tensor, v: Tensor, idx_q: Tensor, idx_k: Tensor, hard: Tensor,
              tau: Tensor) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """Forward: (O in the vectors' dtype, lse2 fp32 [B,H,N], LUT fp32 [H,N+1], workspace)."""
    out, lse2, lut, _, _, _, _, ws = _forward_core(sq, sk, v, idx_q, idx_k, hard, tau, 0, None,
                                                   False)
    return out, lse2, lut, ws


@hard_core.register_fake
def _hard_core_fake(sq, sk, v, idx_q, idx_k, hard, tau):
    b, n, h, r = sq.shape
    dv = v.shape[3]
    nbytes = _lib.workspace_bytes(b, n, h, r, dv, DTYPE_CODE[sq.dtype])
    return (v.new_empty((b, n, h, dv)), sq.new_empty((b, h, n), dtype=torch.float32),
            sq.new_empty((h, n + 1), dtype=torch.float32),
            sq.new_empty((nbytes,), dtype=torch.uint8))


@torch.library.custom_op("dism_amd::hard_core_backward", mutates_args=())
def hard_core_backward(sq: Tensor, sk: Tensor, v: Tensor, dout: Tensor, idx_q: Tensor,
                       idx_k: Tensor, hard: Tensor, tau: Tensor, lse2: Tensor, lut: Tensor,
                       workspace: Tensor) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """Backward on the forward's workspace: (dSQ, dSK, dV, dtau), all fp32."""
    state = dict(log_weights=lut, tau=tau, carry=None, carry_strip=0, workspace=workspace)
    return tuple(backward_hard(sq, sk, v, dout.to(sq.dtype).contiguous(), idx_q, idx_k, hard,
                               lse2, state))


@hard_core_backward.register_fake
def _hard_core_backward_fake(sq, sk, v, dout, idx_q, idx_k, hard, tau, lse2, lut, workspace):
    f32 = dict(dtype=torch.float32)
    return (sq.new_empty(sq.shape, **f32), sk.new_empty(sk.shape, **f32),
            v.new_empty(v.shape, **f32), tau.new_empty(tau.shape, **f32))


def _setup_context(ctx, inputs, output):
    sq, sk, v, idx_q, idx_k, hard, tau = inputs
    _, lse2, lut, ws = output
    ctx.save_for_backward(sq, sk, v, idx_q, idx_k, hard, tau, lse2, lut, ws)


def _hard_core_autograd(ctx, dout, _dlse2, _dlut, _dws):
    sq, sk, v, idx_q, idx_k, hard, tau, lse2, lut, ws = ctx.saved_tensors
    dsq, dsk, dv, dtau = hard_core_backward(sq, sk, v, dout, idx_q, idx_k, hard, tau, lse2,
                                            lut, ws)
    return dsq, dsk, dv, None, None, None, dtau


hard_core.register_autograd(_hard_core_autograd, setup_context=_setup_context)


class _PackedHardCore(torch.autograd.Function):
    """Packed batch-1 hard core (VarlenLayout): forward keeps the workspace, LUT and log2
    normalizer; backward runs the packed backward on them (no recompute)."""

    @staticmethod
    def forward(ctx, sq, sk, v, iq, ik, hard, tau, layout):
        out, lse2, lut, _, _, ws = _packed_forward_core(sq, sk, v, iq, ik, hard, tau, layout,
                                                        None, False)
        ctx.layout = layout
        ctx.save_for_backward(sq, sk, v, iq, ik, hard, tau, lse2, lut, ws)
        return out

    @staticmethod
    def backward(ctx, dout):
        sq, sk, v, iq, ik, hard, tau, lse2, lut, ws = ctx.saved_tensors
        dlut = hard_dlog_weights(tau, lut.shape[1])
        dsq, dsk, dv, dtau = packed_backward(sq, sk, v, dout.to(sq.dtype).contiguous(), iq, ik,
                                             hard, lse2, lut, dlut, ctx.layout, workspace=ws)
        return dsq, dsk, dv, None, None, None, dtau, None


def dism_core_hard(sq, sk, v, idx_q, idx_k, hard, tau, *, layout=None):
    """Hard-only DISM core with autograd: O = hard readout; grads for sq, sk, v and tau.

    sq, sk [B,N,H,R], v [B,N,H,DV] (bf16 or f32), labels [B,H,N] int, hard [B,H] bool,
    tau [H] (natural-log match coefficient).  Returns O [B,N,H,DV] in the vectors' dtype.
    Soft rows give zero output and zero gradients.  ``layout`` (VarlenLayout) selects packed
    batch-1 execution with hard [training_rows, H].
    """
    iq = idx_q.to(torch.int32).contiguous()
    ik = idx_k.to(torch.int32).contiguous()
    if layout is not None:
        return _PackedHardCore.apply(sq.contiguous(), sk.contiguous(), v.contiguous(), iq, ik,
                                     hard.contiguous(), tau.float().contiguous(), layout)
    return hard_core(sq.contiguous(), sk.contiguous(), v.contiguous(), iq, ik, hard.contiguous(),
                     tau.float().contiguous())[0]


def dism_core(q, k, sq, sk, v, q_lse, k_lse, idx_q, idx_k, direction, hard, rtau, *,
              cu_seqlens=None, layout=None, ctas=0, hard_planner=None, _lse_preabsorbed=False,
              all_hard=None):
    """Differentiable core with the reference's signature (flash_dism/__init__.py:20-40,
    backward.py:41-54) for sequences that are all hard: O = hard output (the soft core skips
    hard rows), gradients for sq, sk, v and rtau; q, k, q_lse, k_lse receive zero gradients.
    Soft rows raise NotImplementedError (they need the soft core).  ``rtau`` is the natural-log
    coefficient, used as is (no softplus), as in the reference's hard path.  ``cu_seqlens`` or
    ``layout`` selects packed batch-1 execution (hard [training_rows, H]).

    The soft-row check reads ``hard`` on the host.  Inside torch.compile that read is not
    possible, so a compiled caller must assert ``all_hard=True`` (otherwise tracing raises);
    ``all_hard=True`` also skips the host read in eager mode.

    ``hard_planner``: the reference routes an explicit AsyncHardPlanner to its hybrid core
    (flash_dism/__init__.py:29-37), which plans the hard rows on the host.  This core plans
    every row on the device, so a planner object is accepted and not used; the result is
    the same hard output (soft rows still need the soft core, see dism_core_hybrid)."""
    packed = cu_seqlens is not None or layout is not None
    if packed:
        if ctas:
            raise ValueError("ctas is only supported for fixed-length execution")
        if cu_seqlens is not None:
            if layout is not None:
                raise ValueError("provide either layout or cu_seqlens, not both")
            layout = VarlenLayout.from_cu_seqlens(cu_seqlens, sq.shape[1])
    check_ctas(ctas)
    b, n, h = sq.shape[0], sq.shape[1], sq.shape[2]
    require(tuple(q.shape[:3]) == (b, n, h) and tuple(k.shape[:3]) == (b, n, h),
            "q/k must match sq/sk in [B,N,H]")
    require(tuple(q_lse.shape) == (b, h, n) and tuple(k_lse.shape) == (b, h, n),
            "q_lse/k_lse must be [B,H,N]")
    if packed:
        require(b == 1, "packed execution needs batch 1")
        require(isinstance(hard, torch.Tensor) and hard.dim() == 2 and hard.shape[1] == h,
                "hard must be contiguous bool [training_rows,H]; token-level masks are "
                "unsupported")
        require(direction.dim() == 2 and direction.shape[1] == h,
                "direction must be [training_rows,H]")
    else:
        require(tuple(direction.shape) == (b, h), "direction must be [B,H]")
        require(isinstance(hard, torch.Tensor) and tuple(hard.shape) == (b, h),
                "fixed hard must be [B,H]")
    if torch.compiler.is_compiling():
        if all_hard is not True:
            raise NotImplementedError(
                "dism_core under torch.compile cannot check the hard flags on the host: pass "
                "all_hard=True to assert that every row is hard (soft rows need the soft DISM "
                "core, which the MI355X hard core does not provide)")
    elif all_hard is not True and not bool(hard.all()):
        raise NotImplementedError(
            "soft rows need the soft DISM core, which the MI355X hard core does not provide")
    out = dism_core_hard(sq, sk, v, idx_q, idx_k, hard, rtau, layout=layout)
    return _SoftOperands.apply(out, q, k, q_lse, k_lse)


def dism_core_hybrid(q, k, sq, sk, v, lq, lk, iq, ik, direction, hard, tau, *, soft_core,
                     layout=None, ctas=0, _lse_preabsorbed=False):
    """The reference's mixed training core (_MixedCore / dism_core_hybrid,
    flash_dism/hard_training.py:343-409) with the soft part supplied by the caller: O = the
    soft core's output + the hard core's output, gradients the sum of both (the reference adds
    backward_hard_recompute's FP32 gradients for sq, sk, v and tau to the soft ones).

    ``soft_core(q, k, sq, sk, v, lq, lk, iq, ik, direction, hard, tau, layout=..., ctas=...,
    _lse_preabsorbed=...)`` must return the soft DISM output [B,N,H,DV] with autograd, zero on
    hard rows (the reference's soft core skips them, include/forward/producer.cuh:18); the soft
    DISM kernels are not part of this build.  The hard part is ``dism_core_hard``, which gives
    zero output and zero gradients on soft rows.  With an empty hard side (sq.shape[1] == 0)
    the result is the soft output alone, as in the reference."""
    if not callable(soft_core):
        raise TypeError("soft_core must be a callable returning the soft DISM output")
    if layout is not None and ctas:
        raise ValueError("ctas is only supported for fixed-length execution")
    soft = soft_core(q, k, sq, sk, v, lq, lk, iq, ik, direction, hard, tau, layout=layout,
                     ctas=ctas, _lse_preabsorbed=_lse_preabsorbed)
    if sq.shape[1] == 0:
        return soft
    hard_out = dism_core_hard(sq, sk, v, iq, ik, hard, tau, layout=layout)
    return soft + hard_out.to(soft.dtype)


def voc_dism(q, k, sq, sk, v, q_vocab, k_vocab, rtau, *, direction, hard, cu_seqlens=None,
             layout=None, ctas=0, beta=1.0, hard_planner=None, all_hard=None):
    """The reference's vocabulary entry (flash_dism/__init__.py:43-56, voc.py:7-40) for rows
    that are all hard: q, k bf16 [B,N,H,D] are labelled by the exact codebook argmax against
    q_vocab / k_vocab ([H,V,D] or shared [V,D], D in {32, 64, 128}; first index on ties) --
    the indices the reference's interpolation kernel returns for its hard rows
    (flash_dism/emb_kernel.py:96-156, reference oracle dism_v3_ref.py:159-162) -- and the
    hard core runs on sq, sk, v with those labels (dism_core).  The interpolated embeddings
    and their normalizers feed only the soft core, so for hard rows q, k, q_vocab and k_vocab
    receive zero gradients and ``beta`` (the soft gate's vocabulary temperature, a positive
    finite scalar or 0-dim tensor) does not change the result.  Soft rows raise
    NotImplementedError; under torch.compile pass ``all_hard=True`` (see dism_core).
    ``hard_planner`` is accepted and not used, as in dism_core."""
    if not torch.compiler.is_compiling():
        bv = float(beta.detach().item()) if isinstance(beta, torch.Tensor) else float(beta)
        require(bv > 0.0 and bv != float("inf"), "beta must be a positive finite temperature")
    require(q.dim() == 4 and tuple(k.shape) == tuple(q.shape), "q and k must be [B,N,H,D]")
    idx_q = vocab_labels_op(q.detach().contiguous(), q_vocab.detach().contiguous())
    idx_k = vocab_labels_op(k.detach().contiguous(), k_vocab.detach().contiguous())
    b, n, h = sq.shape[0], sq.shape[1], sq.shape[2]
    lse = torch.zeros((b, h, n), dtype=torch.float32, device=sq.device)
    out = dism_core(q, k, sq, sk, v, lse, lse, idx_q, idx_k, direction, hard, rtau,
                    cu_seqlens=cu_seqlens, layout=layout, ctas=ctas, all_hard=all_hard)
    return _SoftOperands.apply(out, q_vocab, k_vocab, lse, lse)


class _SoftOperands(torch.autograd.Function):
    """Identity on O; zero gradients for the soft core's operands (q, k, q_lse, k_lse), which
    all-hard rows do not read."""

    @staticmethod
    def forward(ctx, out, q, k, q_lse, k_lse):
        ctx.save_for_backward(q, k, q_lse, k_lse)
        return out.view_as(out)

    @staticmethod
    def backward(ctx, grad):
        return (grad, *(torch.zeros_like(t) if ctx.needs_input_grad[i + 1] else None
                        for i, t in enumerate(ctx.saved_tensors)))
