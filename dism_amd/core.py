"""Differentiable hard core (autograd) on the MI355X library.

The hard-row part of the reference's training op: _MixedCore / dism_core_hybrid
(dism_v3/python/flash_dism/hard_training.py:343-409) add the hard output to the soft core's
output and, in backward, add backward_hard_recompute's FP32 gradients.  This build has no soft
core, so ``dism_core_hard`` is the all-hard specialisation: forward_hard in forward, the
hard backward in backward.  Unlike the reference default (which re-runs the forward in
backward), the forward's O(B*H*N) log2 normalizer and its carry boundary are saved, so the
backward does not recompute the forward.
"""
import torch

from .hard_backward import backward_hard
from .hard_forward import _forward_core


class HardCore(torch.autograd.Function):
    @staticmethod
    def forward(ctx, sq, sk, v, idx_q, idx_k, hard, tau):
        iq = idx_q.to(torch.int32).contiguous()
        ik = idx_k.to(torch.int32).contiguous()
        sq_c, sk_c, v_c = sq.contiguous(), sk.contiguous(), v.contiguous()
        hard_c, tau_c = hard.contiguous(), tau.detach().float().contiguous()
        out, lse2, lut, carry, strip, _, _, ws = _forward_core(
            sq_c, sk_c, v_c, iq, ik, hard_c, tau_c, None, None, False)
        ctx.save_for_backward(sq_c, sk_c, v_c, iq, ik, hard_c, tau_c, lse2, lut, ws,
                              *(() if carry is None else (carry,)))
        ctx.strip = strip
        ctx.has_carry = carry is not None
        return out

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, dout):
        saved = ctx.saved_tensors
        sq, sk, v, iq, ik, hard, tau, lse2, lut, ws = saved[:10]
        carry = saved[10] if ctx.has_carry else None
        dout = dout.to(sq.dtype).contiguous()
        state = dict(log_weights=lut, tau=tau, carry=carry, carry_strip=ctx.strip, workspace=ws)
        dsq, dsk, dv, dtau = backward_hard(sq, sk, v, dout, iq, ik, hard, lse2, state)
        return dsq, dsk, dv, None, None, None, dtau


def dism_core_hard(sq, sk, v, idx_q, idx_k, hard, tau):
    """Hard-only DISM core with autograd: O = hard readout; grads for sq, sk, v and tau.

    sq, sk [B,N,H,R], v [B,N,H,DV] (bf16 or f32), labels [B,H,N] int, hard [B,H] bool,
    tau [H] (natural-log match coefficient).  Returns O [B,N,H,DV] in the vectors' dtype.
    """
    return HardCore.apply(sq, sk, v, idx_q, idx_k, hard, tau)
