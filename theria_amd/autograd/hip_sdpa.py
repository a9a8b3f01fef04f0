"""autograd wiring of the HIP SDPA operator: exact first and second order, forward-mode JVP.

SDPAOp            O = softmax(scale Q K^T) V (optional causal mask); forward kernel, saves (O, lse).
  .backward       -> SDPABackwardOp.apply(...), itself an autograd.Function, so gradients computed
                     with create_graph=True stay differentiable (MAML's full second order).
  .jvp            -> the frozen-stats JVP kernel (torch.func.jvp / forward-mode AD).
SDPABackwardOp    (dQ, dK, dV) from the backward kernel; its backward is the explicit double-backward
                  kernel set (G_Q, G_K, G_V, G_dO).

The reference's Triton path returns backward outputs with no graph (theria/attention/triton_qk.py:
379-387), which silently drops attention's second-order terms under MAML create_graph=True. Here the
second-order terms are explicit kernels. Third-order derivatives are not implemented: if a graph built
with create_graph=True through the double backward is differentiated again, a RuntimeError is raised
instead of silently returning graph-less tensors.
"""

from __future__ import annotations

import torch

from .. import _ops


class _ThirdOrderBarrier(torch.autograd.Function):
    """Identity on the double-backward outputs whose own backward refuses to run."""

    @staticmethod
    def forward(ctx, n_out: int, *tensors):
        ctx.n_out = n_out
        return tuple(t.clone() for t in tensors[:n_out])

    @staticmethod
    def backward(ctx, *grads):
        raise RuntimeError(
            "theria_amd HIP SDPA: third-order derivatives through attention are not implemented "
            "(the double-backward kernels are not themselves differentiable)"
        )


class SDPABackwardOp(torch.autograd.Function):
    """(q, k, v, o, lse, dout) -> (dq, dk, dv). o and lse are treated as constants of q, k, v."""

    @staticmethod
    def forward(ctx, q, k, v, o, lse, dout, scale, causal):
        dq, dk, dv, delta = _ops.bwd(q, k, v, o, lse, dout, scale, causal)
        ctx.save_for_backward(q, k, v, o, lse, dout, delta)
        ctx.scale = scale
        ctx.causal = causal
        return dq, dk, dv

    @staticmethod
    def backward(ctx, gq, gk, gv):
        q, k, v, o, lse, dout, delta = ctx.saved_tensors
        if gq is None and gk is None and gv is None:
            return None, None, None, None, None, None, None, None
        g_q, g_k, g_v, g_do = _ops.bwd_bwd(q, k, v, o, dout, lse, delta, gq, gk, gv, ctx.scale, ctx.causal)
        g_do = g_do.to(dout.dtype)
        if torch.is_grad_enabled():
            anchors = [t for t in (q, k, v, dout, gq, gk, gv) if t is not None and t.requires_grad]
            if anchors:
                g_q, g_k, g_v, g_do = _ThirdOrderBarrier.apply(4, g_q, g_k, g_v, g_do, *anchors)
        return g_q, g_k, g_v, None, None, g_do, None, None


class SDPAOp(torch.autograd.Function):
    """(q, k, v, scale, causal, out_fp32) -> (o, lse)."""

    @staticmethod
    def forward(q, k, v, scale, causal, out_fp32):
        o, lse, _, _ = _ops.fwd(q, k, v, scale, causal, out_fp32=out_fp32)
        return o, lse

    @staticmethod
    def setup_context(ctx, inputs, output):
        q, k, v, scale, causal, out_fp32 = inputs
        o, lse = output
        ctx.scale = scale
        ctx.causal = causal
        ctx.mark_non_differentiable(lse)
        ctx.save_for_backward(q, k, v, o, lse)
        ctx.save_for_forward(q, k, v, o, lse)

    @staticmethod
    def backward(ctx, do, _dlse):
        if do is None:
            return None, None, None, None, None, None
        q, k, v, o, lse = ctx.saved_tensors
        dq, dk, dv = SDPABackwardOp.apply(q, k, v, o.detach(), lse, do, ctx.scale, ctx.causal)
        return dq, dk, dv, None, None, None

    @staticmethod
    def jvp(ctx, tq, tk, tv, _ts, _tc, _tf):
        q, k, v, o, lse = ctx.saved_tensors
        to = _ops.jvp(q, k, v, o, lse, tq, tk, tv, ctx.scale, ctx.causal)
        if to.dtype != o.dtype:
            to = to.to(o.dtype)
        return to, None


def hip_sdpa(q, k, v, *, causal: bool = False, scale: float | None = None, out_fp32: bool = False):
    """Differentiable (to second order) SDPA through the HIP kernels. Returns O only."""
    if scale is None:
        scale = _ops.default_scale(q.shape[-1])
    o, _ = SDPAOp.apply(q, k, v, float(scale), bool(causal), bool(out_fp32))
    return o


def hip_sdpa_with_lse(q, k, v, *, causal: bool = False, scale: float | None = None):
    """(O, lse) with lse = log-sum-exp of the scaled scores per query row (not differentiable)."""
    if scale is None:
        scale = _ops.default_scale(q.shape[-1])
    return SDPAOp.apply(q, k, v, float(scale), bool(causal), False)


__all__ = ["SDPAOp", "SDPABackwardOp", "hip_sdpa", "hip_sdpa_with_lse"]
