"""Fused SDPA forward on the HIP kernels, under the reference's public names.

triton_sdpa_fused / TritonFusedSDPAFunction / triton_sdpa_fused_autograd keep the signatures and
return conventions of theria/attention/triton_qk.py:307-391 (float32 O; optional saved stats m, l), but
run the gfx950 kernels; the names are kept only so callers work unchanged. Unlike the reference's
Function, the autograd path here is exact to second order (its backward is itself differentiable).
Widened contract: D <= 128 (reference: D <= 64) and any strides with a contiguous last dimension.
"""

from __future__ import annotations

import torch

from .. import _ops
from ..autograd.hip_sdpa import SDPABackwardOp, hip_sdpa


def _fused_guards(q, k, v) -> None:
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise AssertionError("fused SDPA requires GPU tensors")
    B, H, T, D = q.shape
    _, _, M, Dk = k.shape
    _, _, Mv, Dv = v.shape
    if D != Dk:
        raise AssertionError("q and k head dims differ")
    if M != Mv:
        raise AssertionError("k and v lengths differ")
    if Dv != D:
        raise AssertionError("fused path requires Dv == D")
    if D > _ops.MAX_HEAD_DIM:
        raise AssertionError(f"fused kernel supports D <= {_ops.MAX_HEAD_DIM}")


def triton_sdpa_fused(q, k, v, return_stats: bool = False):
    """Fused forward: O (float32) or (O, m, l) with m = row max of scaled scores, l = sum exp(S - m)."""
    _fused_guards(q, k, v)
    o, _, m, l = _ops.fwd(q, k, v, _ops.default_scale(q.shape[-1]), False, out_fp32=True, stats=return_stats)
    if return_stats:
        return o, m, l
    return o


class TritonFusedSDPAFunction(torch.autograd.Function):
    """The reference's autograd.Function (triton_qk.py:372-391): ``TritonFusedSDPAFunction.apply(q, k, v)``
    returns float32 O. Its backward runs the backward kernels through SDPABackwardOp, which is itself
    differentiable (double backward on the second-order kernels), and its jvp the JVP kernel; the
    reference's backward runs under no_grad and drops the second-order terms."""

    @staticmethod
    def forward(q, k, v):
        _fused_guards(q, k, v)
        return _ops.fwd(q, k, v, _ops.default_scale(q.shape[-1]), False, out_fp32=True)[:2]

    @staticmethod
    def setup_context(ctx, inputs, output):
        q, k, v = inputs
        o, lse = output
        ctx.scale = _ops.default_scale(q.shape[-1])
        ctx.mark_non_differentiable(lse)
        ctx.save_for_backward(q, k, v, o, lse)
        ctx.save_for_forward(q, k, v, o, lse)

    @staticmethod
    def backward(ctx, do, _dlse):
        if do is None:
            return None, None, None
        q, k, v, o, lse = ctx.saved_tensors
        dq, dk, dv = SDPABackwardOp.apply(q, k, v, o.detach(), lse, do, ctx.scale, False)
        return dq, dk, dv

    @staticmethod
    def jvp(ctx, tq, tk, tv):
        q, k, v, o, lse = ctx.saved_tensors
        return _ops.jvp(q, k, v, o, lse, tq, tk, tv, ctx.scale, False, normalize=True).float(), None

    @classmethod
    def apply(cls, q, k, v):  # O only, as the reference returns
        return super().apply(q, k, v)[0]


def triton_sdpa_fused_autograd(q, k, v):
    return TritonFusedSDPAFunction.apply(q, k, v)


# Native names.
sdpa_fused = triton_sdpa_fused

__all__ = ["triton_sdpa_fused", "TritonFusedSDPAFunction", "triton_sdpa_fused_autograd", "sdpa_fused", "hip_sdpa"]
