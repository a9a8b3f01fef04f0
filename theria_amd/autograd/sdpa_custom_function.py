"""SDPACustom: autograd-in-backward SDPA in pure PyTorch (theria/autograd/sdpa_custom_function.py:14-70).

The backward re-runs the forward under autograd and differentiates it with create_graph=True, so any
order of derivative is exact. It is the "custom" backend of sdpa_custom and a correctness reference,
not a fast path. jvp / hvp are explicit analytic helpers for tests.
"""

from __future__ import annotations

import math

import torch

from ..attention.reference_hvp_sdpa import sdpa_hvp
from ..attention.reference_jvp_sdpa import sdpa_jvp


def _attend(q, k, v, scale):
    return torch.matmul(torch.softmax(torch.matmul(q, k.transpose(-2, -1)) * scale, dim=-1), v)


class SDPACustom(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v):
        scale = 1.0 / math.sqrt(q.shape[-1])
        ctx.scale = scale
        ctx.save_for_backward(q, k, v)
        return _attend(q, k, v, scale)

    @staticmethod
    def backward(ctx, grad_out):
        q, k, v = ctx.saved_tensors
        with torch.enable_grad():
            out = _attend(q, k, v, ctx.scale)
        return torch.autograd.grad(out, (q, k, v), grad_out, retain_graph=True, create_graph=True, allow_unused=False)

    @staticmethod
    def hvp(q, k, v, dq, dk, dv):
        """Analytic HVP of sum(O) (reference_hvp_sdpa.sdpa_hvp)."""
        return sdpa_hvp(q, k, v, dq, dk, dv)

    @staticmethod
    def jvp(q, k, v, dq, dk, dv):
        """Analytic JVP accumulated in float64 (reference_jvp_sdpa.sdpa_jvp_reference)."""
        return sdpa_jvp(q, k, v, dq, dk, dv, 1.0 / math.sqrt(q.shape[-1]))


__all__ = ["SDPACustom"]
