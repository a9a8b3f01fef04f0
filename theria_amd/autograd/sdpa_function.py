"""theria.sdpa: the opaque pure-PyTorch SDPA Function (theria/autograd/sdpa_function.py:6-44).

Its backward recomputes the reference forward under autograd and returns plain gradients, so it
supports first-order gradients only: double backward through it fails and forward-mode AD is not
implemented. That boundary is part of theria's contract (pinned by the reference's
tests/test_sdpa_hvp.py:4-34 and tests/test_attention_boundary.py:96-151) and is kept unchanged.
"""

from __future__ import annotations

import torch
from torch.autograd import Function

from ..attention.reference_attention import sdpa_reference


def sdpa(q, k, v):
    """Public SDPA entry point: (B,H,T,D) inputs -> (B,H,T,D) output, first-order differentiable."""
    return SDPAFunction.apply(q, k, v)


class SDPAFunction(Function):
    @staticmethod
    def forward(ctx, q, k, v):
        ctx.save_for_backward(q, k, v)
        return sdpa_reference(q, k, v)

    @staticmethod
    def backward(ctx, grad_out):
        saved = ctx.saved_tensors
        leaves = [t.detach().requires_grad_(True) for t in saved]
        with torch.enable_grad():
            out = sdpa_reference(*leaves)
        # create_graph stays False: the returned gradients carry no graph (the pinned boundary).
        return torch.autograd.grad(out, leaves, grad_out, retain_graph=False, allow_unused=False)


__all__ = ["sdpa", "SDPAFunction"]
