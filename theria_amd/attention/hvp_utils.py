"""Finite-difference HVP over the explicit VJP (theria/attention/hvp_utils.py:17-49 in the reference).

hvp_fd_vjp(q, k, v, dq, dk, dv, eps) central-differences the explicit gradient of L = sum(O), with
the forward statistics recomputed at each perturbed point (the true function, not the frozen-stats
one). Kept as a sanity utility; the exact HVP comes from double backward through SDPAOp.
"""

from __future__ import annotations

import torch

from .. import _ops


def _explicit_grads_sum(q, k, v):
    """Gradients of sum(O) with respect to q, k, v through the HIP forward + backward."""
    scale = _ops.default_scale(q.shape[-1])
    o, lse, _, _ = _ops.fwd(q, k, v, scale, False, out_fp32=True)
    dout = torch.ones(o.shape, dtype=q.dtype, device=q.device)
    dq, dk, dv, _ = _ops.bwd(q, k, v, o, lse, dout, scale, False)
    return dq, dk, dv


def hvp_fd_vjp(q, k, v, dq, dk, dv, eps: float = 1e-3):
    """Central difference of the explicit VJP along (dq, dk, dv)."""
    with torch.no_grad():
        gp = _explicit_grads_sum(q + eps * dq, k + eps * dk, v + eps * dv)
        gm = _explicit_grads_sum(q - eps * dq, k - eps * dk, v - eps * dv)
    inv = 0.5 / eps
    return tuple((a - b) * inv for a, b in zip(gp, gm))


__all__ = ["hvp_fd_vjp"]
