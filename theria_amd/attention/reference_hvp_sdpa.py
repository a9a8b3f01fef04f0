"""Analytic JVP and HVP of SDPA in pure PyTorch (correctness reference, not optimized).

Contract of theria/attention/reference_hvp_sdpa.py:20-97:
  * sdpa_jvp(q, k, v, dq, dk, dv): directional derivative of softmax(q k^T / sqrt(D)) v;
  * sdpa_hvp(q, k, v, vq, vk, vv): Hessian-vector product of L = sum(O) along (vq, vk, vv).
For L = sum(O) the gradient with respect to P is g_ij = sum_d V_jd (the same for every row i), so
  grad_S = P o (g - rowsum(g o P)),  dq = s grad_S k,  dk = s grad_S^T q,  dv = P^T 1,
and the HVP is the directional derivative of these three expressions.
"""

from __future__ import annotations

import math

import torch


def _softmax_dir(p: torch.Tensor, ds: torch.Tensor) -> torch.Tensor:
    return p * (ds - (ds * p).sum(dim=-1, keepdim=True))


def _scores_dir(q, k, dq, dk, s):
    return (torch.matmul(dq, k.transpose(-2, -1)) + torch.matmul(q, dk.transpose(-2, -1))) * s


def sdpa_jvp(q, k, v, dq, dk, dv):
    """J_sdpa(q, k, v) . (dq, dk, dv), scale 1/sqrt(D)."""
    s = 1.0 / math.sqrt(q.shape[-1])
    p = torch.softmax(torch.matmul(q, k.transpose(-2, -1)) * s, dim=-1)
    dp = _softmax_dir(p, _scores_dir(q, k, dq, dk, s))
    return torch.matmul(dp, v) + torch.matmul(p, dv)


def sdpa_hvp(q, k, v, vq, vk, vv):
    """HVP of L = sum(reference_attention(q, k, v)) along (vq, vk, vv); returns (hq, hk, hv)."""
    s = 1.0 / math.sqrt(q.shape[-1])
    p = torch.softmax(torch.matmul(q, k.transpose(-2, -1)) * s, dim=-1)
    dp = _softmax_dir(p, _scores_dir(q, k, vq, vk, s))  # direction of P

    g = v.sum(dim=-1).unsqueeze(-2).expand_as(p)  # dL/dP
    dg = vv.sum(dim=-1).unsqueeze(-2).expand_as(p)  # its direction
    c = (g * p).sum(dim=-1, keepdim=True)
    dc = (dg * p + g * dp).sum(dim=-1, keepdim=True)
    grad_s = p * (g - c)
    dgrad_s = dp * (g - c) + p * (dg - dc)

    hq = s * (torch.matmul(dgrad_s, k) + torch.matmul(grad_s, vk))
    hk = s * (torch.matmul(dgrad_s.transpose(-2, -1), q) + torch.matmul(grad_s.transpose(-2, -1), vq))
    hv = dp.sum(dim=-2).unsqueeze(-1).expand_as(v)  # direction of P^T 1
    return hq, hk, hv


sdpa_hvp_reference = sdpa_hvp

__all__ = ["sdpa_hvp", "sdpa_hvp_reference", "sdpa_jvp"]
