"""Pure-PyTorch scaled dot-product attention: theria's "reference" backend.

Same contract as theria/attention/reference_attention.py:9-19 in the reference: scores scaled by
1/sqrt(D), softmax over the key axis, then the value product. Written for differentiability to any
order (plain torch ops), not for speed.
"""

from __future__ import annotations

import math

import torch


def reference_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """softmax(q k^T / sqrt(D)) v for q (B,H,N,D), k (B,H,M,D), v (B,H,M,Dv)."""
    inv_sqrt_d = 1.0 / math.sqrt(q.shape[-1])
    weights = torch.softmax(torch.matmul(q, k.transpose(-2, -1)) * inv_sqrt_d, dim=-1)
    return torch.matmul(weights, v)


# Legacy name kept by the reference (reference_attention.py:24).
sdpa_reference = reference_attention

__all__ = ["reference_attention", "sdpa_reference"]
