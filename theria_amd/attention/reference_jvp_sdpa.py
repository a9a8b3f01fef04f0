"""Forward-mode (JVP) ground truth for SDPA in pure PyTorch, accumulated in float64.

Contract of theria/attention/reference_jvp_sdpa.py:12-44: with P = softmax(scale q k^T),
  dS = scale (dq k^T + q dk^T),  dP = P o (dS - rowsum(dS o P)),  dO = dP v + P dv,
computed in float64 and returned in q's dtype.
"""

from __future__ import annotations

import torch


def softmax_jvp(scores: torch.Tensor, dscores: torch.Tensor, p: torch.Tensor) -> torch.Tensor:
    """Directional derivative of softmax(scores) along dscores, given p = softmax(scores)."""
    del scores  # the derivative only needs p
    return p * (dscores - (dscores * p).sum(dim=-1, keepdim=True))


def sdpa_jvp_reference(q, k, v, dq, dk, dv, scale):
    q64, k64, v64, dq64, dk64, dv64 = (t.to(torch.float64) for t in (q, k, v, dq, dk, dv))
    kt = k64.transpose(-2, -1)
    scores = torch.matmul(q64, kt) * scale
    p = torch.softmax(scores, dim=-1)
    dscores = (torch.matmul(dq64, kt) + torch.matmul(q64, dk64.transpose(-2, -1))) * scale
    out = torch.matmul(softmax_jvp(scores, dscores, p), v64) + torch.matmul(p, dv64)
    return out.to(q.dtype)


sdpa_jvp = sdpa_jvp_reference

__all__ = ["sdpa_jvp_reference", "softmax_jvp", "sdpa_jvp"]
