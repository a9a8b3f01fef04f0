"""Explicit SDPA backward in pure PyTorch (no autograd).

Contract of theria/attention/reference_backward_sdpa.py:12-53: given upstream dout and the softmax
scale, returns (dq, dk, dv) with
  P = softmax(scale q k^T), dv = P^T dout, dP = dout v^T, z = rowsum(dP o P),
  dS = P o (dP - z), dq = scale dS k, dk = scale dS^T q.
"""

from __future__ import annotations

import torch

from .reference_attention import reference_attention


def sdpa_backward_reference(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, dout: torch.Tensor, scale: float):
    with torch.no_grad():
        q, k, v, dout = (t.detach() for t in (q, k, v, dout))
        p = torch.softmax(torch.matmul(q, k.transpose(-2, -1)) * scale, dim=-1)
        dp = torch.matmul(dout, v.transpose(-2, -1))
        ds = p * (dp - (dp * p).sum(dim=-1, keepdim=True))
        dq = torch.matmul(ds, k) * scale
        dk = torch.matmul(ds.transpose(-2, -1), q) * scale
        dv = torch.matmul(p.transpose(-2, -1), dout)
    return dq, dk, dv


__all__ = ["sdpa_backward_reference", "reference_attention"]
