"""sdpa_custom: theria's backend-string dispatcher (theria/attention/custom.py:15-71), the drop-in boundary.

Backends:
  "reference"                                  pure-PyTorch softmax attention (any order of derivative)
  "custom"                                     SDPACustom (autograd-in-backward, any order)
  "triton_full_fused", "triton_full_fused_phase8"
                                               the gfx950 HIP operator (names kept for drop-in
                                               compatibility; no Triton underneath), output in q.dtype
  "hip", "hip_fused"                           the same HIP operator under its own name; also Dv != D
  "triton_qk", "triton_ref", "triton"          HIP Q K^T scores (float32), softmax and PV in PyTorch
                                               (custom.py:30-36)
  "triton_fast"                                HIP Q K^T scores in the input dtype, then the same
                                               (custom.py:37-43)
  "triton_qk_softmax"                          HIP fused Q K^T + scale + softmax, PV in PyTorch; as in
                                               the reference no gradient reaches q or k (custom.py:44-49)
Unknown names raise ValueError (custom.py:57).
"""

from __future__ import annotations

import torch

from ..autograd.hip_sdpa import hip_sdpa
from ..autograd.sdpa_custom_function import SDPACustom
from .reference import reference_attention
from .scores import triton_qk, triton_qk_fast, triton_qk_softmax

HIP_BACKENDS = ("triton_full_fused", "triton_full_fused_phase8", "hip", "hip_fused")
PARTIAL_FUSION_BACKENDS = ("triton_qk", "triton_ref", "triton", "triton_fast", "triton_qk_softmax")


def sdpa_custom(q, k, v, *, backend: str = "reference", causal: bool = False):
    """Attention output (B,H,T,Dv) through the named backend. causal is honoured by the HIP backends."""
    if backend == "reference":
        if causal:
            raise AssertionError("the reference backend has no causal mask; use a HIP backend")
        return reference_attention(q, k, v)
    if backend == "custom":
        if causal:
            raise AssertionError("the custom backend has no causal mask; use a HIP backend")
        return SDPACustom.apply(q, k, v)
    if backend in HIP_BACKENDS:
        if backend.startswith("triton") and q.shape[-1] != v.shape[-1]:
            raise AssertionError(f"{backend} requires Dv == D")  # the reference's guard, custom.py:52
        return hip_sdpa(q, k, v, causal=causal).to(q.dtype)
    if backend in PARTIAL_FUSION_BACKENDS and causal:
        raise AssertionError(f"the {backend} backend has no causal mask; use a HIP fused backend")
    if backend in ("triton_qk", "triton_ref", "triton"):
        scores = triton_qk(q, k).to(torch.float32) / (q.shape[-1] ** 0.5)
        probs = torch.softmax(scores, dim=-1)
        return torch.matmul(probs, v.to(probs.dtype)).to(q.dtype)
    if backend == "triton_fast":
        scores = triton_qk_fast(q, k).to(torch.float32) / (q.shape[-1] ** 0.5)
        probs = torch.softmax(scores, dim=-1)
        return torch.matmul(probs, v.to(probs.dtype)).to(q.dtype)
    if backend == "triton_qk_softmax":
        probs = triton_qk_softmax(q, k).to(torch.float32)
        return torch.matmul(probs, v.to(probs.dtype)).to(q.dtype)
    raise ValueError(f"Unsupported sdpa_custom backend: {backend}")


def sdpa_custom_hvp(q, k, v, dq, dk, dv):
    """Explicit HVP of sum(O) for the custom backend (test/debug helper)."""
    return SDPACustom.hvp(q, k, v, dq, dk, dv)


def sdpa_custom_jvp(q, k, v, dq, dk, dv):
    """Explicit JVP for the custom backend (test/debug helper)."""
    return SDPACustom.jvp(q, k, v, dq, dk, dv)


__all__ = ["sdpa_custom", "sdpa_custom_hvp", "sdpa_custom_jvp", "HIP_BACKENDS", "PARTIAL_FUSION_BACKENDS"]
