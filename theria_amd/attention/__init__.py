"""Attention operators: the HIP SDPA family under theria's public names, plus the pure-PyTorch references.

Stable surface (the reference's theria/attention/__init__.py:12-26): triton_sdpa_fused, sdpa_bwd_dq,
sdpa_bwd_dk, sdpa_bwd_dv, sdpa_jvp, all running the gfx950 kernels. Importing this package does not
touch the GPU; the kernel library is loaded on first use.
"""

from ..autograd.hip_sdpa import hip_sdpa, hip_sdpa_hvp, hip_sdpa_with_lse
from .explicit import sdpa_bwd, sdpa_bwd_dk, sdpa_bwd_dq, sdpa_bwd_dv, sdpa_jvp
from .fused import TritonFusedSDPAFunction, sdpa_fused, triton_sdpa_fused, triton_sdpa_fused_autograd

__all__ = [
    "triton_sdpa_fused",
    "sdpa_bwd_dq",
    "sdpa_bwd_dk",
    "sdpa_bwd_dv",
    "sdpa_jvp",
    "sdpa_bwd",
    "sdpa_fused",
    "hip_sdpa",
    "hip_sdpa_with_lse",
    "hip_sdpa_hvp",
    "TritonFusedSDPAFunction",
    "triton_sdpa_fused_autograd",
]
