"""autograd.Functions: the HIP operator (SDPAOp / SDPABackwardOp) and the pure-PyTorch references."""

from .graphed_hvp import GraphedSDPAHVP
from .hip_sdpa import SDPABackwardOp, SDPAOp, hip_sdpa, hip_sdpa_hvp, hip_sdpa_with_lse
from .sdpa_custom_function import SDPACustom
from .sdpa_function import SDPAFunction, sdpa

__all__ = ["SDPAOp", "SDPABackwardOp", "hip_sdpa", "hip_sdpa_with_lse", "hip_sdpa_hvp", "GraphedSDPAHVP", "SDPACustom", "SDPAFunction", "sdpa"]
