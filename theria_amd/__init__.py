"""theria_amd: theria's SDPA operator family as gfx950 (MI355X) HIP kernels behind theria's API.

Layout mirrors the reference package so callers switch by import name:
  theria_amd.sdpa                    the opaque pure-PyTorch SDPA (theria/__init__.py:1)
  theria_amd.attention               fused forward / explicit backward / frozen-stats JVP on HIP,
                                     sdpa_custom dispatcher, pure-PyTorch references, FD HVP
  theria_amd.autograd                SDPAOp / SDPABackwardOp (HIP, exact to second order),
                                     SDPAFunction, SDPACustom
  theria_amd.maml / models / tasks   the MAML loops and tiny models that drive double backward
"""

from .autograd.sdpa_function import sdpa

__version__ = "0.1.0"

__all__ = ["sdpa"]
