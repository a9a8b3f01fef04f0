"""Re-exports of the pure-PyTorch reference helpers (the reference's theria/attention/reference.py)."""

from .reference_attention import reference_attention, sdpa_reference
from .reference_backward_sdpa import sdpa_backward_reference
from .reference_hvp_sdpa import sdpa_hvp_reference
from .reference_jvp_sdpa import sdpa_jvp_reference

__all__ = [
    "reference_attention",
    "sdpa_reference",
    "sdpa_backward_reference",
    "sdpa_jvp_reference",
    "sdpa_hvp_reference",
]
