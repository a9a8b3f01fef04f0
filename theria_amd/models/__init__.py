from .mha_classifier import MHAClassifier, MHAConfig
from .tiny_attention import BackendAttentionModel, TinyAttentionConfig, TinyAttentionModel, sdpa_explicit

__all__ = [
    "MHAClassifier",
    "MHAConfig",
    "BackendAttentionModel",
    "TinyAttentionConfig",
    "TinyAttentionModel",
    "sdpa_explicit",
]
