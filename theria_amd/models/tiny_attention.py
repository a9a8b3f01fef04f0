"""Tiny attention classifiers used by the MAML loops.

TinyAttentionModel mirrors theria/models/tiny_attention.py:37-95: single head, token 0 is a CLS-like
query over all tokens, own eager attention (sdpa_explicit). BackendAttentionModel is the same model
with its attention routed through sdpa_custom(backend=...), as the reference's Phase-10 experiment
model does (experiments/phase10/scripts/run_maml_backend_compare.py:48-87): q (B,1,1,D), k/v (B,1,T,D).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn as nn

from ..attention.custom import sdpa_custom


def sdpa_explicit(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """softmax(q k^T / sqrt(d)) v for (B, Tq, D) / (B, Tk, D), max-subtracted for stability."""
    scores = torch.matmul(q, k.transpose(-2, -1)) / math.sqrt(q.shape[-1])
    scores = scores - scores.max(dim=-1, keepdim=True).values
    return torch.matmul(scores.softmax(dim=-1), v)


@dataclass(frozen=True)
class TinyAttentionConfig:
    d_model: int = 64
    num_classes: int = 5


class TinyAttentionModel(nn.Module):
    """x (B, T, D) -> logits (B, C); token 0 queries every token."""

    def __init__(self, cfg: TinyAttentionConfig):
        super().__init__()
        self.cfg = cfg
        D = cfg.d_model
        self.q_proj = nn.Linear(D, D, bias=False)
        self.k_proj = nn.Linear(D, D, bias=False)
        self.v_proj = nn.Linear(D, D, bias=False)
        self.classifier = nn.Linear(D, cfg.num_classes)

    def _attend(self, x):
        return sdpa_explicit(self.q_proj(x[:, :1, :]), self.k_proj(x), self.v_proj(x)).squeeze(1)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.classifier(self._attend(x))

    def forward_with_params(self, params: dict, x: torch.Tensor) -> torch.Tensor:
        from torch.func import functional_call

        return functional_call(self, params, (x,))


class BackendAttentionModel(nn.Module):
    """TinyAttentionModel with a swappable attention backend (sdpa_custom backend string)."""

    def __init__(self, cfg: TinyAttentionConfig | None = None, backend: str = "reference"):
        super().__init__()
        self.cfg = cfg or TinyAttentionConfig()
        self.backend = backend
        D = self.cfg.d_model
        self.q_proj = nn.Linear(D, D, bias=False)
        self.k_proj = nn.Linear(D, D, bias=False)
        self.v_proj = nn.Linear(D, D, bias=False)
        self.classifier = nn.Linear(D, self.cfg.num_classes)

    def set_attention_backend(self, backend: str) -> None:
        self.backend = backend

    def _resolve_backend(self) -> str:
        return "triton_full_fused" if self.backend == "triton_fused" else self.backend

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        q = self.q_proj(x[:, :1, :]).unsqueeze(1)
        k = self.k_proj(x).unsqueeze(1)
        v = self.v_proj(x).unsqueeze(1)
        h = sdpa_custom(q, k, v, backend=self._resolve_backend())
        return self.classifier(h.squeeze(1).squeeze(1))


__all__ = ["sdpa_explicit", "TinyAttentionConfig", "TinyAttentionModel", "BackendAttentionModel"]
