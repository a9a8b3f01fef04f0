"""Multi-head attention sequence classifier for the MAML benchmark (config 5: 2 layers, d_model 64, 4 heads).

Not in the reference (nearest: examples/minimal_decoder_transformer.py:82-263 and the Phase-10 model).
Token embedding (no positions: the token-count task is order-free), `layers` pre-norm blocks of
multi-head self-attention + GELU MLP with residuals, final LayerNorm, mean-pool over tokens, linear
head. Attention goes through sdpa_custom(backend=...), so the same weights run on the pure-PyTorch
"reference" backend or on the HIP operator, and full MAML differentiates through it twice.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F

from ..attention.custom import sdpa_custom


@dataclass(frozen=True)
class MHAConfig:
    vocab: int = 32
    d_model: int = 64
    heads: int = 4
    layers: int = 2
    mlp_ratio: int = 2
    num_classes: int = 5


class _Block(nn.Module):
    def __init__(self, cfg: MHAConfig):
        super().__init__()
        d = cfg.d_model
        self.heads = cfg.heads
        self.ln1 = nn.LayerNorm(d)
        self.qkv = nn.Linear(d, 3 * d)
        self.proj = nn.Linear(d, d)
        self.ln2 = nn.LayerNorm(d)
        self.fc1 = nn.Linear(d, cfg.mlp_ratio * d)
        self.fc2 = nn.Linear(cfg.mlp_ratio * d, d)

    def forward(self, x: torch.Tensor, backend: str) -> torch.Tensor:
        B, T, d = x.shape
        H = self.heads
        qkv = self.qkv(self.ln1(x)).view(B, T, 3, H, d // H).permute(2, 0, 3, 1, 4)
        att = sdpa_custom(qkv[0], qkv[1], qkv[2], backend=backend)  # (B, H, T, d/H)
        x = x + self.proj(att.transpose(1, 2).reshape(B, T, d))
        return x + self.fc2(F.gelu(self.fc1(self.ln2(x))))


class MHAClassifier(nn.Module):
    """token ids (B, T) -> logits (B, num_classes)."""

    def __init__(self, cfg: MHAConfig | None = None, backend: str = "reference"):
        super().__init__()
        self.cfg = cfg or MHAConfig()
        self.backend = backend
        self.embed = nn.Embedding(self.cfg.vocab, self.cfg.d_model)
        self.blocks = nn.ModuleList(_Block(self.cfg) for _ in range(self.cfg.layers))
        self.ln_f = nn.LayerNorm(self.cfg.d_model)
        self.head = nn.Linear(self.cfg.d_model, self.cfg.num_classes)

    def set_attention_backend(self, backend: str) -> None:
        self.backend = backend

    def forward(self, tokens: torch.Tensor) -> torch.Tensor:
        x = self.embed(tokens)
        for blk in self.blocks:
            x = blk(x, self.backend)
        return self.head(self.ln_f(x).mean(dim=1))

    def forward_batched(self, params: dict, tokens: torch.Tensor) -> torch.Tensor:
        """Many parameter sets at once: params[name] is (n, *shape), tokens (n, N, T) -> logits (n, N, C).

        The same computation as forward() for each of the n parameter sets, with every layer batched
        over n: per-set linear layers and layer-norm affines are batched matmuls (bias folded in as a
        ones column), the embedding is a one-hot matmul and attention is one sdpa_custom call over
        n * N sequences. Every gradient of these is a matmul or elementwise, so no derivative order
        needs a device memset or atomics: the pass is deterministic and can be captured in a graph.
        """
        cfg = self.cfg
        n, N, T = tokens.shape
        d, H = cfg.d_model, cfg.heads

        def affine(x, wt, b):
            # x @ wt + b as one batched matmul of [x, 1] with [wt; b]: its gradients are GEMMs, not
            # multi-block sums over the broadcast rows (those issue device memsets, which a captured
            # graph must not contain)
            x2 = x.reshape(n, -1, x.shape[-1])
            xa = torch.cat([x2, x2.new_ones(n, x2.shape[1], 1)], dim=2)
            y = torch.matmul(xa, torch.cat([wt, b.unsqueeze(1)], dim=1))
            return y.reshape(*x.shape[:-1], wt.shape[-1])

        def lin(x, name):
            return affine(x, params[name + ".weight"].transpose(1, 2), params[name + ".bias"])

        def norm(x, name):
            y = F.layer_norm(x, (x.shape[-1],))
            return affine(y, torch.diag_embed(params[name + ".weight"]), params[name + ".bias"])

        # one-hot by comparison: elementwise, so the pass has no host synchronisation (graph capture)
        ids = torch.arange(cfg.vocab, device=tokens.device)
        onehot = (tokens.reshape(n, N * T, 1) == ids).to(params["embed.weight"].dtype)
        x = torch.matmul(onehot, params["embed.weight"]).reshape(n, N, T, d)
        for i in range(cfg.layers):
            pre = f"blocks.{i}."
            qkv = lin(norm(x, pre + "ln1"), pre + "qkv").reshape(n * N, T, 3, H, d // H).permute(2, 0, 3, 1, 4)
            att = sdpa_custom(qkv[0], qkv[1], qkv[2], backend=self.backend)  # (n*N, H, T, d/H)
            x = x + lin(att.transpose(1, 2).reshape(n, N, T, d), pre + "proj")
            x = x + lin(F.gelu(lin(norm(x, pre + "ln2"), pre + "fc1")), pre + "fc2")
        return lin(norm(x, "ln_f").mean(dim=2), "head")


__all__ = ["MHAConfig", "MHAClassifier"]
