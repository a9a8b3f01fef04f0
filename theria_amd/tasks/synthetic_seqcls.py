"""Prototype-injection sequence classification tasks (theria/tasks/synthetic_seqcls.py:45-89).

Each task picks signal positions (never position 0, the query token) and per-class prototypes; a
sequence is Gaussian noise with its class prototype (plus half-strength noise) injected at the signal
positions.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class TaskBatch:
    x_s: torch.Tensor  # support inputs
    y_s: torch.Tensor  # support labels
    x_q: torch.Tensor  # query inputs
    y_q: torch.Tensor  # query labels


def _make_split(B, T, D, num_classes, positions, prototypes, noise_std, device, dtype):
    y = torch.randint(0, num_classes, (B,), device=device)
    x = torch.randn((B, T, D), device=device, dtype=dtype) * noise_std
    signal = prototypes[y]
    for pos in positions.tolist():
        x[:, pos, :] = signal + torch.randn((B, D), device=device, dtype=dtype) * (0.5 * noise_std)
    return x, y


def task_sampler(
    *,
    B_s: int = 16,
    B_q: int = 16,
    T: int = 32,
    D: int = 64,
    num_classes: int = 5,
    num_signal_positions: int = 4,
    noise_std: float = 1.0,
    device: torch.device | None = None,
    dtype: torch.dtype = torch.float32,
) -> TaskBatch:
    device = torch.device("cpu") if device is None else device
    candidates = torch.arange(1, T, device=device)
    positions = candidates[torch.randperm(candidates.numel(), device=device)[:num_signal_positions]]
    prototypes = torch.randn((num_classes, D), device=device, dtype=dtype)
    x_s, y_s = _make_split(B_s, T, D, num_classes, positions, prototypes, noise_std, device, dtype)
    x_q, y_q = _make_split(B_q, T, D, num_classes, positions, prototypes, noise_std, device, dtype)
    return TaskBatch(x_s=x_s, y_s=y_s, x_q=x_q, y_q=y_q)


__all__ = ["TaskBatch", "task_sampler"]
