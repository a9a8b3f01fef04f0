"""Continuous-input few-shot tasks for the tiny attention models: a hidden position read by a linear teacher.

A task draws a position p in 1..T-1 and a teacher matrix W of shape (num_classes, D) with unit-norm rows.
A sequence x is standard normal noise of shape (T, D); its label is argmax_c W_c . x_p. The models classify
from the query token at position 0, so a task is solved by attending to p and reading x_p through W:
adaptation has to move both the attention (where to look) and the head (what to read), which is what the
second-order terms of full MAML carry. Labels are not balanced; with the default sizes every class occurs.
"""

from __future__ import annotations

import torch

from .batch import TaskBatch


def teacher_readout_task(
    *,
    support: int = 16,
    query: int = 16,
    T: int = 32,
    D: int = 64,
    num_classes: int = 5,
    generator: torch.Generator | None = None,
    device: torch.device | None = None,
    dtype: torch.dtype = torch.float32,
) -> TaskBatch:
    """One task with `support` + `query` labelled sequences of shape (T, D)."""
    if T < 2:
        raise ValueError("teacher_readout_task needs T >= 2 (position 0 is the query token)")
    pos = int(torch.randint(1, T, (1,), generator=generator))
    W = torch.randn(num_classes, D, generator=generator, dtype=torch.float64)
    W = W / W.norm(dim=1, keepdim=True)
    x = torch.randn(support + query, T, D, generator=generator, dtype=torch.float64)
    y = (x[:, pos] @ W.T).argmax(dim=1)
    dev = torch.device("cpu") if device is None else device
    x = x.to(dtype=dtype, device=dev)
    y = y.to(dev)
    return TaskBatch(x_s=x[:support], y_s=y[:support], x_q=x[support:], y_q=y[support:])


__all__ = ["teacher_readout_task"]
