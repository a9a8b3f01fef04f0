"""The few-shot task container of the MAML loops (field names follow theria's TaskBatch)."""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class TaskBatch:
    x_s: torch.Tensor  # support inputs, (N_s, ...) with the sequence dimension after the batch
    y_s: torch.Tensor  # support labels, (N_s,) long
    x_q: torch.Tensor  # query inputs
    y_q: torch.Tensor  # query labels


__all__ = ["TaskBatch"]
