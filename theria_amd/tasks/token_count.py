"""Token-count classification tasks for the multi-head MAML benchmark (config 5: 16 tasks, vocab 32, length 64, 5-way).

Not in the reference.
A task partitions the vocabulary at random into `num_classes` class-token sets (sizes differ by at most
one). A sequence is `seq_len` token ids drawn uniformly from the vocabulary; its label is the class
whose tokens occur most often in it, ties going to the lowest class index. Support and query sets are
class-balanced: `shots` support and `queries` query sequences per class, drawn by rejection from
uniform sequences (vectorised, in rounds).
"""

from __future__ import annotations

import torch

from .batch import TaskBatch


def label_sequences(tokens: torch.Tensor, token_class: torch.Tensor, num_classes: int) -> torch.Tensor:
    """Label = argmax over classes of the class-token count (first maximum on ties)."""
    cls = token_class[tokens]  # (N, T)
    counts = torch.zeros(tokens.shape[0], num_classes, dtype=torch.long, device=tokens.device)
    counts.scatter_add_(1, cls, torch.ones_like(cls))
    return counts.argmax(dim=1)


def sample_token_count_task(
    *,
    vocab: int = 32,
    seq_len: int = 64,
    num_classes: int = 5,
    shots: int = 5,
    queries: int = 15,
    generator: torch.Generator | None = None,
    device: torch.device | None = None,
) -> tuple[TaskBatch, torch.Tensor]:
    """One task: (TaskBatch with long token ids, token_class map of shape (vocab,))."""
    perm = torch.randperm(vocab, generator=generator)
    token_class = torch.empty(vocab, dtype=torch.long)
    token_class[perm] = torch.arange(vocab) % num_classes
    need = shots + queries
    picked: list[list[torch.Tensor]] = [[] for _ in range(num_classes)]
    have = [0] * num_classes
    rounds = 0
    while min(have) < need:
        rounds += 1
        if rounds > 1000:
            raise RuntimeError("token-count task sampling did not converge")
        toks = torch.randint(0, vocab, (512, seq_len), generator=generator)
        labels = label_sequences(toks, token_class, num_classes)
        for c in range(num_classes):
            if have[c] >= need:
                continue
            sel = toks[labels == c][: need - have[c]]
            if sel.numel():
                picked[c].append(sel)
                have[c] += sel.shape[0]
    per_class = [torch.cat(p)[:need] for p in picked]
    x_s = torch.cat([p[:shots] for p in per_class])
    y_s = torch.arange(num_classes).repeat_interleave(shots)
    x_q = torch.cat([p[shots:] for p in per_class])
    y_q = torch.arange(num_classes).repeat_interleave(queries)
    dev = torch.device("cpu") if device is None else device
    task = TaskBatch(x_s=x_s.to(dev), y_s=y_s.to(dev), x_q=x_q.to(dev), y_q=y_q.to(dev))
    return task, token_class.to(dev)


__all__ = ["label_sequences", "sample_token_count_task"]
