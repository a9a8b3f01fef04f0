"""Task-batched MAML: every task of a meta-batch adapts at once, in one batched forward and backward.

Same mathematics as meta_loss_on_tasks (theria/maml/loops.py:42-123 in the reference): each task t starts
from phi_t = theta and takes `inner_steps` SGD steps on its support loss, and the meta-loss is the mean
of the query losses at the adapted phi_t. Here the per-task parameters carry a leading task dimension
(theta expanded n times, so the meta-gradient sums over tasks through the expand) and the model runs all
tasks in one forward_batched call. The inner gradient is taken of the sum of the per-task support losses:
phi_t influences only task t's loss, so each task receives exactly its own gradient. One call per layer
instead of one per task and layer divides the number of kernel launches, which bound the sequential loop
on this small model, by the number of tasks.

The model must provide forward_batched(params, x) with params[name] of shape (n, *param.shape) and x
stacked over tasks; every task in the meta-batch must have the same support and query shapes.
"""

from __future__ import annotations

from collections import OrderedDict

import torch
import torch.nn as nn
import torch.nn.functional as F


def stack_tasks(tasks: list):
    """(x_s, y_s, x_q, y_q), each stacked over the tasks along a new leading dimension."""
    return tuple(torch.stack([getattr(t, f) for t in tasks]) for f in ("x_s", "y_s", "x_q", "y_q"))


def _task_losses(logits: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    """Mean cross-entropy per task: logits (n, N, C), y (n, N) -> (n,)."""
    n, N = y.shape
    return F.cross_entropy(logits.reshape(n * N, -1), y.reshape(n * N), reduction="none").reshape(n, N).mean(1)


def inner_adapt_batched(model: nn.Module, params, x_s, y_s, *, inner_lr: float = 0.1, inner_steps: int = 1,
                        fo: bool = False):
    """Per-task adapted parameters (n, *shape) after `inner_steps` SGD steps; create_graph unless fo."""
    n = x_s.shape[0]
    # theta repeated n times as ones(n, 1) @ theta: the meta-gradient's sum over tasks is then a GEMM
    # (an expand's backward would be a multi-block sum, which issues a device memset)
    ones = next(iter(params.values())).new_ones(n, 1)
    phi = OrderedDict((name, torch.matmul(ones, w.reshape(1, -1)).reshape(n, *w.shape)) for name, w in params.items())
    for _ in range(inner_steps):
        support = _task_losses(model.forward_batched(phi, x_s), y_s).sum()
        grads = torch.autograd.grad(support, tuple(phi.values()), create_graph=not fo, retain_graph=True)
        phi = OrderedDict((name, w - inner_lr * g) for (name, w), g in zip(phi.items(), grads))
    return phi


def meta_loss_on_tasks_batched(
    model: nn.Module,
    tasks: list,
    *,
    inner_lr: float = 0.1,
    inner_steps: int = 1,
    fo: bool = False,
    fo_strict: bool = False,
    return_metrics: bool = False,
):
    """J(theta) = mean over tasks of L_query(phi_K(theta; support)), all tasks batched."""
    x_s, y_s, x_q, y_q = stack_tasks(tasks)
    params = OrderedDict(model.named_parameters())
    phi = inner_adapt_batched(model, params, x_s, y_s, inner_lr=inner_lr, inner_steps=inner_steps, fo=fo)
    if fo_strict:
        phi = OrderedDict((name, w.detach().clone()) for name, w in phi.items())
    logits = model.forward_batched(phi, x_q)
    outer = _task_losses(logits, y_q).mean()
    if return_metrics:
        acc = (logits.argmax(dim=-1) == y_q).float().mean()
        return outer, {"post_adapt_loss": outer.item(), "post_adapt_acc": acc.item()}
    return outer


__all__ = ["stack_tasks", "inner_adapt_batched", "meta_loss_on_tasks_batched"]
