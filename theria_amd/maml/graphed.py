"""A task-batched MAML meta-step captured once in a HIP graph and replayed.

The meta-step (task-batched meta-loss, its backward through the inner steps, and the optimizer step)
is a fixed sequence of device work for fixed task shapes, so it is recorded once with torch's graph
capture (hipGraph on ROCm) and replayed: each replay launches the whole step without Python or
launch overhead. New tasks are copied into the static input buffers before each replay.

Requirements, checked where possible: the optimizer must have been built with capturable=True (its
step counter lives on the device), every task must have the shapes of the template tasks, and nothing
in the step may synchronise with the host. The model's parameters are updated in place by the replay.
The warm-up steps run before capture are undone (parameters and optimizer state restored in place), so
the first replay is the first meta-step from the state the caller passed in; optimizer state that the
warm-up created is reset to zeros, which is the fresh state of SGD momentum and Adam.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from .batched import meta_loss_on_tasks_batched, stack_tasks


class GraphedMetaStep:
    """step(tasks) -> meta-loss tensor (device), one graph replay per call."""

    def __init__(self, model: nn.Module, optimizer: torch.optim.Optimizer, template_tasks: list, *,
                 inner_lr: float = 0.1, inner_steps: int = 1, fo: bool = False, warmup: int = 3):
        for group in optimizer.param_groups:
            if not group.get("capturable", False):
                raise ValueError("GraphedMetaStep needs an optimizer constructed with capturable=True")
        self.model, self.optimizer = model, optimizer
        self.kw = dict(inner_lr=inner_lr, inner_steps=inner_steps, fo=fo)
        self.static = [t.clone() for t in stack_tasks(template_tasks)]
        self.n = len(template_tasks)
        params = [p for p in model.parameters()]
        saved_params = [p.detach().clone() for p in params]
        saved_state = {p: {k: v.clone() if torch.is_tensor(v) else v for k, v in st.items()}
                       for p, st in optimizer.state.items()}
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):  # warm-up outside the graph (allocator pools, lazy state)
            for _ in range(warmup):
                self._body()
        torch.cuda.current_stream().wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.loss = self._body()
        # undo the warm-up steps in place (the graph holds these very tensors): the first replay is the
        # first meta-step from the model and optimizer state the caller passed in
        with torch.no_grad():
            for p, p0 in zip(params, saved_params):
                p.copy_(p0)
            for p, st in optimizer.state.items():
                old = saved_state.get(p)
                for k, v in st.items():
                    if torch.is_tensor(v):
                        if old is None:
                            v.zero_()  # state the warm-up created: fresh Adam / SGD state is zeros
                        else:
                            v.copy_(old[k])

    def _tasks(self):
        x_s, y_s, x_q, y_q = self.static
        return [_Task(x_s[i], y_s[i], x_q[i], y_q[i]) for i in range(self.n)]

    def _body(self):
        self.optimizer.zero_grad(set_to_none=True)
        loss = meta_loss_on_tasks_batched(self.model, self._tasks(), **self.kw)
        loss.backward()
        self.optimizer.step()
        return loss.detach()

    def step(self, tasks: list | None = None) -> torch.Tensor:
        if tasks is not None:
            if len(tasks) != self.n:
                raise ValueError(f"expected {self.n} tasks, got {len(tasks)}")
            for dst, src in zip(self.static, stack_tasks(tasks)):
                if dst.shape != src.shape:
                    raise ValueError(f"task shape {tuple(src.shape)} differs from the captured {tuple(dst.shape)}")
                dst.copy_(src)
        self.graph.replay()
        return self.loss


class _Task:
    __slots__ = ("x_s", "y_s", "x_q", "y_q")

    def __init__(self, x_s, y_s, x_q, y_q):
        self.x_s, self.y_s, self.x_q, self.y_q = x_s, y_s, x_q, y_q


__all__ = ["GraphedMetaStep"]
