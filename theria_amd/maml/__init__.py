from .batched import inner_adapt_batched, meta_loss_on_tasks_batched, stack_tasks
from .graphed import GraphedMetaStep
from .diagnostics import attention_second_order_ok, meta_gradient_probe
from .loops import inner_adapt, loss_fn, meta_loss_on_tasks, named_buffers, named_params, outer_loss

__all__ = [
    "GraphedMetaStep",
    "inner_adapt_batched",
    "meta_loss_on_tasks_batched",
    "stack_tasks",
    "attention_second_order_ok",
    "meta_gradient_probe",
    "inner_adapt", "loss_fn", "meta_loss_on_tasks", "named_buffers", "named_params", "outer_loss"]
