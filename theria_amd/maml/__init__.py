from .loops import inner_adapt, loss_fn, meta_loss_on_tasks, named_buffers, named_params, outer_loss

__all__ = ["inner_adapt", "loss_fn", "meta_loss_on_tasks", "named_buffers", "named_params", "outer_loss"]
