"""Second-order safety probes: does an attention backend carry curvature into the meta-gradient?

The reference classifies attention backends for meta-learning with two probes (its safety taxonomy,
docs/STATUS.md:142-150: "detach" collapses to first order, "explicit backward" is safe):

attention_second_order_ok   grad of ||grad_{q,k,v} sum(O)||^2 through the attention call alone is
                            nonzero (experiments/phase11/scripts/run_bad_backend_diagnostics.py:54-86).
meta_gradient_probe         on a MAML model: whether the full meta-gradient can be differentiated again
                            (globally, through the q/k/v projections, through the classifier head), and
                            the relative difference between the full and first-order meta-gradients
                            (run_bad_backend_diagnostics.py:89-175, experiments/phase10/scripts/
                            run_maml_backend_compare.py:169-215).

A backend that silently drops attention's second-order terms (the reference's Triton autograd path,
theria/attention/triton_qk.py:379-387) keeps every flag true, because second order still reaches each
parameter through attention's first-order terms, but its full meta-gradient and full-vs-first-order
difference move (smaller than the exact backends' in the reference's runs). So the HIP operator is held
to the exact pure-PyTorch backend's values, not only to the flags.
"""

from __future__ import annotations

from typing import Callable, Iterable

import torch
import torch.nn as nn

from .loops import meta_loss_on_tasks

ATTENTION_PARAMS = ("q_proj.weight", "k_proj.weight", "v_proj.weight")


def _nonzero(g, eps: float) -> bool:
    return g is not None and float(g.detach().abs().sum()) > eps


def _sum_of_squares(grads: Iterable):
    total = None
    for g in grads:
        if g is None:
            continue
        term = g.pow(2).sum()
        total = term if total is None else total + term
    return total


def attention_second_order_ok(
    sdpa_fn: Callable[..., torch.Tensor],
    *,
    device,
    dtype: torch.dtype = torch.float32,
    eps: float = 1e-12,
    generator: torch.Generator | None = None,
) -> bool:
    """True when grad ||grad sum(sdpa_fn(q, k, v))||^2 w.r.t. (q, k, v) is nonzero; False on any error.

    Shapes as in the reference probe: one query, two keys, head dim 4.
    """
    try:
        shapes = ((1, 1, 1, 4), (1, 1, 2, 4), (1, 1, 2, 4))
        q, k, v = (torch.randn(s, generator=generator).to(device=device, dtype=dtype).requires_grad_(True)
                   for s in shapes)
        out = sdpa_fn(q, k, v)
        g1 = torch.autograd.grad(out.sum(), (q, k, v), retain_graph=True, create_graph=True, allow_unused=True)
        g1_scalar = _sum_of_squares(g1)
        if g1_scalar is None:
            return False
        g2 = torch.autograd.grad(g1_scalar, (q, k, v), allow_unused=True)
        return any(_nonzero(g, eps) for g in g2)
    except Exception:
        return False


def _flat(grads) -> torch.Tensor | None:
    if not any(g is not None for g in grads):
        return None
    return torch.cat([g.flatten() for g in grads if g is not None])


def meta_gradient_probe(
    model: nn.Module,
    task,
    *,
    inner_steps: int = 1,
    inner_lr: float = 0.1,
    eps: float = 1e-12,
    attention_params: Iterable[str] = ATTENTION_PARAMS,
    head_prefix: str = "classifier.",
) -> dict:
    """Second-order flags and the full-vs-first-order meta-gradient difference for one task.

    Returns {"second_order_path", "second_order_attn", "second_order_head": bool,
    "rel_diff_full_vs_fo": float (nan when the full meta-gradient vanishes),
    "meta_grad_full", "meta_grad_fo": flattened meta-gradients, "meta_curvature": the flattened
    gradient of ||full meta-gradient||^2 that the second_order_path flag tests, or None}.
    """
    named = [(n, p) for n, p in model.named_parameters() if p.requires_grad]
    names = [n for n, _ in named]
    params = [p for _, p in named]
    full = meta_loss_on_tasks(model, [task], inner_lr=inner_lr, inner_steps=inner_steps, fo=False)
    fo = meta_loss_on_tasks(model, [task], inner_lr=inner_lr, inner_steps=inner_steps, fo=True)

    flags = {"second_order_path": False, "second_order_attn": False, "second_order_head": False}
    curvature = None
    try:
        g1 = torch.autograd.grad(full, params, retain_graph=True, create_graph=True, allow_unused=True)
        g1_scalar = _sum_of_squares(g1)
        if g1_scalar is not None:
            g2 = dict(zip(names, torch.autograd.grad(g1_scalar, params, retain_graph=True, allow_unused=True)))
            curvature = _flat(tuple(g2.values()))
            flags["second_order_path"] = any(_nonzero(g, eps) for g in g2.values())
            flags["second_order_attn"] = any(_nonzero(g2.get(n), eps) for n in attention_params)
            flags["second_order_head"] = any(_nonzero(g, eps) for n, g in g2.items() if n.startswith(head_prefix))
    except RuntimeError:
        pass

    v_full = _flat(torch.autograd.grad(full, params, retain_graph=True, allow_unused=True))
    v_fo = _flat(torch.autograd.grad(fo, params, retain_graph=True, allow_unused=True))
    rel = float("nan")
    if v_full is not None and v_fo is not None and float(v_full.norm()) > 1e-9:
        rel = float((v_full - v_fo).norm()) / (float(v_full.norm()) + 1e-9)
    return dict(flags, rel_diff_full_vs_fo=rel, meta_grad_full=v_full, meta_grad_fo=v_fo, meta_curvature=curvature)


__all__ = ["attention_second_order_ok", "meta_gradient_probe", "ATTENTION_PARAMS"]
