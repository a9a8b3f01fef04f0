"""The second-order safety probes (theria_amd.maml.diagnostics) on the CPU with the pure-PyTorch backend.

The probes must tell an exact backend from one that drops attention curvature. The mistakes are planted
here, around the pure-PyTorch reference attention (the reference's experiment-only wrappers,
experiments/phase11/scripts/bad_backends.py, restated): a detached output, attention under no_grad, a
once-differentiable backward, and a backward that returns graph-less gradients the way the reference's
Triton autograd path does (theria/attention/triton_qk.py:379-387).
"""

import math

import pytest
import torch
from torch.autograd.function import once_differentiable

import theria_amd.models.tiny_attention as tiny
from theria_amd.attention.custom import sdpa_custom
from theria_amd.attention.reference import reference_attention
from theria_amd.maml.diagnostics import attention_second_order_ok, meta_gradient_probe
from theria_amd.models.tiny_attention import BackendAttentionModel, TinyAttentionConfig
from theria_amd.tasks import teacher_readout_task


def detach_output(fn):
    def wrapped(q, k, v, **kw):
        out = fn(q, k, v, **kw)
        return out.detach() + out * 0.0

    return wrapped


def no_grad(fn):
    def wrapped(q, k, v, **kw):
        with torch.no_grad():
            return fn(q, k, v, **kw)

    return wrapped


class _OnceDifferentiable(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v):
        ctx.save_for_backward(q, k, v)
        return reference_attention(q, k, v)

    @staticmethod
    @once_differentiable
    def backward(ctx, g):
        q, k, v = (t.detach().requires_grad_(True) for t in ctx.saved_tensors)
        with torch.enable_grad():
            out = reference_attention(q, k, v)
        return torch.autograd.grad(out, (q, k, v), g)


class _GraphlessBackward(torch.autograd.Function):
    """First-order exact, but the gradients it returns carry no graph (silent curvature loss)."""

    @staticmethod
    def forward(ctx, q, k, v):
        ctx.save_for_backward(q, k, v)
        return reference_attention(q, k, v)

    @staticmethod
    def backward(ctx, g):
        q, k, v = (t.detach().requires_grad_(True) for t in ctx.saved_tensors)
        with torch.enable_grad():
            out = reference_attention(q, k, v)
            grads = torch.autograd.grad(out, (q, k, v), g.detach())
        return tuple(x.detach() for x in grads)


def _backend(name):
    return lambda q, k, v, **kw: sdpa_custom(q, k, v, backend=name)


def test_attention_probe_accepts_exact_backends():
    gen = torch.Generator().manual_seed(0)
    for name in ("reference", "custom"):
        assert attention_second_order_ok(_backend(name), device="cpu", generator=gen)


@pytest.mark.parametrize(
    "bad",
    [
        detach_output(_backend("reference")),
        no_grad(_backend("reference")),
        lambda q, k, v: _OnceDifferentiable.apply(q, k, v),
        lambda q, k, v: _GraphlessBackward.apply(q, k, v),
    ],
    ids=["detach_output", "no_grad", "once_differentiable", "graphless_backward"],
)
def test_attention_probe_rejects_planted_mistakes(bad):
    assert not attention_second_order_ok(bad, device="cpu", generator=torch.Generator().manual_seed(0))


def _model_and_task(seed=0):
    torch.manual_seed(seed)
    model = BackendAttentionModel(TinyAttentionConfig(d_model=16, num_classes=3), backend="reference")
    task = teacher_readout_task(support=8, query=8, T=6, D=16, num_classes=3,
                                generator=torch.Generator().manual_seed(seed))
    return model, task


def test_meta_probe_exact_backend_is_safe():
    model, task = _model_and_task()
    r = meta_gradient_probe(model, task, inner_steps=2, inner_lr=0.4)
    assert r["second_order_path"] and r["second_order_attn"] and r["second_order_head"]
    assert math.isfinite(r["rel_diff_full_vs_fo"]) and r["rel_diff_full_vs_fo"] > 1e-4


def test_meta_probe_flags_silent_curvature_loss(monkeypatch):
    model, task = _model_and_task()
    exact = meta_gradient_probe(model, task, inner_steps=2, inner_lr=0.4)
    monkeypatch.setattr(tiny, "sdpa_custom", lambda q, k, v, backend: _GraphlessBackward.apply(q, k, v))
    lossy = meta_gradient_probe(model, task, inner_steps=2, inner_lr=0.4)
    # first order is unchanged, so the first-order meta-gradients agree ...
    torch.testing.assert_close(lossy["meta_grad_fo"], exact["meta_grad_fo"], rtol=1e-5, atol=1e-7)
    # ... but the full one lost attention's second-order terms. The flags cannot see it (second order
    # still reaches every parameter through the first-order attention terms: the loss is silent, as the
    # reference found for its Triton path); the full-vs-first-order difference moves
    assert not torch.allclose(lossy["meta_grad_full"], exact["meta_grad_full"], rtol=1e-4, atol=1e-6)
    assert lossy["second_order_path"] and lossy["second_order_head"] and lossy["second_order_attn"]
    assert abs(lossy["rel_diff_full_vs_fo"] - exact["rel_diff_full_vs_fo"]) > 1e-2 * exact["rel_diff_full_vs_fo"]


def test_meta_probe_detach_collapses_attention(monkeypatch):
    model, task = _model_and_task()
    monkeypatch.setattr(tiny, "sdpa_custom", detach_output(sdpa_custom))
    r = meta_gradient_probe(model, task, inner_steps=1, inner_lr=0.4)
    assert not r["second_order_attn"]
