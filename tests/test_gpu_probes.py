"""Second-order safety probes on the HIP backends (GPU): the operator classifies as exact.

The reference's own Triton autograd path keeps the probe flags but shows a smaller full-vs-first-order
meta-gradient difference than its exact backends (0.12 vs 0.20 in experiments/phase10/
phase10_summary.tsv:2,8), because its backward returns graph-less gradients. Here the HIP backends must
give the same flags and the same meta-gradients as the pure-PyTorch reference backend on the same
weights and task. The meta-gradient probe differentiates a create_graph'ed meta-gradient again, which is
third order through attention. Bars: float32 meta-gradients within 1e-4 relative (they pass through
two to three levels of differentiation and the inner SGD steps).
"""

import copy
import math

import pytest
import torch

from theria_amd.attention.custom import sdpa_custom
from theria_amd.maml.diagnostics import attention_second_order_ok, meta_gradient_probe
from theria_amd.models.tiny_attention import BackendAttentionModel, TinyAttentionConfig
from theria_amd.tasks import teacher_readout_task

pytestmark = pytest.mark.gpu

HIP = ("triton_full_fused", "hip")


@pytest.mark.parametrize("backend", HIP)
def test_attention_probe_hip(backend, hip_device):
    print(f"attention probe {backend}", flush=True)
    fn = lambda q, k, v: sdpa_custom(q, k, v, backend=backend)  # noqa: E731
    assert attention_second_order_ok(fn, device=hip_device, generator=torch.Generator().manual_seed(0))


@pytest.mark.parametrize("backend", HIP)
@pytest.mark.parametrize("inner_steps", [1, 2])
def test_meta_probe_hip_matches_reference_backend(backend, inner_steps, hip_device):
    print(f"meta probe {backend} k={inner_steps}", flush=True)
    torch.manual_seed(0)
    ref_model = BackendAttentionModel(TinyAttentionConfig(d_model=64, num_classes=5), backend="reference")
    ref_model = ref_model.to(hip_device)
    task = teacher_readout_task(support=16, query=16, T=32, D=64, num_classes=5, device=hip_device,
                                generator=torch.Generator().manual_seed(0))
    model = copy.deepcopy(ref_model)
    model.set_attention_backend(backend)
    ref = meta_gradient_probe(ref_model, task, inner_steps=inner_steps, inner_lr=0.4)
    got = meta_gradient_probe(model, task, inner_steps=inner_steps, inner_lr=0.4)
    for flag in ("second_order_path", "second_order_attn", "second_order_head"):
        assert got[flag] and ref[flag], flag
    assert math.isfinite(got["rel_diff_full_vs_fo"])
    assert got["rel_diff_full_vs_fo"] == pytest.approx(ref["rel_diff_full_vs_fo"], rel=1e-4)
    for key in ("meta_grad_full", "meta_grad_fo", "meta_curvature"):
        a, b = got[key].double(), ref[key].double()
        assert float((a - b).norm()) <= 1e-4 * float(b.norm()), key
