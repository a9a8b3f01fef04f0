"""Full MAML (create_graph=True) through the HIP operator vs the same model on the pure-PyTorch
"reference" backend (GPU). BASELINE config 5 (reduced meta-batch): 2-layer, d_model 64, 4-head
token-count classifier, 5 inner SGD steps at lr 0.4. The meta-gradients must agree (attention's
second-order terms are kept), and full MAML must differ from first-order MAML.
"""

import copy

import pytest
import torch

from theria_amd.maml import meta_loss_on_tasks, meta_loss_on_tasks_batched
from theria_amd.models import BackendAttentionModel, MHAClassifier, MHAConfig, TinyAttentionConfig
from theria_amd.tasks import sample_token_count_task, task_sampler

pytestmark = pytest.mark.gpu


def _flat(grads):
    return torch.cat([g.reshape(-1) for g in grads if g is not None]).double()


def _metagrad(model, tasks, fo=False, inner_steps=5, inner_lr=0.4):
    params = [p for p in model.parameters() if p.requires_grad]
    loss = meta_loss_on_tasks(model, tasks, inner_lr=inner_lr, inner_steps=inner_steps, fo=fo)
    return loss.detach(), _flat(torch.autograd.grad(loss, params, allow_unused=True))


def test_config5_full_maml_metagradient_matches_reference_backend(hip_device):
    dev = hip_device
    torch.manual_seed(0)
    ref_model = MHAClassifier(MHAConfig(), backend="reference").to(dev)
    hip_model = copy.deepcopy(ref_model)
    hip_model.set_attention_backend("hip")
    g = torch.Generator().manual_seed(0)
    tasks = [sample_token_count_task(generator=g, device=dev)[0] for _ in range(4)]
    l_ref, g_ref = _metagrad(ref_model, tasks)
    l_hip, g_hip = _metagrad(hip_model, tasks)
    torch.testing.assert_close(l_hip.double(), l_ref.double(), rtol=1e-4, atol=1e-5)
    rel = float((g_hip - g_ref).norm() / g_ref.norm())
    cos = float(torch.nn.functional.cosine_similarity(g_hip, g_ref, dim=0))
    print(f"[maml] config5 rel_l2={rel:.3e} cosine={cos:.8f}", flush=True)
    assert rel < 1e-3 and cos > 0.99999
    _, g_fo = _metagrad(hip_model, tasks, fo=True)
    assert float((g_hip - g_fo).norm() / g_hip.norm()) > 1e-3


def test_phase10_model_full_vs_reference(hip_device):
    """The Phase-10 model (Tq = 1 query, H = 1, D = 64, T = 32) with backend 'triton_fused'."""
    dev = hip_device
    torch.manual_seed(0)
    ref_model = BackendAttentionModel(TinyAttentionConfig(), backend="reference").to(dev)
    hip_model = copy.deepcopy(ref_model)
    hip_model.set_attention_backend("triton_fused")
    torch.manual_seed(1)
    tasks = [task_sampler(device=dev) for _ in range(2)]
    _, g_ref = _metagrad(ref_model, tasks, inner_lr=0.1)
    _, g_hip = _metagrad(hip_model, tasks, inner_lr=0.1)
    rel = float((g_hip - g_ref).norm() / g_ref.norm())
    print(f"[maml] phase10 rel_l2={rel:.3e}", flush=True)
    assert rel < 1e-3


def test_config5_task_batched_full_maml_matches_reference_loop(hip_device):
    """All tasks adapted at once (one SDPA call over tasks x sequences) through the HIP operator, against
    the per-task loop on the pure-PyTorch backend: the same meta-loss and meta-gradient."""
    dev = hip_device
    torch.manual_seed(0)
    ref_model = MHAClassifier(MHAConfig(), backend="reference").to(dev)
    hip_model = copy.deepcopy(ref_model)
    hip_model.set_attention_backend("hip")
    g = torch.Generator().manual_seed(0)
    tasks = [sample_token_count_task(generator=g, device=dev)[0] for _ in range(4)]
    params = list(hip_model.parameters())
    for fo in (False, True):
        l_ref, g_ref = _metagrad(ref_model, tasks, fo=fo)
        loss = meta_loss_on_tasks_batched(hip_model, tasks, inner_lr=0.4, inner_steps=5, fo=fo)
        g_hip = _flat(torch.autograd.grad(loss, params, allow_unused=True))
        torch.testing.assert_close(loss.detach().double(), l_ref.double(), rtol=1e-4, atol=1e-5)
        rel = float((g_hip - g_ref).norm() / g_ref.norm())
        print(f"[maml] task-batched fo={fo} rel_l2={rel:.3e}", flush=True)
        assert rel < 1e-3
