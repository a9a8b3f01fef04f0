"""Full MAML (create_graph=True) through the HIP operator vs the same model on the pure-PyTorch
"reference" backend (GPU). Config 5 at its full meta-batch of 16 tasks: 2-layer, d_model 64, 4-head
token-count classifier, 5 inner SGD steps at lr 0.4. The meta-gradients must agree to a relative L2 of
1e-5 (attention's second-order terms are kept; float32 accumulation differences between the two backends
measure ~4e-6), and full MAML must differ from first-order MAML.
"""

import copy

import pytest
import torch

from theria_amd.maml import meta_loss_on_tasks, meta_loss_on_tasks_batched
from theria_amd.models import BackendAttentionModel, MHAClassifier, MHAConfig, TinyAttentionConfig
from theria_amd.tasks import sample_token_count_task, teacher_readout_task

pytestmark = pytest.mark.gpu

META_BATCH = 16
REL_L2 = 1e-5


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
    tasks = [sample_token_count_task(generator=g, device=dev)[0] for _ in range(META_BATCH)]
    l_ref, g_ref = _metagrad(ref_model, tasks)
    l_hip, g_hip = _metagrad(hip_model, tasks)
    torch.testing.assert_close(l_hip.double(), l_ref.double(), rtol=1e-4, atol=1e-5)
    rel = float((g_hip - g_ref).norm() / g_ref.norm())
    cos = float(torch.nn.functional.cosine_similarity(g_hip, g_ref, dim=0))
    print(f"[maml] config5 rel_l2={rel:.3e} cosine={cos:.8f}", flush=True)
    assert rel < REL_L2 and cos > 0.99999
    _, g_fo = _metagrad(hip_model, tasks, fo=True)
    assert float((g_hip - g_fo).norm() / g_hip.norm()) > 1e-3


def test_phase10_model_full_vs_reference(hip_device):
    """The Phase-10 model (Tq = 1 query, H = 1, D = 64, T = 32) with backend 'triton_fused'."""
    dev = hip_device
    torch.manual_seed(0)
    ref_model = BackendAttentionModel(TinyAttentionConfig(), backend="reference").to(dev)
    hip_model = copy.deepcopy(ref_model)
    hip_model.set_attention_backend("triton_fused")
    g = torch.Generator().manual_seed(1)
    tasks = [teacher_readout_task(generator=g, device=dev) for _ in range(2)]
    _, g_ref = _metagrad(ref_model, tasks, inner_lr=0.1)
    _, g_hip = _metagrad(hip_model, tasks, inner_lr=0.1)
    rel = float((g_hip - g_ref).norm() / g_ref.norm())
    print(f"[maml] phase10 rel_l2={rel:.3e}", flush=True)
    assert rel < REL_L2


def test_config5_task_batched_full_maml_matches_reference_loop(hip_device):
    """All tasks adapted at once (one SDPA call over tasks x sequences) through the HIP operator, against
    the per-task loop on the pure-PyTorch backend: the same meta-loss and meta-gradient."""
    dev = hip_device
    torch.manual_seed(0)
    ref_model = MHAClassifier(MHAConfig(), backend="reference").to(dev)
    hip_model = copy.deepcopy(ref_model)
    hip_model.set_attention_backend("hip")
    g = torch.Generator().manual_seed(0)
    tasks = [sample_token_count_task(generator=g, device=dev)[0] for _ in range(META_BATCH)]
    params = list(hip_model.parameters())
    for fo in (False, True):
        l_ref, g_ref = _metagrad(ref_model, tasks, fo=fo)
        loss = meta_loss_on_tasks_batched(hip_model, tasks, inner_lr=0.4, inner_steps=5, fo=fo)
        g_hip = _flat(torch.autograd.grad(loss, params, allow_unused=True))
        torch.testing.assert_close(loss.detach().double(), l_ref.double(), rtol=1e-4, atol=1e-5)
        rel = float((g_hip - g_ref).norm() / g_ref.norm())
        print(f"[maml] task-batched fo={fo} rel_l2={rel:.3e}", flush=True)
        assert rel < REL_L2


def test_graphed_task_batched_meta_step_matches_eager(hip_device):
    """GraphedMetaStep replays equal eager task-batched meta-steps (parameters after every step), with
    new tasks copied in before each replay and eager work between the replays."""
    from theria_amd.maml import GraphedMetaStep

    dev = hip_device
    torch.manual_seed(0)
    eager = MHAClassifier(MHAConfig(), backend="hip").to(dev)
    graphed = copy.deepcopy(eager)
    g = torch.Generator().manual_seed(5)
    batches = [[sample_token_count_task(generator=g, device=dev)[0] for _ in range(4)] for _ in range(4)]
    opt_e = torch.optim.Adam(eager.parameters(), lr=1e-3, capturable=True)
    opt_g = torch.optim.Adam(graphed.parameters(), lr=1e-3, capturable=True)
    step = GraphedMetaStep(graphed, opt_g, batches[0], inner_lr=0.4, inner_steps=2)
    for i, tasks in enumerate(batches):
        print(f"[graphed meta-step] step {i}", flush=True)
        opt_e.zero_grad(set_to_none=True)
        loss_e = meta_loss_on_tasks_batched(eager, tasks, inner_lr=0.4, inner_steps=2)
        loss_e.backward()
        opt_e.step()
        loss_g = step.step(tasks)
        torch.cuda.synchronize()
        torch.testing.assert_close(loss_g, loss_e.detach(), rtol=1e-5, atol=1e-6)
        for (name, a), b in zip(eager.named_parameters(), graphed.parameters()):
            torch.testing.assert_close(b, a, rtol=1e-5, atol=1e-6, msg=lambda m: f"step {i} {name}: {m}")


def test_task_batched_meta_step_issues_no_memset(hip_device):
    """The step GraphedMetaStep captures must contain no device memset (memset nodes in a replayed graph
    are not trusted): profile one eager step at config 5's meta-batch and count memset activities."""
    from torch.profiler import ProfilerActivity, profile

    dev = hip_device
    torch.manual_seed(0)
    model = MHAClassifier(MHAConfig(), backend="hip").to(dev)
    g = torch.Generator().manual_seed(9)
    tasks = [sample_token_count_task(generator=g, device=dev)[0] for _ in range(16)]
    opt = torch.optim.Adam(model.parameters(), lr=1e-3, capturable=True)

    def step():
        opt.zero_grad(set_to_none=True)
        meta_loss_on_tasks_batched(model, tasks, inner_lr=0.4, inner_steps=5).backward()
        opt.step()

    step()
    torch.cuda.synchronize()
    with profile(activities=[ProfilerActivity.CPU, ProfilerActivity.CUDA]) as prof:
        step()
        torch.cuda.synchronize()
    memsets = [e.name for e in prof.events() if "memset" in e.name.lower() or "fillbuffer" in e.name.lower()]
    assert not memsets, f"{len(memsets)} memset activities, e.g. {memsets[:3]}"
