"""CPU checks: the committed config-1 fixture still matches the oracle and the reference backends;
the MAML loops and tasks behave as theria's (tests/test_maml_full_vs_fo.py, test_maml_smoke.py)."""

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import sdpa_oracle as O
from theria_amd.attention.reference import reference_attention, sdpa_backward_reference, sdpa_jvp_reference
from theria_amd.maml import meta_loss_on_tasks
from theria_amd.models import BackendAttentionModel, MHAClassifier, MHAConfig, TinyAttentionConfig, TinyAttentionModel
from theria_amd.tasks import label_sequences, sample_token_count_task, teacher_readout_task

GOLDEN = Path(__file__).resolve().parent / "golden" / "c1_fp32.npz"


def _golden():
    z = np.load(GOLDEN, allow_pickle=False)
    inp = {k[3:]: torch.from_numpy(z[k]) for k in z.files if k.startswith("in_")}
    out = {k[4:]: torch.from_numpy(z[k]) for k in z.files if k.startswith("out_")}
    return inp, out


def test_golden_fixture_matches_oracle():
    inp, out = _golden()
    q, k, v = inp["q"], inp["k"], inp["v"]
    o, lse, m, l = O.forward(q, k, v)
    for name, val in dict(o=o, lse=lse, m=m, l=l).items():
        torch.testing.assert_close(val, out[name], rtol=1e-12, atol=1e-12)
    for name, val in zip(("dq", "dk", "dv"), O.backward(q, k, v, inp["dout"])):
        torch.testing.assert_close(val, out[name], rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(O.jvp(q, k, v, inp["tq"], inp["tk"], inp["tv"]), out["jvp"], rtol=1e-12, atol=1e-12)
    for name, val in zip(("hvp_q", "hvp_k", "hvp_v"), O.hvp_weighted_sum(q, k, v, inp["w"], inp["vq"], inp["vk"], inp["vv"])):
        torch.testing.assert_close(val, out[name], rtol=1e-12, atol=1e-12)


def test_golden_fixture_matches_reference_cpu_path_fp32():
    """Config 1 (B2 H2 S16 D8, float32) on the existing pure-PyTorch path, 1e-5."""
    inp, out = _golden()
    q, k, v = inp["q"], inp["k"], inp["v"]
    tol = dict(rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(reference_attention(q, k, v).double(), out["o"], **tol)
    for name, val in zip(("dq", "dk", "dv"), sdpa_backward_reference(q, k, v, inp["dout"], 1 / 8**0.5)):
        torch.testing.assert_close(val.double(), out[name], **tol)
    torch.testing.assert_close(sdpa_jvp_reference(q, k, v, inp["tq"], inp["tk"], inp["tv"], 1 / 8**0.5).double(), out["jvp"], **tol)
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
    g = torch.autograd.grad((reference_attention(qq, kk, vv) * inp["w"]).sum(), (qq, kk, vv), create_graph=True)
    h = torch.autograd.grad(sum((a * b).sum() for a, b in zip(g, (inp["vq"], inp["vk"], inp["vv"]))), (qq, kk, vv))
    for name, val in zip(("hvp_q", "hvp_k", "hvp_v"), h):
        torch.testing.assert_close(val.double(), out[name], **tol)


def _toy_tasks(n, D=8, seed=0):
    g = torch.Generator().manual_seed(seed)
    return [teacher_readout_task(support=4, query=4, T=6, D=D, num_classes=3, generator=g, dtype=torch.float64)
            for _ in range(n)]


def test_maml_full_differs_from_first_order():
    torch.manual_seed(0)
    model = TinyAttentionModel(TinyAttentionConfig(d_model=8, num_classes=3)).double()
    tasks = _toy_tasks(2)
    params = list(model.parameters())
    g_full = torch.autograd.grad(meta_loss_on_tasks(model, tasks, inner_lr=0.5, inner_steps=2), params)
    g_fo = torch.autograd.grad(meta_loss_on_tasks(model, tasks, inner_lr=0.5, inner_steps=2, fo=True), params)
    assert any(not torch.allclose(a, b) for a, b in zip(g_full, g_fo))
    for g in g_full:
        assert torch.isfinite(g).all()


@pytest.mark.parametrize("backend", ["reference", "custom"])
def test_backend_model_maml_smoke(backend):
    torch.manual_seed(0)
    model = BackendAttentionModel(TinyAttentionConfig(d_model=8, num_classes=3), backend=backend).double()
    loss, metrics = meta_loss_on_tasks(model, _toy_tasks(2), inner_lr=0.3, inner_steps=2, return_metrics=True)
    loss.backward()
    assert all(p.grad is not None and torch.isfinite(p.grad).all() for p in model.parameters())
    assert 0.0 <= metrics["post_adapt_acc"] <= 1.0


def test_fo_strict_blocks_inner_graph():
    torch.manual_seed(1)
    model = TinyAttentionModel(TinyAttentionConfig(d_model=8, num_classes=3)).double()
    loss = meta_loss_on_tasks(model, _toy_tasks(1), inner_steps=1, fo_strict=True)
    assert not loss.requires_grad  # strict FO detaches the adapted weights from theta


def test_token_count_task_labels_and_balance():
    g = torch.Generator().manual_seed(3)
    task, token_class = sample_token_count_task(generator=g)
    assert task.x_s.shape == (25, 64) and task.x_q.shape == (75, 64)
    assert torch.bincount(task.y_s, minlength=5).tolist() == [5] * 5
    assert torch.bincount(task.y_q, minlength=5).tolist() == [15] * 5
    assert torch.bincount(token_class, minlength=5).tolist() in ([7, 7, 6, 6, 6],)
    # brute-force relabel
    for x, y in ((task.x_s, task.y_s), (task.x_q, task.y_q)):
        for row, lab in zip(x, y):
            counts = [int((token_class[row] == c).sum()) for c in range(5)]
            assert lab == max(range(5), key=lambda c: (counts[c], -c))
    assert torch.equal(label_sequences(task.x_s, token_class, 5), task.y_s)


def test_mha_classifier_full_maml_on_reference_backend():
    torch.manual_seed(0)
    model = MHAClassifier(MHAConfig(), backend="reference")
    g = torch.Generator().manual_seed(0)
    tasks = [sample_token_count_task(generator=g, shots=2, queries=2)[0] for _ in range(2)]
    loss = meta_loss_on_tasks(model, tasks, inner_lr=0.4, inner_steps=2)
    loss.backward()
    assert all(torch.isfinite(p.grad).all() for p in model.parameters() if p.grad is not None)


def test_task_batched_maml_equals_sequential_loop():
    """meta_loss_on_tasks_batched is the same function of theta as the per-task loop (float64)."""
    from theria_amd.maml import meta_loss_on_tasks, meta_loss_on_tasks_batched
    from theria_amd.models import MHAClassifier, MHAConfig
    from theria_amd.tasks import sample_token_count_task

    torch.manual_seed(0)
    model = MHAClassifier(MHAConfig(), backend="reference").double()
    g = torch.Generator().manual_seed(3)
    tasks = [sample_token_count_task(generator=g)[0] for _ in range(3)]
    params = list(model.parameters())
    one = {k: v.unsqueeze(0) for k, v in model.named_parameters()}
    torch.testing.assert_close(model.forward_batched(one, tasks[0].x_q.unsqueeze(0))[0], model(tasks[0].x_q))
    for kw in (dict(fo=False), dict(fo=True), dict(fo=True, fo_strict=True)):
        a = meta_loss_on_tasks(model, tasks, inner_lr=0.4, inner_steps=2, **kw)
        b = meta_loss_on_tasks_batched(model, tasks, inner_lr=0.4, inner_steps=2, **kw)
        torch.testing.assert_close(b, a, rtol=1e-12, atol=1e-12)
        assert a.requires_grad == b.requires_grad
        if not a.requires_grad:  # fo_strict: the adapted weights are cut from theta in both
            continue
        ga = torch.autograd.grad(a, params, allow_unused=True)
        gb = torch.autograd.grad(b, params, allow_unused=True)
        for x, y in zip(ga, gb):
            if x is None or y is None:
                assert x is None and y is None
            else:
                torch.testing.assert_close(y, x, rtol=1e-10, atol=1e-12)
