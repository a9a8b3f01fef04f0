"""The HIP operator through torch.autograd: gradients, forward-mode JVP, HVP by double backward,
the reference-named entry points, and the second-order boundary (GPU).

Config 4: B8 H8 S512 D64 in float32 and bfloat16; primals ~ N(0,1), tangents ~ N(0, 0.1^2);
HVP of 0.5 ||O - T||^2 with T, v ~ N(0,1) via double backward through the explicit kernels.
Bars (tests/bars.py): float32 1e-5 abs/rel, bfloat16/float16 2e-2 abs plus one output rounding unit relative.
"""

import math

import pytest
import torch

import bars
from oracle import sdpa_oracle as O
from theria_amd.attention import (
    TritonFusedSDPAFunction,
    hip_sdpa,
    sdpa_bwd_dk,
    sdpa_bwd_dq,
    sdpa_bwd_dv,
    sdpa_jvp,
    triton_sdpa_fused,
)
from theria_amd.attention.custom import sdpa_custom
from theria_amd.attention.hvp_utils import hvp_fd_vjp

pytestmark = pytest.mark.gpu


tol = bars.tol


def close(gpu, ref, dtype, what):
    bars.close(gpu, ref, what=what, **tol(dtype))


def make(shape, dtype, dev, seed, std=1.0, grad=False):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(*shape, generator=g) * std).to(dtype)
    return x.to(dev).requires_grad_(grad), x.double()


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("causal", [False, True])
def test_autograd_first_order(dt, causal, hip_device):
    dev = hip_device
    q, qc = make((2, 3, 100, 64), dt, dev, 1, grad=True)
    k, kc = make((2, 3, 100, 64), dt, dev, 2, grad=True)
    v, vc = make((2, 3, 100, 64), dt, dev, 3, grad=True)
    do, doc = make((2, 3, 100, 64), dt, dev, 4)
    o = hip_sdpa(q, k, v, causal=causal)
    close(o, O.forward(qc, kc, vc, causal=causal)[0], dt, "O")
    grads = torch.autograd.grad(o, (q, k, v), do)
    for name, a, b in zip(("dQ", "dK", "dV"), grads, O.backward(qc, kc, vc, doc, causal=causal)):
        close(a, b, dt, name)


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_config4_jvp_forward_mode(dt, hip_device):
    dev = hip_device
    B, H, S, D = 8, 8, 512, 64
    print(f"[autograd] config4 jvp {dt}", flush=True)
    q, qc = make((B, H, S, D), dt, dev, 31)
    k, kc = make((B, H, S, D), dt, dev, 32)
    v, vc = make((B, H, S, D), dt, dev, 33)
    tq, tqc = make((B, H, S, D), dt, dev, 34, std=0.1)
    tk, tkc = make((B, H, S, D), dt, dev, 35, std=0.1)
    tv, tvc = make((B, H, S, D), dt, dev, 36, std=0.1)
    o, jv = torch.func.jvp(lambda a, b, c: hip_sdpa(a, b, c), (q, k, v), (tq, tk, tv))
    ref = O.jvp(qc, kc, vc, tqc, tkc, tvc)
    close(jv, ref, dt, "JVP")
    with torch.autograd.forward_ad.dual_level():
        dual = torch.autograd.forward_ad.make_dual(q, tq)
        tangent = torch.autograd.forward_ad.unpack_dual(hip_sdpa(dual, k, v)).tangent
    close(tangent, O.jvp(qc, kc, vc, tqc, None, None), dt, "JVP(forward_ad, q only)")


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_config4_hvp_double_backward(dt, hip_device):
    dev = hip_device
    B, H, S, D = 8, 8, 512, 64
    print(f"[autograd] config4 hvp {dt}", flush=True)
    q, qc = make((B, H, S, D), dt, dev, 41, grad=True)
    k, kc = make((B, H, S, D), dt, dev, 42, grad=True)
    v, vc = make((B, H, S, D), dt, dev, 43, grad=True)
    T_, Tc = make((B, H, S, D), dt, dev, 44)
    vq, vqc = make((B, H, S, D), dt, dev, 45)
    vk, vkc = make((B, H, S, D), dt, dev, 46)
    vv, vvc = make((B, H, S, D), dt, dev, 47)
    out = hip_sdpa(q, k, v)
    loss = 0.5 * ((out.float() - T_.float()) ** 2).sum()
    g = torch.autograd.grad(loss, (q, k, v), create_graph=True)
    dot = sum((a.float() * b.float()).sum() for a, b in zip(g, (vq, vk, vv)))
    hvp = torch.autograd.grad(dot, (q, k, v))
    ref = O.hvp_quadratic(qc, kc, vc, Tc, vqc, vkc, vvc)
    for name, a, b in zip(("Hq", "Hk", "Hv"), hvp, ref):
        close(a, b, dt, name)


def test_config1_hvp_weighted_sum_fp32(hip_device):
    dev = hip_device
    q, qc = make((2, 2, 16, 8), torch.float32, dev, 51, grad=True)
    k, kc = make((2, 2, 16, 8), torch.float32, dev, 52, grad=True)
    v, vc = make((2, 2, 16, 8), torch.float32, dev, 53, grad=True)
    W, Wc = make((2, 2, 16, 8), torch.float32, dev, 54)
    u = [make((2, 2, 16, 8), torch.float32, dev, 55 + i) for i in range(3)]
    g = torch.autograd.grad((hip_sdpa(q, k, v) * W).sum(), (q, k, v), create_graph=True)
    h = torch.autograd.grad(sum((a * b[0]).sum() for a, b in zip(g, u)), (q, k, v))
    for name, a, b in zip(("Hq", "Hk", "Hv"), h, O.hvp_weighted_sum(qc, kc, vc, Wc, *(x[1] for x in u))):
        close(a, b, torch.float32, name)


def test_autograd_functional_jvp_uses_double_backward(hip_device):
    """torch.autograd.functional.jvp runs the double-backward trick: it exercises G_dO."""
    dev = hip_device
    q, qc = make((1, 2, 24, 32), torch.float32, dev, 61)
    k, kc = make((1, 2, 24, 32), torch.float32, dev, 62)
    v, vc = make((1, 2, 24, 32), torch.float32, dev, 63)
    t = [make((1, 2, 24, 32), torch.float32, dev, 64 + i) for i in range(3)]
    _, jv = torch.autograd.functional.jvp(lambda a, b, c: hip_sdpa(a, b, c), (q, k, v), tuple(x[0] for x in t))
    close(jv, O.jvp(qc, kc, vc, *(x[1] for x in t)), torch.float32, "functional.jvp")


def _third_order(fn, q, k, v):
    """grad of sum(g2) where g2 = grad ||grad ||O||^2||^2: a third derivative of O through attention."""
    g = torch.autograd.grad(fn(q, k, v).pow(2).sum(), (q, k, v), create_graph=True)
    g2 = torch.autograd.grad(sum(x.pow(2).sum() for x in g), (q, k, v), create_graph=True)
    return torch.autograd.grad(sum(x.sum() for x in g2), (q, k, v))


@pytest.mark.parametrize("causal", [False, True])
def test_third_order_matches_oracle(causal, hip_device):
    """Differentiating a create_graph'ed double backward (orders >= 3) is exact, not a dropped term."""
    dev = hip_device
    q, qc = make((1, 2, 9, 16), torch.float32, dev, 71, grad=True)
    k, kc = make((1, 2, 12, 16), torch.float32, dev, 72, grad=True)
    v, vc = make((1, 2, 12, 16), torch.float32, dev, 73, grad=True)
    got = _third_order(lambda a, b, c: hip_sdpa(a, b, c, causal=causal), q, k, v)
    ref = _third_order(lambda a, b, c: O.autograd_attention(a, b, c, causal=causal),
                       *(t.clone().requires_grad_(True) for t in (qc, kc, vc)))
    # the same derivative of textbook attention in float32 (theria's pure-PyTorch path): its error against float64
    # sets the bar where float32 arithmetic itself cannot reach 1e-5 (third derivatives sum many large products)
    ref32 = _third_order(lambda a, b, c: O.autograd_attention(a, b, c, causal=causal),
                         *(t.float().clone().requires_grad_(True) for t in (qc, kc, vc)))
    for name, a, b, c in zip(("q", "k", "v"), got, ref, ref32):
        err32 = float((c.double() - b).abs().max())
        bars.close(a, b, rtol=1e-5, atol=max(1e-5, 2 * err32), what=f"d3/d{name} (float32 reference error {err32:.2e})")


def test_autograd_functional_hvp(hip_device):
    """torch.autograd.functional.hvp differentiates the double backward with respect to its cotangent."""
    dev = hip_device
    q, qc = make((1, 2, 24, 32), torch.float32, dev, 81)
    k, kc = make((1, 2, 24, 32), torch.float32, dev, 82)
    v, vc = make((1, 2, 24, 32), torch.float32, dev, 83)
    w, wc = make((1, 2, 24, 32), torch.float32, dev, 84)
    u = [make((1, 2, 24, 32), torch.float32, dev, 85 + i) for i in range(3)]
    _, h = torch.autograd.functional.hvp(lambda a, b, c: (hip_sdpa(a, b, c) * w).sum(), (q, k, v),
                                         tuple(x[0] for x in u))
    for name, a, b in zip(("q", "k", "v"), h, O.hvp_weighted_sum(qc, kc, vc, wc, *(x[1] for x in u))):
        close(a, b, torch.float32, f"hvp {name}")


def test_second_order_probe_sees_attention_curvature(hip_device):
    """The Phase-11 probe (_attention_second_order_ok): grad of ||grad||^2 through SDPA alone is nonzero."""
    dev = hip_device
    torch.manual_seed(0)
    q = torch.randn(1, 1, 1, 4, device=dev, requires_grad=True)
    k = torch.randn(1, 1, 2, 4, device=dev, requires_grad=True)
    v = torch.randn(1, 1, 2, 4, device=dev, requires_grad=True)
    out = sdpa_custom(q, k, v, backend="triton_full_fused")
    g1 = torch.autograd.grad(out.sum(), (q, k, v), retain_graph=True, create_graph=True)
    g2 = torch.autograd.grad(sum(x.pow(2).sum() for x in g1), (q, k, v), allow_unused=True)
    assert any(x is not None and float(x.abs().sum()) > 1e-12 for x in g2)
    # and it equals the exact value from the oracle
    qc, kc, vc = (t.detach().double().cpu() for t in (q, k, v))
    g1c = O.backward(qc, kc, vc, torch.ones(1, 1, 1, 4, dtype=torch.float64))
    ref = O.double_backward(qc, kc, vc, torch.ones(1, 1, 1, 4, dtype=torch.float64), *(2 * x for x in g1c))
    for a, b in zip(g2, ref[:3]):
        close(a, b, torch.float32, "probe")


# ---- reference-named entry points (the drop-in surface) ----------------------------------------


@pytest.mark.parametrize("shape", [(1, 1, 32, 32, 32), (4, 8, 128, 128, 64), (1, 1, 1, 1, 32)])
def test_sdpa_custom_fused_matches_reference_backend(shape, hip_device):
    B, H, T, M, D = shape
    torch.manual_seed(0)
    q = torch.randn(B, H, T, D, device=hip_device, dtype=torch.float16)
    k = torch.randn(B, H, M, D, device=hip_device, dtype=torch.float16)
    v = torch.randn(B, H, M, D, device=hip_device, dtype=torch.float16)
    fused = sdpa_custom(q, k, v, backend="triton_full_fused")
    assert fused.dtype == q.dtype
    ref = O.forward(q.double().cpu(), k.double().cpu(), v.double().cpu())[0]
    close(fused, ref, torch.float16, "sdpa_custom fused")


def test_triton_sdpa_fused_returns_fp32_and_stats(hip_device):
    torch.manual_seed(0)
    q, k, v = (torch.randn(2, 3, 50, 64, device=hip_device, dtype=torch.bfloat16) for _ in range(3))
    o, m, l = triton_sdpa_fused(q, k, v, return_stats=True)
    assert o.dtype == torch.float32 and m.shape == (2, 3, 50) and l.shape == (2, 3, 50)
    Or, _, mr, lr = O.forward(q.double().cpu(), k.double().cpu(), v.double().cpu())
    close(o, Or, torch.bfloat16, "O")
    torch.testing.assert_close(m.double().cpu(), mr, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(l.double().cpu(), lr, rtol=1e-5, atol=1e-5)
    o2 = TritonFusedSDPAFunction.apply(q, k, v)
    assert o2.dtype == torch.float32


@pytest.mark.parametrize("shape", [(1, 1, 32, 32, 32), (2, 4, 128, 128, 64)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_explicit_backward_with_torch_stats(shape, dtype, hip_device):
    """The reference's kernel tests: stats (m, l) computed by torch, inputs fed as given."""
    B, H, T, M, D = shape
    torch.manual_seed(0)
    dev = hip_device
    q = torch.randn(B, H, T, D, device=dev, dtype=torch.float16).to(dtype)
    k = torch.randn(B, H, M, D, device=dev, dtype=torch.float16).to(dtype)
    v = torch.randn(B, H, M, D, device=dev, dtype=torch.float16).to(dtype)
    dout = torch.randn(B, H, T, D, device=dev, dtype=torch.float16).to(dtype)
    scale = 1.0 / D**0.5
    scores = torch.matmul(q.float(), k.float().transpose(-2, -1)) * scale
    m = scores.max(dim=-1).values
    l = torch.exp(scores - m.unsqueeze(-1)).sum(dim=-1)
    ref = O.backward(*(t.double().cpu() for t in (q, k, v, dout)), scale)
    for name, fn, r in (
        ("dq", lambda: sdpa_bwd_dq(q, k, v, dout, m, l, scale), ref[0]),
        ("dk", lambda: sdpa_bwd_dk(q, k, v, dout, m, l, scale), ref[1]),
        ("dv", lambda: sdpa_bwd_dv(q, k, dout, m, l, scale), ref[2]),
    ):
        out = fn()
        assert out.dtype == dtype
        close(out, r, dtype, name)


def test_explicit_jvp_matches_frozen_stats_oracle(hip_device):
    torch.manual_seed(0)
    dev = hip_device
    q, k, v = (torch.randn(2, 2, 64, 64, device=dev, dtype=torch.float16) for _ in range(3))
    dq, dk, dv = (torch.randn_like(q) for _ in range(3))
    _, m, l = triton_sdpa_fused(q, k, v, return_stats=True)
    out = sdpa_jvp(q, k, v, dq, dk, dv, m, l, 1 / 8.0)
    ref = O.frozen_jvp(*(t.double().cpu() for t in (q, k, v, dq, dk, dv, m, l)), 1 / 8.0)
    close(out, ref, torch.float16, "sdpa_jvp")


def test_explicit_guards_raise_assertion(hip_device):
    q = torch.randn(1, 1, 4, 8, device=hip_device)
    m = torch.zeros(1, 1, 4, device=hip_device)
    with pytest.raises(AssertionError):
        sdpa_bwd_dq(q, q, q, q, m, m.unsqueeze(-1), 0.3)  # wrong stats shape
    with pytest.raises(AssertionError):
        sdpa_jvp(q, q, q, q, q, q, m, m, 0.3)  # l <= 0
    with pytest.raises(AssertionError):
        sdpa_bwd_dq(q.double(), q.double(), q.double(), q.double(), m, m + 1, 0.3)  # float64 unsupported


def test_hvp_fd_vjp_agrees_with_exact_hvp(hip_device):
    torch.manual_seed(0)
    dev = hip_device
    q, k, v = (torch.randn(1, 1, 8, 8, device=dev) for _ in range(3))
    d = [torch.randn_like(q) for _ in range(3)]
    fd = hvp_fd_vjp(q, k, v, *d, eps=1e-2)
    exact = O.hvp_sum(*(t.double().cpu() for t in (q, k, v, *d)))
    cos = torch.nn.functional.cosine_similarity(torch.cat([x.double().cpu().flatten() for x in fd]), torch.cat([x.flatten() for x in exact]), dim=0)
    assert float(cos) > 0.99


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("T,M,D,Dv,causal", [(37, 45, 32, 64, False), (37, 45, 64, 24, True), (37, 45, 16, 128, False),
                                            (200, 260, 64, 40, False)])
def test_value_head_dim_differs(T, M, D, Dv, causal, dt, hip_device):
    """Dv != D through hip_sdpa: O, first order, HVP by double backward and forward-mode JVP. The last shape
    takes the pipelined 16-bit kernels (more than 128 queries, head dim 64 after padding)."""
    dev = hip_device
    print(f"Dv != D: {dt} T={T} M={M} D={D} Dv={Dv} causal={causal}", flush=True)
    q, qc = make((2, 2, T, D), dt, dev, 91, grad=True)
    k, kc = make((2, 2, M, D), dt, dev, 92, grad=True)
    v, vc = make((2, 2, M, Dv), dt, dev, 93, grad=True)
    w, wc = make((2, 2, T, Dv), dt, dev, 94)
    u = [make(t.shape, dt, dev, 95 + i) for i, t in enumerate((q, k, v))]
    o = hip_sdpa(q, k, v, causal=causal)
    assert o.shape == (2, 2, T, Dv)
    close(o, O.forward(qc, kc, vc, causal=causal)[0], dt, "O")
    g = torch.autograd.grad((o * w).sum(), (q, k, v), create_graph=True)
    for name, a, b in zip(("dQ", "dK", "dV"), g, O.backward(qc, kc, vc, wc, causal=causal)):
        close(a, b, dt, name)
    h = torch.autograd.grad(sum((a * b[0]).sum() for a, b in zip(g, u)), (q, k, v))
    for name, a, b in zip(("q", "k", "v"), h, O.hvp_weighted_sum(qc, kc, vc, wc, *(x[1] for x in u), causal=causal)):
        close(a, b, dt, f"hvp {name}")
    _, jv = torch.func.jvp(lambda a, b, c: hip_sdpa(a, b, c, causal=causal), (q.detach(), k.detach(), v.detach()),
                           tuple(x[0] for x in u))
    close(jv, O.jvp(qc, kc, vc, *(x[1] for x in u), causal=causal), dt, "jvp")
    assert sdpa_custom(q, k, v, backend="hip", causal=causal).shape[-1] == Dv
    with pytest.raises(AssertionError):
        sdpa_custom(q, k, v, backend="triton_full_fused")


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("causal", [False, True])
def test_kernel_only_hvp_matches_oracle_and_autograd(dt, causal, hip_device):
    """hip_sdpa_hvp (no autograd graph) for sum(O), <W, O> and 0.5 ||O - T||^2, against the oracle and,
    for the quadratic loss, against autograd double backward through hip_sdpa."""
    from theria_amd.autograd.hip_sdpa import hip_sdpa_hvp

    dev = hip_device
    print(f"kernel-only HVP {dt} causal={causal}", flush=True)
    q, qc = make((2, 2, 70, 64), dt, dev, 101)
    k, kc = make((2, 2, 90, 64), dt, dev, 102)
    v, vc = make((2, 2, 90, 64), dt, dev, 103)
    w, wc = make((2, 2, 70, 64), dt, dev, 104)
    t_, tc = make((2, 2, 70, 64), dt, dev, 105)
    u = [make(x.shape, dt, dev, 106 + i, std=0.1) for i, x in enumerate((q, k, v))]
    uv, uc = [x[0] for x in u], [x[1] for x in u]
    ones = torch.ones_like(wc)
    cases = [
        ("sum", {}, O.hvp_weighted_sum(qc, kc, vc, ones, *uc, causal=causal)),
        ("weight", {"weight": w}, O.hvp_weighted_sum(qc, kc, vc, wc, *uc, causal=causal)),
        ("quadratic", {"target": t_}, O.hvp_quadratic(qc, kc, vc, tc, *uc, causal=causal)),
    ]
    for name, kw, ref in cases:
        got = hip_sdpa_hvp(q, k, v, *uv, causal=causal, **kw)
        for part, a, b in zip("qkv", got, ref):
            close(a, b, dt, f"hvp {name} {part}")
    qg, kg, vg = (x.detach().clone().requires_grad_(True) for x in (q, k, v))
    o = hip_sdpa(qg, kg, vg, causal=causal)
    g = torch.autograd.grad(0.5 * ((o.float() - t_.float()) ** 2).sum(), (qg, kg, vg), create_graph=True)
    ag = torch.autograd.grad(sum((a.float() * b.float()).sum() for a, b in zip(g, uv)), (qg, kg, vg))
    for part, a, b in zip("qkv", hip_sdpa_hvp(q, k, v, *uv, target=t_, causal=causal), ag):
        close(a, b.detach().double().cpu(), dt, f"hvp vs autograd {part}")


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_kernel_only_hvp_with_peaked_rows(dt, D, causal, hip_device):
    """hip_sdpa_hvp of 0.5 ||O - T||^2 against the float64 oracle on inputs with rows whose probability sits
    on one key: the 16-bit double backward's exact row pass and split column products run there."""
    from theria_amd.autograd.hip_sdpa import hip_sdpa_hvp

    dev = hip_device
    print(f"kernel-only HVP, peaked rows, {dt} D{D} causal={causal}", flush=True)
    B, H, T, M = 2, 2, 160, 192
    g = torch.Generator().manual_seed(211)
    qh, kh = torch.randn(B, H, T, D, generator=g), torch.randn(B, H, M, D, generator=g)
    for r in (5, 77, 150):
        qh[:, :, r] = kh[:, :, r]  # score ~ sqrt(D) on key r against N(0, 1) elsewhere
    q, k = qh.to(dt).to(dev), kh.to(dt).to(dev)
    qc, kc = q.double().cpu(), k.double().cpu()
    v, vc = make((B, H, M, D), dt, dev, 212)
    t_, tc = make((B, H, T, D), dt, dev, 213)
    u = [make(x.shape, dt, dev, 214 + i, std=0.1) for i, x in enumerate((q, k, v))]
    uv, uc = [x[0] for x in u], [x[1] for x in u]
    ref = O.hvp_quadratic(qc, kc, vc, tc, *uc, causal=causal)
    for part, a, b in zip("qkv", hip_sdpa_hvp(q, k, v, *uv, target=t_, causal=causal), ref):
        close(a, b, dt, f"hvp {part}")
