"""Pins every function of oracle/sdpa_oracle.py (CPU, float64) to something the mathematics fixes:
torch.autograd / torch.func on the textbook expression, gradcheck, central finite differences,
closed-form special cases and invariants. A planted mistake in the oracle must fail these checks.
"""

import math

import pytest
import torch

from oracle import sdpa_oracle as O

D64 = torch.float64


def _rand(*shape, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=D64)


def _qkv(B=2, H=2, T=5, M=7, D=4, seed=0):
    q = _rand(B, H, T, D, seed=seed)
    k = _rand(B, H, M, D, seed=seed + 1)
    v = _rand(B, H, M, D, seed=seed + 2)
    return q, k, v


CASES = [(2, 2, 5, 7, 4, False), (1, 3, 6, 6, 8, True), (2, 2, 16, 16, 8, False), (1, 1, 1, 9, 3, False)]


@pytest.mark.parametrize("B,H,T,M,D,causal", CASES)
def test_forward_matches_textbook_and_logsumexp(B, H, T, M, D, causal):
    q, k, v = _qkv(B, H, T, M, D)
    o, lse, m, l = O.forward(q, k, v, causal=causal)
    torch.testing.assert_close(o, O.autograd_attention(q, k, v, causal=causal), rtol=1e-12, atol=1e-12)
    S = (q @ k.transpose(-2, -1)) / math.sqrt(D)
    if causal:
        S = S.masked_fill(~torch.ones(T, M, dtype=torch.bool).tril(), float("-inf"))
    torch.testing.assert_close(lse, torch.logsumexp(S, dim=-1), rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(m, S.max(dim=-1).values, rtol=1e-14, atol=1e-14)
    torch.testing.assert_close(lse, m + torch.log(l), rtol=1e-12, atol=1e-12)
    P = O.probs(q, k, causal=causal)
    torch.testing.assert_close(P.sum(-1), torch.ones(B, H, T, dtype=D64), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("B,H,T,M,D,causal", CASES)
def test_backward_matches_autograd(B, H, T, M, D, causal):
    q, k, v = (t.requires_grad_(True) for t in _qkv(B, H, T, M, D))
    do = _rand(B, H, T, D, seed=9)
    ref = torch.autograd.grad(O.autograd_attention(q, k, v, causal=causal), (q, k, v), do)
    for a, b in zip(O.backward(q, k, v, do, causal=causal), ref):
        torch.testing.assert_close(a, b, rtol=1e-10, atol=1e-12)


def test_delta_identity():
    """z_i = rowsum(dP o P) equals dO_i . O_i (the backward's row term computed once per row)."""
    q, k, v = _qkv(2, 2, 6, 9, 5)
    do = _rand(2, 2, 6, 5, seed=4)
    P = O.probs(q, k)
    z = ((do @ v.transpose(-2, -1)) * P).sum(-1)
    o, _, _, _ = O.forward(q, k, v)
    torch.testing.assert_close(z, (do * o).sum(-1), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("B,H,T,M,D,causal", CASES)
def test_jvp_matches_forward_mode(B, H, T, M, D, causal):
    q, k, v = _qkv(B, H, T, M, D)
    tq, tk, tv = _rand(*q.shape, seed=11), _rand(*k.shape, seed=12), _rand(*v.shape, seed=13)
    _, ref = torch.func.jvp(lambda a, b, c: O.autograd_attention(a, b, c, causal=causal), (q, k, v), (tq, tk, tv))
    torch.testing.assert_close(O.jvp(q, k, v, tq, tk, tv, causal=causal), ref, rtol=1e-10, atol=1e-12)


def test_frozen_jvp_equals_true_jvp_at_exact_stats():
    q, k, v = _qkv(1, 2, 4, 6, 3)
    tq, tk, tv = _rand(*q.shape, seed=1), _rand(*k.shape, seed=2), _rand(*v.shape, seed=3)
    _, _, m, l = O.forward(q, k, v)
    s = 1 / math.sqrt(3)
    torch.testing.assert_close(O.frozen_jvp(q, k, v, tq, tk, tv, m, l, s), O.jvp(q, k, v, tq, tk, tv), rtol=1e-12, atol=1e-12)
    # with perturbed stats the frozen JVP is the JVP of P = exp(S - m)/l at fixed (m, l): check by autograd
    m2, l2 = m + 0.1, l * 1.3

    def f(a, b, c):
        P = torch.exp((a @ b.transpose(-2, -1)) * s - m2.unsqueeze(-1)) / l2.unsqueeze(-1)
        return P @ c

    _, ref = torch.func.jvp(f, (q, k, v), (tq, tk, tv))
    Pf = torch.exp((q @ k.transpose(-2, -1)) * s - m2.unsqueeze(-1)) / l2.unsqueeze(-1)
    G = (tq @ k.transpose(-2, -1) + q @ tk.transpose(-2, -1)) * s
    centred = ref - ((G * Pf).sum(-1, keepdim=True) * (Pf @ v))  # the contract centres dS (docs/phase9.md:33)
    torch.testing.assert_close(O.frozen_jvp(q, k, v, tq, tk, tv, m2, l2, s), centred, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("causal", [False, True])
def test_frozen_backward_closed_form(causal):
    """frozen_backward at the exact lse is the true gradient; with lse + c (a per-row shift, i.e. l scaled by
    e^c) P is scaled by e^-c per row, and the frozen formula then differs from the true gradient by the
    closed form below (dS_f = e^-c (dS + (1 - e^-c) z P), with z = rowsum(dP P) of the true P)."""
    q, k, v = _qkv(2, 2, 6, 7, 5, seed=4)
    do = _rand(*q.shape, seed=8)
    s = 1 / math.sqrt(5)
    _, lse, _, _ = O.forward(q, k, v, s, causal)
    ref = O.backward(q, k, v, do, s, causal)
    for a_, b_ in zip(O.frozen_backward(q, k, v, do, lse, s, causal), ref):
        torch.testing.assert_close(a_, b_, rtol=1e-12, atol=1e-12)
    c = _rand(*lse.shape, seed=9).abs() * 0.5
    dq_f, dk_f, dv_f = O.frozen_backward(q, k, v, do, lse + c, s, causal)
    e = torch.exp(-c).unsqueeze(-1)
    P = O.probs(q, k, s, causal)
    z = ((do @ v.transpose(-2, -1)) * P).sum(-1, keepdim=True)
    dq_t, dk_t, dv_t = ref
    torch.testing.assert_close(dv_f, O.backward(q, k, v, do * e, s, causal)[2], rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(dq_f, e * (dq_t + s * (1 - e) * z * (P @ k)), rtol=1e-12, atol=1e-12)
    dS = P * ((do @ v.transpose(-2, -1)) - z)
    torch.testing.assert_close(dk_f, s * ((e * (dS + (1 - e) * z * P)).transpose(-2, -1) @ q), rtol=1e-12, atol=1e-12)
    # the shift term is not negligible here: a frozen formula without it (e^-c times the true dQ) is far off
    assert not torch.allclose(dq_f, e * dq_t, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("B,H,T,M,D,causal", CASES)
def test_double_backward_matches_autograd(B, H, T, M, D, causal):
    q, k, v = (t.requires_grad_(True) for t in _qkv(B, H, T, M, D))
    do = _rand(B, H, T, D, seed=5).requires_grad_(True)
    gq, gk, gv = _rand(*q.shape, seed=6), _rand(*k.shape, seed=7), _rand(*v.shape, seed=8)
    first = torch.autograd.grad(O.autograd_attention(q, k, v, causal=causal), (q, k, v), do, create_graph=True)
    ref = torch.autograd.grad(first, (q, k, v, do), (gq, gk, gv))
    for a, b in zip(O.double_backward(q, k, v, do, gq, gk, gv, causal=causal), ref):
        torch.testing.assert_close(a, b, rtol=1e-10, atol=1e-12)


def test_double_backward_gdo_is_jvp():
    """G_dO of the double backward equals the JVP with the cotangents as tangents (it is linear in dO)."""
    q, k, v = _qkv(2, 1, 5, 6, 4)
    do = _rand(2, 1, 5, 4, seed=3)
    gq, gk, gv = _rand(*q.shape, seed=4), _rand(*k.shape, seed=5), _rand(*v.shape, seed=6)
    torch.testing.assert_close(O.double_backward(q, k, v, do, gq, gk, gv)[3], O.jvp(q, k, v, gq, gk, gv), rtol=1e-12, atol=1e-12)


def test_gradcheck_and_gradgradcheck_of_textbook():
    q, k, v = (t.requires_grad_(True) for t in _qkv(1, 1, 3, 4, 2))
    assert torch.autograd.gradcheck(O.autograd_attention, (q, k, v))
    assert torch.autograd.gradgradcheck(O.autograd_attention, (q, k, v))


def test_hvp_quadratic_matches_autograd_and_fd():
    q, k, v = (t.requires_grad_(True) for t in _qkv(2, 2, 6, 6, 4))
    T_ = _rand(2, 2, 6, 4, seed=20)
    vq, vk, vv = _rand(*q.shape, seed=21), _rand(*k.shape, seed=22), _rand(*v.shape, seed=23)

    def loss(a, b, c):
        return 0.5 * ((O.autograd_attention(a, b, c) - T_) ** 2).sum()

    g = torch.autograd.grad(loss(q, k, v), (q, k, v), create_graph=True)
    ref = torch.autograd.grad(sum((x * y).sum() for x, y in zip(g, (vq, vk, vv))), (q, k, v))
    mine = O.hvp_quadratic(q, k, v, T_, vq, vk, vv)
    for a, b in zip(mine, ref):
        torch.testing.assert_close(a, b, rtol=1e-10, atol=1e-12)
    # central finite difference of the directional derivative of the gradient
    eps = 1e-5

    def dirderiv(t):
        a, b, c = (x.detach() + t * d for x, d in zip((q, k, v), (vq, vk, vv)))
        gr = O.backward(a, b, c, O.forward(a, b, c)[0] - T_)
        return sum((x * d).sum() for x, d in zip(gr, (vq, vk, vv)))

    fd = (dirderiv(eps) - dirderiv(-eps)) / (2 * eps)
    inner = sum((x * d).sum() for x, d in zip(mine, (vq, vk, vv)))
    assert abs(float(fd - inner)) < 1e-6 * max(1.0, abs(float(inner)))


def test_hvp_sum_matches_autograd_and_is_symmetric():
    q, k, v = (t.requires_grad_(True) for t in _qkv(2, 1, 8, 8, 16))
    u = [_rand(*t.shape, seed=30 + i) for i, t in enumerate((q, k, v))]
    w = [_rand(*t.shape, seed=40 + i) for i, t in enumerate((q, k, v))]
    g = torch.autograd.grad(O.autograd_attention(q, k, v).sum(), (q, k, v), create_graph=True)
    ref = torch.autograd.grad(sum((x * y).sum() for x, y in zip(g, u)), (q, k, v))
    hu = O.hvp_sum(q, k, v, *u)
    for a, b in zip(hu, ref):
        torch.testing.assert_close(a, b, rtol=1e-10, atol=1e-12)
    hw = O.hvp_sum(q, k, v, *w)
    lhs = sum((a * b).sum() for a, b in zip(w, hu))
    rhs = sum((a * b).sum() for a, b in zip(u, hw))
    assert abs(float(lhs - rhs)) < 1e-10 * max(1.0, abs(float(lhs)))


def test_hvp_weighted_sum_matches_autograd():
    q, k, v = (t.requires_grad_(True) for t in _qkv(2, 2, 16, 16, 8))
    W = _rand(2, 2, 16, 8, seed=50)
    u = [_rand(*t.shape, seed=51 + i) for i, t in enumerate((q, k, v))]
    g = torch.autograd.grad((O.autograd_attention(q, k, v) * W).sum(), (q, k, v), create_graph=True)
    ref = torch.autograd.grad(sum((x * y).sum() for x, y in zip(g, u)), (q, k, v))
    for a, b in zip(O.hvp_weighted_sum(q, k, v, W, *u), ref):
        torch.testing.assert_close(a, b, rtol=1e-10, atol=1e-12)


def test_special_case_single_key():
    """M = 1: P = 1, O = V (broadcast), dQ = dK = 0, dV = sum over queries of dO."""
    q, k, v = _qkv(1, 2, 5, 1, 4)
    o, lse, m, l = O.forward(q, k, v)
    torch.testing.assert_close(o, v.expand_as(o), rtol=0, atol=1e-15)
    torch.testing.assert_close(l, torch.ones_like(l), rtol=0, atol=0)
    do = _rand(1, 2, 5, 4, seed=2)
    dq, dk, dv = O.backward(q, k, v, do)
    assert float(dq.abs().max()) < 1e-15 and float(dk.abs().max()) < 1e-15
    torch.testing.assert_close(dv, do.sum(-2, keepdim=True), rtol=1e-14, atol=1e-14)


def test_special_case_constant_keys():
    """Identical keys give uniform P: O is the mean of V over keys for every query."""
    q = _rand(1, 1, 4, 3)
    k = _rand(1, 1, 1, 3).expand(1, 1, 6, 3).contiguous()
    v = _rand(1, 1, 6, 3, seed=5)
    o, _, _, _ = O.forward(q, k, v)
    torch.testing.assert_close(o, v.mean(-2, keepdim=True).expand_as(o), rtol=1e-14, atol=1e-14)


def test_causal_first_row_is_v0():
    """Causal: query 0 sees only key 0, so O_0 = V_0 and the row's lse is its single score."""
    q, k, v = _qkv(1, 1, 5, 5, 4)
    o, lse, _, _ = O.forward(q, k, v, causal=True)
    torch.testing.assert_close(o[..., 0, :], v[..., 0, :], rtol=1e-14, atol=1e-14)
    torch.testing.assert_close(lse[..., 0], (q[..., 0, :] * k[..., 0, :]).sum(-1) / 2.0, rtol=1e-14, atol=1e-14)


def test_causal_first_row_second_order_terms_vanish():
    """Causal query 0 sees one key, so P = 1 on that row whatever q_0 is: dQ_0 = 0 and the double
    backward's G_Q row 0 = 0 (the row's softmax has no derivative), while G_Q of later rows is not."""
    q, k, v = _qkv(1, 2, 6, 6, 4)
    do = _rand(1, 2, 6, 4, seed=7)
    gq, gk, gv = (_rand(1, 2, 6, 4, seed=8 + i) for i in range(3))
    dq, _, _ = O.backward(q, k, v, do, causal=True)
    assert float(dq[..., 0, :].abs().max()) < 1e-14
    G = O.double_backward(q, k, v, do, gq, gk, gv, causal=True)
    assert float(G[0][..., 0, :].abs().max()) < 1e-13
    assert float(G[0][..., 1:, :].abs().max()) > 1e-3


def test_planted_mistake_in_double_backward_is_caught():
    """Dropping the -r o dP term of Gbar_P (a plausible derivation slip) must break autograd parity."""
    q, k, v = (t.requires_grad_(True) for t in _qkv(1, 2, 5, 6, 4))
    do = _rand(1, 2, 5, 4, seed=5).requires_grad_(True)
    gq, gk, gv = _rand(*q.shape, seed=6), _rand(*k.shape, seed=7), _rand(*v.shape, seed=8)
    first = torch.autograd.grad(O.autograd_attention(q, k, v), (q, k, v), do, create_graph=True)
    ref = torch.autograd.grad(first, (q, k, v, do), (gq, gk, gv))

    def mutated(q, k, v, dout, gq, gk, gv):
        s = 1 / math.sqrt(q.shape[-1])
        P = O.probs(q, k, s)
        dP = dout @ v.transpose(-2, -1)
        z = (P * dP).sum(-1, keepdim=True)
        Gam = s * (gq @ k.transpose(-2, -1) + q @ gk.transpose(-2, -1))
        W = dout @ gv.transpose(-2, -1)
        Gbar_P = Gam * (dP - z) + W  # missing "- r * dP"
        Gbar_S = P * (Gbar_P - (P * Gbar_P).sum(-1, keepdim=True))
        dS = P * (dP - z)
        return s * (Gbar_S @ k + dS @ gk)

    bad = mutated(*(t.detach() for t in (q, k, v, do)), gq, gk, gv)
    assert not torch.allclose(bad, ref[0], rtol=1e-6, atol=1e-8)
    torch.testing.assert_close(O.double_backward(q, k, v, do, gq, gk, gv)[0], ref[0], rtol=1e-10, atol=1e-12)
