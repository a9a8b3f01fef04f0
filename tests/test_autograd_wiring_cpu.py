"""The autograd wiring of the HIP operator (SDPAOp / SDPABackwardOp), checked on the CPU.

The kernel calls (_ops.fwd, _ops.bwd, _ops.bwd_bwd, _ops.jvp) are replaced by the float64 oracle, so
what is tested is the graph logic alone: which derivative each node returns, and that derivatives of
every order equal autograd through textbook attention (oracle.autograd_attention). It also pins which
path runs: up to second order the double-backward "kernel" is called, and only when the double backward
must itself be differentiable does the PyTorch restatement of the backward map take over.
"""

import importlib

import pytest
import torch

from oracle import sdpa_oracle as O
from theria_amd import _ops

H = importlib.import_module("theria_amd.autograd.hip_sdpa")


@pytest.fixture
def kernels(monkeypatch):
    calls = {"bwd_bwd": 0}

    def fwd(q, k, v, scale, causal, out_fp32=False, stats=False, checked=True):
        o, lse, m, l = O.forward(q, k, v, scale, causal)
        return o.to(q.dtype), lse, (m if stats else None), (l if stats else None)

    def bwd(q, k, v, o, lse, dout, scale, causal, need_dq=True, need_dk=True, out=None, checked=True):
        dq, dk, dv = O.backward(q, k, v, dout, scale, causal)
        return dq, dk, dv, (dout.double() * o.double()).sum(-1)

    def bwd_bwd(q, k, v, o, dout, lse, delta, gq, gk, gv, scale, causal, noalloc=False, out=None, checked=True):
        calls["bwd_bwd"] += 1
        z = lambda t, like: torch.zeros_like(like) if t is None else t  # noqa: E731
        return O.double_backward(q, k, v, dout, z(gq, q), z(gk, k), z(gv, v), scale, causal)

    def jvp(q, k, v, o, lse, tq, tk, tv, scale, causal, normalize=True, checked=True):
        z = lambda t, like: torch.zeros_like(like) if t is None else t  # noqa: E731
        return O.jvp(q, k, v, z(tq, q), z(tk, k), z(tv, v), scale, causal)

    for name, fn in (("fwd", fwd), ("bwd", bwd), ("bwd_bwd", bwd_bwd), ("jvp", jvp)):
        monkeypatch.setattr(_ops, name, fn)
    return calls


def _inputs(seed, T=5, M=7, D=4):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(1, 2, n, D, generator=g, dtype=torch.float64) for n in (T, M, M)]


def _pair(seed, **kw):
    base = _inputs(seed, **kw)
    return [t.clone().requires_grad_(True) for t in base], [t.clone().requires_grad_(True) for t in base]


def _hip(causal):
    return lambda q, k, v: H.hip_sdpa(q, k, v, causal=causal)


def _ref(causal):
    return lambda q, k, v: O.autograd_attention(q, k, v, causal=causal)


def _close(a, b, tol=1e-10):
    for x, y in zip(a, b):
        torch.testing.assert_close(x, y, rtol=tol, atol=tol)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("create_graph", [False, True])
def test_hvp_of_quadratic_loss(kernels, causal, create_graph):
    (a, b), t = _pair(1), _inputs(2)
    u = _inputs(3)

    def hvp(fn, qkv):
        loss = 0.5 * (fn(*qkv) - t[0].new_ones(1)).pow(2).sum()
        g = torch.autograd.grad(loss, qkv, create_graph=True)
        return torch.autograd.grad(sum((x * w).sum() for x, w in zip(g, u)), qkv, create_graph=create_graph)

    _close(hvp(_hip(causal), a), hvp(_ref(causal), b))
    # without create_graph the double backward is the kernel; with it, the differentiable restatement
    assert (kernels["bwd_bwd"] > 0) == (not create_graph)


@pytest.mark.parametrize("causal", [False, True])
def test_third_order(kernels, causal):
    def third(fn, qkv):
        g = torch.autograd.grad(fn(*qkv).pow(2).sum(), qkv, create_graph=True)
        g2 = torch.autograd.grad(sum(x.pow(2).sum() for x in g), qkv, create_graph=True)
        return torch.autograd.grad(sum(x.sum() for x in g2), qkv)

    a, b = _pair(4)
    _close(third(_hip(causal), a), third(_ref(causal), b), tol=1e-9)


def test_fourth_order_along_a_direction(kernels):
    def fourth(fn, qkv):
        g = torch.autograd.grad(fn(*qkv).sum(), qkv, create_graph=True)
        for _ in range(3):
            g = torch.autograd.grad(sum(x.pow(2).sum() for x in g), qkv, create_graph=True)
        return g

    a, b = _pair(5, T=3, M=4, D=3)
    _close(fourth(_hip(False), a), fourth(_ref(False), b), tol=1e-8)


def test_functional_hvp_and_jvp(kernels):
    q, k, v = _inputs(6)
    w = _inputs(7)[0]
    u = _inputs(8)
    for fn_h, fn_r in ((_hip(False), _ref(False)),):
        _, h1 = torch.autograd.functional.hvp(lambda a, b, c: (fn_h(a, b, c) * w).sum(), (q, k, v), tuple(u))
        _, h2 = torch.autograd.functional.hvp(lambda a, b, c: (fn_r(a, b, c) * w).sum(), (q, k, v), tuple(u))
        _close(h1, h2)
        _, j1 = torch.autograd.functional.jvp(fn_h, (q, k, v), tuple(u))
        _, j2 = torch.autograd.functional.jvp(fn_r, (q, k, v), tuple(u))
        _close((j1,), (j2,))


def test_forward_mode_in_both_function_forms(kernels, monkeypatch):
    """Outside torch.func transforms hip_sdpa takes the ctx-first Function (no per-call signature binding),
    inside them the setup_context one: both give the JVP kernel's tangent, and reverse mode through the
    ctx-first form gives the oracle's gradient."""
    q, k, v = _inputs(10)
    tq, tk, tv = _inputs(11)
    used = []

    def spy(name, apply):  # records which Function's apply ran, then runs it
        return classmethod(lambda cls, *args: (used.append(name), apply(*args))[1])

    for cls in (H.SDPAOp, H._SDPAOpEager):
        monkeypatch.setattr(cls, "apply", spy(cls.__name__, cls.apply))
    with torch.autograd.forward_ad.dual_level():
        duals = [torch.autograd.forward_ad.make_dual(x, t) for x, t in ((q, tq), (k, tk), (v, tv))]
        t_eager = torch.autograd.forward_ad.unpack_dual(H.hip_sdpa(*duals)).tangent
    assert used == ["_SDPAOpEager"]
    _, t_func = torch.func.jvp(lambda a, b, c: H.hip_sdpa(a, b, c), (q, k, v), (tq, tk, tv))
    assert used[0] == "_SDPAOpEager" and set(used[1:]) == {"SDPAOp"}  # torch.func re-enters apply per level
    expect = O.jvp(q, k, v, tq, tk, tv, q.shape[-1] ** -0.5, False)
    _close((t_eager, t_func), (expect, expect))
    a, b = _pair(12)
    g1 = torch.autograd.grad(H.hip_sdpa(*a).pow(2).sum(), a)
    g2 = torch.autograd.grad(_ref(False)(*b).pow(2).sum(), b)
    _close(g1, g2)


def test_gradient_of_dout_path_is_not_double_counted(kernels):
    """dO = 2 O depends on q, k, v: differentiating the create_graph'ed double backward must take
    partial derivatives of the backward map and leave the dO path to G_dO."""
    (a, b) = _pair(9)

    def second(fn, qkv):
        g = torch.autograd.grad(fn(*qkv).pow(2).sum(), qkv, create_graph=True)
        return torch.autograd.grad(sum(x.pow(2).sum() for x in g), qkv, create_graph=True)

    _close(second(_hip(False), a), second(_ref(False), b))


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("loss", ["sum", "weight", "target"])
def test_graphed_hvp_body_is_the_autograd_hvp(kernels, loss, causal):
    """The body GraphedSDPAHVP captures (run here eagerly, without a graph) is the HVP of its loss: sum(O),
    <W, O> or 0.5 ||O - T||^2, against autograd's double backward through textbook attention. The second
    gradient runs the double-backward kernel (grad mode is off there)."""
    from theria_amd.autograd.graphed_hvp import GraphedSDPAHVP

    q, k, v = _inputs(3)
    u = _inputs(4)
    extra = _inputs(5)[0]  # shaped like O
    G = object.__new__(GraphedSDPAHVP)
    G.causal, G.scale = causal, _ops.default_scale(q.shape[-1])
    G.q, G.k, G.v = (t.clone().requires_grad_(True) for t in (q, k, v))
    G.vq, G.vk, G.vv = u
    G.target = extra if loss == "target" else None
    G.weight = extra if loss == "weight" else None
    got = G._body()
    assert kernels["bwd_bwd"] == 1

    qr, kr, vr = (t.clone().requires_grad_(True) for t in (q, k, v))
    o = O.autograd_attention(qr, kr, vr, causal=causal)
    losses = {"sum": lambda: o.sum(), "weight": lambda: (o * extra).sum(),
              "target": lambda: 0.5 * ((o - extra) ** 2).sum()}
    L = losses[loss]()
    g = torch.autograd.grad(L, (qr, kr, vr), create_graph=True)
    want = torch.autograd.grad(g, (qr, kr, vr), grad_outputs=tuple(u))
    _close(got, want)


def test_graphed_hvp_refuses_cpu_inputs_and_two_losses():
    from theria_amd.autograd import GraphedSDPAHVP

    q, k, v = _inputs(1)
    with pytest.raises(ValueError, match="weight or target"):
        GraphedSDPAHVP(q, k, v, q, k, v, target=q, weight=q)
    with pytest.raises(ValueError, match="GPU"):
        GraphedSDPAHVP(q, k, v, q, k, v)
