"""CPU tests of the pure-PyTorch reference surface (the theria API that needs no GPU).

Mirrors the intent of the reference's CPU tests: test_sdpa_reference_backward.py,
test_reference_jvp.py, test_reference_attention_hvp.py, test_sdpa_hvp.py, test_custom_attention_jvp.py,
test_custom_attention_hvp.py, test_attention_boundary.py, test_sdpa_gradcheck.py. The pure-PyTorch
functions are checked against the oracle and against torch.autograd.
"""

import math

import pytest
import torch

from oracle import sdpa_oracle as O
from theria_amd import sdpa
from theria_amd.attention.custom import sdpa_custom, sdpa_custom_hvp, sdpa_custom_jvp
from theria_amd.attention.reference import (
    reference_attention,
    sdpa_backward_reference,
    sdpa_hvp_reference,
    sdpa_jvp_reference,
)
from theria_amd.attention.reference_hvp_sdpa import sdpa_jvp as hvp_module_jvp
from theria_amd.autograd.sdpa_function import SDPAFunction


def _qkv(B, H, T, M, D, dtype=torch.float64, seed=0, grad=False):
    g = torch.Generator().manual_seed(seed)
    mk = lambda *s: torch.randn(*s, generator=g, dtype=dtype).requires_grad_(grad)  # noqa: E731
    return mk(B, H, T, D), mk(B, H, M, D), mk(B, H, M, D)


def test_reference_attention_matches_oracle():
    q, k, v = _qkv(2, 3, 7, 9, 8)
    torch.testing.assert_close(reference_attention(q, k, v), O.forward(q, k, v)[0], rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.float64, 1e-10)])
def test_explicit_backward_matches_autograd(dtype, tol):
    q, k, v = _qkv(1, 1, 8, 16, 16, dtype=dtype, grad=True)
    dout = torch.randn(1, 1, 8, 16, dtype=dtype)
    ref = torch.autograd.grad(reference_attention(q, k, v), (q, k, v), dout)
    mine = sdpa_backward_reference(q, k, v, dout, 1 / 4.0)
    for a, b in zip(mine, ref):
        torch.testing.assert_close(a, b, rtol=tol, atol=tol)


@pytest.mark.parametrize("shape", [(1, 1, 4, 4, 4), (1, 1, 4, 3, 4), (1, 2, 5, 6, 4)])
def test_reference_jvp_matches_autograd_functional(shape):
    B, H, T, M, D = shape
    q, k, v = _qkv(B, H, T, M, D)
    tq, tk, tv = _qkv(B, H, T, M, D, seed=5)
    _, ref = torch.autograd.functional.jvp(reference_attention, (q, k, v), (tq, tk, tv))
    torch.testing.assert_close(sdpa_jvp_reference(q, k, v, tq, tk, tv, 1 / math.sqrt(D)), ref, rtol=1e-9, atol=1e-9)
    torch.testing.assert_close(hvp_module_jvp(q, k, v, tq, tk, tv), ref, rtol=1e-9, atol=1e-9)


def test_reference_jvp_casts_back_to_input_dtype():
    q, k, v = _qkv(1, 1, 4, 4, 4, dtype=torch.float32)
    assert sdpa_jvp_reference(q, k, v, q, k, v, 0.5).dtype == torch.float32


def test_reference_hvp_sum_matches_oracle_and_fd():
    q, k, v = _qkv(1, 1, 3, 3, 4, grad=True)
    dq, dk, dv = _qkv(1, 1, 3, 3, 4, seed=3)
    hq, hk, hv = sdpa_hvp_reference(q, k, v, dq, dk, dv)
    for a, b in zip((hq, hk, hv), O.hvp_sum(q, k, v, dq, dk, dv)):
        torch.testing.assert_close(a, b, rtol=1e-10, atol=1e-12)
    eps = 1e-4

    def dd(t):
        qt, kt, vt = (x + t * d for x, d in zip((q, k, v), (dq, dk, dv)))
        g = torch.autograd.grad(SDPAFunction.apply(qt, kt, vt).sum(), (qt, kt, vt))
        return sum((a * d).sum() for a, d in zip(g, (dq, dk, dv)))

    fd = (dd(eps) - dd(-eps)) / (2 * eps)
    inner = sum((a * d).sum() for a, d in zip((hq, hk, hv), (dq, dk, dv)))
    assert torch.allclose(inner, fd, rtol=1e-3, atol=1e-4)


def test_sdpa_function_is_first_order_only():
    """theria.sdpa's backward is opaque: double backward raises (the reference's pinned boundary)."""
    q, k, v = _qkv(1, 1, 3, 3, 4, grad=True)
    grads = torch.autograd.grad(SDPAFunction.apply(q, k, v).sum(), (q, k, v), create_graph=True)
    with pytest.raises(RuntimeError):
        torch.autograd.grad(sum(g.sum() for g in grads), (q, k, v))
    torch.testing.assert_close(sdpa(q, k, v), reference_attention(q, k, v))


def test_sdpa_function_has_no_forward_mode():
    q, k, v = _qkv(1, 1, 3, 3, 4)
    with pytest.raises(Exception):
        with torch.autograd.forward_ad.dual_level():
            dual = torch.autograd.forward_ad.make_dual(q, torch.ones_like(q))
            SDPAFunction.apply(dual, k, v)


def test_sdpa_gradcheck():
    q, k, v = _qkv(1, 1, 3, 3, 2, grad=True)
    assert torch.autograd.gradcheck(sdpa, (q, k, v))
    assert torch.autograd.gradcheck(lambda a, b, c: sdpa_custom(a, b, c, backend="custom"), (q, k, v))


@pytest.mark.parametrize("backend", ["reference", "custom"])
def test_backends_support_double_backward(backend):
    q, k, v = _qkv(1, 1, 4, 4, 8, grad=True)
    u = [t.detach() / t.detach().norm() for t in _qkv(1, 1, 4, 4, 8, seed=2)]
    g = torch.autograd.grad(sdpa_custom(q, k, v, backend=backend).sum(), (q, k, v), create_graph=True)
    h = torch.autograd.grad(sum((a * b).sum() for a, b in zip(g, u)), (q, k, v))
    for a, b in zip(h, O.hvp_sum(q, k, v, *u)):
        torch.testing.assert_close(a, b, rtol=1e-9, atol=1e-10)


def test_custom_backend_jvp_hvp_helpers():
    q, k, v = _qkv(1, 1, 4, 4, 8)
    u = _qkv(1, 1, 4, 4, 8, seed=7)
    torch.testing.assert_close(sdpa_custom_jvp(q, k, v, *u), O.jvp(q, k, v, *u), rtol=1e-10, atol=1e-12)
    for a, b in zip(sdpa_custom_hvp(q, k, v, *u), O.hvp_sum(q, k, v, *u)):
        torch.testing.assert_close(a, b, rtol=1e-10, atol=1e-12)


def test_dispatcher_errors():
    q, k, v = _qkv(1, 1, 2, 2, 4)
    with pytest.raises(ValueError):
        sdpa_custom(q, k, v, backend="no_such_backend")
    for backend in ("triton_full_fused", "triton_qk", "triton_fast", "triton_qk_softmax"):
        with pytest.raises(AssertionError):
            sdpa_custom(q, k, v, backend=backend)  # CPU tensors: the HIP guards reject them
    with pytest.raises(AssertionError):
        sdpa_custom(q, k, v, backend="triton_qk", causal=True)
