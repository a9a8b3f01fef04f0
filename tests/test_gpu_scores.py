"""GPU parity of the partial-fusion score backends (HIP Q K^T and fused Q K^T + softmax) against the oracle.

Mirrors the reference's own tests of these backends (tests/test_triton_qk.py, test_triton_gradcheck.py,
test_triton_fast_relaxed.py, test_triton_double_backward.py, test_triton_forward_matches_reference.py) and
adds ragged, strided and 16-bit cases. Bars: scores and probabilities from float32 inputs within 1e-5
abs/rel of the float64 oracle on the same inputs; float32 scores from 16-bit inputs within 1e-5 as well
(16-bit products are exact in float32, so only the float32 summation rounds); scores rounded to the
16-bit input dtype, and O of the 16-bit partial-fusion backends, within 2e-2 plus one rounding unit of the dtype
relative (tests/bars.py).
"""

import pytest
import torch

from bars import tol
from oracle import sdpa_oracle as O
from theria_amd import _ops
from theria_amd.attention.custom import sdpa_custom, sdpa_custom_jvp
from theria_amd.attention.scores import TritonQKFunction, triton_qk, triton_qk_fast, triton_qk_softmax

pytestmark = pytest.mark.gpu

F32 = dict(rtol=1e-5, atol=1e-5)


def make(shape, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g).to(dtype)
    return x.to("cuda"), x.double()


SHAPES = [
    # B, H, T, M, D
    (1, 1, 4, 4, 8),
    (2, 2, 37, 53, 24),
    (1, 3, 1, 70, 64),
    (2, 1, 65, 1, 16),
    (1, 2, 130, 257, 128),
    (2, 4, 256, 384, 64),
    # 16-bit head dims <= 64 store 128 keys per round: a partial last round (six subtiles) and nine tiles
    (1, 2, 100, 190, 64),
    (1, 1, 300, 520, 32),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shape", SHAPES)
def test_qk_scores_match_oracle(dtype, shape):
    B, H, T, M, D = shape
    print(f"qk_scores {dtype} {shape}", flush=True)
    q, q64 = make((B, H, T, D), dtype, 1)
    k, k64 = make((B, H, M, D), dtype, 2)
    ref = q64 @ k64.transpose(-2, -1)
    s = triton_qk(q, k)
    torch.cuda.synchronize()
    assert s.dtype == torch.float32 and s.shape == (B, H, T, M)
    torch.testing.assert_close(s.double().cpu(), ref, **F32)
    if dtype != torch.float32:
        sf = triton_qk_fast(q, k)
        assert sf.dtype == dtype
        torch.testing.assert_close(sf.double().cpu(), ref, **tol(dtype))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shape", SHAPES)
def test_qk_softmax_matches_oracle(dtype, shape):
    B, H, T, M, D = shape
    print(f"qk_softmax {dtype} {shape}", flush=True)
    q, q64 = make((B, H, T, D), dtype, 3)
    k, k64 = make((B, H, M, D), dtype, 4)
    p = triton_qk_softmax(q, k)
    torch.cuda.synchronize()
    assert p.dtype == torch.float32 and p.shape == (B, H, T, M)
    assert not p.requires_grad
    torch.testing.assert_close(p.double().cpu(), O.probs(q64, k64), **F32)
    torch.testing.assert_close(p.double().sum(-1).cpu(), torch.ones(B, H, T, dtype=torch.float64), **F32)


def test_scores_strided_views():
    # (B, T, H, D) storage read as (B, H, T, D): row stride H*D, head stride D
    print("qk_scores strided views", flush=True)
    B, H, T, M, D = 2, 3, 45, 29, 32
    qs, qs64 = make((B, T, H, D), torch.bfloat16, 5)
    ks, ks64 = make((B, M, H, D), torch.bfloat16, 6)
    q, k = qs.transpose(1, 2), ks.transpose(1, 2)
    q64, k64 = qs64.transpose(1, 2), ks64.transpose(1, 2)
    torch.testing.assert_close(_ops.qk_scores(q, k).double().cpu(), q64 @ k64.transpose(-2, -1), **F32)
    torch.testing.assert_close(_ops.qk_softmax(q, k, D ** -0.5).double().cpu(), O.probs(q64, k64), **F32)


def test_scores_large_magnitude_rows():
    # rows whose scaled scores span a wide range: the online max of pass 1 must keep exp from overflowing
    print("qk_softmax large magnitudes", flush=True)
    q, q64 = make((1, 2, 33, 64), torch.float32, 7)
    k, k64 = make((1, 2, 300, 64), torch.float32, 8)
    q, q64 = q * 30, q64 * 30
    p = triton_qk_softmax(q, k)
    assert torch.isfinite(p).all()
    torch.testing.assert_close(p.double().cpu(), O.probs(q64, k64), **F32)


def test_scores_empty_keys_and_queries():
    q, _ = make((1, 2, 0, 16), torch.float16, 9)
    k, _ = make((1, 2, 5, 16), torch.float16, 10)
    assert triton_qk(q, k).shape == (1, 2, 0, 5)
    q2, _ = make((1, 2, 3, 16), torch.float16, 11)
    k2, _ = make((1, 2, 0, 16), torch.float16, 12)
    assert triton_qk(q2, k2).shape == (1, 2, 3, 0)
    assert triton_qk_softmax(q2, k2).shape == (1, 2, 3, 0)


def test_triton_qk_backend_end_to_end_fp32():
    # forward and first-order gradients of the "triton_qk" composition against the oracle
    print("triton_qk backend fp32", flush=True)
    B, H, T, D = 2, 2, 37, 24
    q, q64 = make((B, H, T, D), torch.float32, 13)
    k, k64 = make((B, H, T + 6, D), torch.float32, 14)
    v, v64 = make((B, H, T + 6, D), torch.float32, 15)
    do, do64 = make((B, H, T, D), torch.float32, 16)
    for t in (q, k, v):
        t.requires_grad_(True)
    for backend in ("triton_qk", "triton_ref", "triton"):
        o = sdpa_custom(q, k, v, backend=backend)
        torch.testing.assert_close(o.detach().double().cpu(), O.forward(q64, k64, v64)[0], **F32)
        g = torch.autograd.grad(o, (q, k, v), do)
        for a, b in zip(g, O.backward(q64, k64, v64, do64)):
            torch.testing.assert_close(a.double().cpu(), b, **F32)


def test_triton_qk_backend_double_backward_fp32():
    # reference test_triton_double_backward.py, plus the value: HVP of sum(O) against the oracle
    print("triton_ref double backward", flush=True)
    q, q64 = make((1, 2, 9, 8), torch.float32, 17)
    k, k64 = make((1, 2, 11, 8), torch.float32, 18)
    v, v64 = make((1, 2, 11, 8), torch.float32, 19)
    u = [make(t.shape, torch.float32, 20 + i) for i, t in enumerate((q, k, v))]
    for t in (q, k, v):
        t.requires_grad_(True)
    g = torch.autograd.grad(sdpa_custom(q, k, v, backend="triton_ref").sum(), (q, k, v), create_graph=True)
    h = torch.autograd.grad(sum((a * b[0]).sum() for a, b in zip(g, u)), (q, k, v))
    ref = O.hvp_sum(q64, k64, v64, *(b[1] for b in u))
    for a, b in zip(h, ref):
        assert torch.isfinite(a).all()
        torch.testing.assert_close(a.double().cpu(), b, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_triton_ref_and_fast_match_reference_16bit(dtype):
    # reference test_triton_forward_matches_reference.py (triton_ref, 2e-2) and
    # test_triton_fast_relaxed.py (triton_fast, cosine > 0.99 and 1e-1)
    print(f"triton_ref/triton_fast {dtype}", flush=True)
    q, q64 = make((2, 2, 40, 64), dtype, 23)
    k, k64 = make((2, 2, 70, 64), dtype, 24)
    v, v64 = make((2, 2, 70, 64), dtype, 25)
    ref = O.forward(q64, k64, v64)[0]
    o = sdpa_custom(q, k, v, backend="triton_ref")
    assert o.dtype == dtype
    torch.testing.assert_close(o.double().cpu(), ref, **tol(dtype))
    of = sdpa_custom(q, k, v, backend="triton_fast").double().cpu()
    cos = torch.nn.functional.cosine_similarity(of.flatten(), ref.flatten(), dim=0)
    assert cos > 0.99
    torch.testing.assert_close(of, ref, rtol=1e-1, atol=1e-1)
    os_ = sdpa_custom(q, k, v, backend="triton_qk_softmax")
    torch.testing.assert_close(os_.double().cpu(), ref, **tol(dtype))


def test_triton_qk_softmax_backend_fp32_and_no_qk_gradient():
    print("triton_qk_softmax backend fp32", flush=True)
    q, q64 = make((1, 2, 21, 32), torch.float32, 26)
    k, k64 = make((1, 2, 35, 32), torch.float32, 27)
    v, v64 = make((1, 2, 35, 32), torch.float32, 28)
    q.requires_grad_(True)
    v.requires_grad_(True)
    o = sdpa_custom(q, k, v, backend="triton_qk_softmax")
    torch.testing.assert_close(o.detach().double().cpu(), O.forward(q64, k64, v64)[0], **F32)
    # as in the reference (the probabilities come from a plain kernel call), only v receives a gradient
    gq, gv = torch.autograd.grad(o.sum(), (q, v), allow_unused=True)
    assert gq is None
    torch.testing.assert_close(gv.double().cpu(), O.backward(q64, k64, v64, torch.ones_like(q64))[2], **F32)


def test_triton_qk_gradcheck_fp32():
    # reference test_triton_gradcheck.py: float32 gradcheck as a coarse check (eps 1e-3, atol 1e-3, rtol 1e-2)
    q, _ = make((1, 1, 2, 3), torch.float32, 29)
    k, _ = make((1, 1, 2, 3), torch.float32, 30)
    q.requires_grad_(True)
    k.requires_grad_(True)
    assert torch.autograd.gradcheck(lambda a, b: TritonQKFunction.apply(a, b), (q, k), eps=1e-3, atol=1e-3,
                                    rtol=1e-2, fast_mode=True)


def test_triton_ref_jvp_matches_finite_difference():
    # reference test_triton_forward_matches_reference.py:38-73: frozen-stats JVP against a central
    # difference of the triton_ref backend, float32, cosine > 0.99 and 5e-2
    q, _ = make((1, 1, 4, 8), torch.float32, 31)
    k, _ = make((1, 1, 4, 8), torch.float32, 32)
    v, _ = make((1, 1, 4, 8), torch.float32, 33)
    d = [make((1, 1, 4, 8), torch.float32, 34 + i)[0] for i in range(3)]
    d = [t / (t.norm() + 1e-6) for t in d]
    eps = 1e-3

    def f(a, b, c):
        return sdpa_custom(a, b, c, backend="triton_ref")

    fd = (f(q + eps * d[0], k + eps * d[1], v + eps * d[2]) - f(q - eps * d[0], k - eps * d[1], v - eps * d[2])) / (2 * eps)
    jv = sdpa_custom_jvp(q, k, v, *d).float()
    cos = torch.nn.functional.cosine_similarity(jv.flatten(), fd.flatten(), dim=0)
    assert cos > 0.99
    torch.testing.assert_close(jv, fd, rtol=5e-2, atol=5e-2)
