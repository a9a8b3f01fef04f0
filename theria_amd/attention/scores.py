"""Materialised-score pieces of the partial-fusion sdpa_custom backends, on the HIP score kernels.

Names and return conventions follow the reference (theria/attention/triton_qk.py):
  triton_qk(q, k)            Q K^T as float32 (B,H,T,M) scores, differentiable (TritonQKFunction,
                             triton_qk.py:67-125): the backward is two matmuls, so it differentiates again
  triton_qk_fast(q, k)       the same, scores in the input dtype (TritonQKFunctionFast, triton_qk.py:456-522)
  triton_qk_softmax(q, k)    softmax(Q K^T / sqrt(D)) as float32 probabilities (triton_qk.py:197-240); as in
                             the reference it is a plain function: the result carries no gradient to q or k
The kernels are gfx950 HIP (csrc/sdpa_scores.hip); the names are kept so callers switch by import.
Differences, each deliberate: the backward accumulates in float32 and returns gradients in the input
dtype (the reference's matmul of float32 gradients with 16-bit k raises on dtype mismatch), and the
fast variant accumulates in float32 before rounding the scores (MFMA has no 16-bit accumulation).
"""

from __future__ import annotations

import torch

from .. import _ops


def _guard(q, k, what: str) -> None:
    if not (q.is_cuda and k.is_cuda):
        raise AssertionError(f"{what} requires CUDA (HIP) tensors")
    if q.shape[-1] != k.shape[-1]:
        raise AssertionError("Q and K last dimensions must match")


class TritonQKFunction(torch.autograd.Function):
    """scores = Q K^T (float32) through the HIP score kernel."""

    @staticmethod
    def forward(ctx, q, k):
        _guard(q, k, "TritonQKFunction")
        ctx.save_for_backward(q, k)
        return _ops.qk_scores(q, k, out_f32=True)

    @staticmethod
    def backward(ctx, grad_out):
        q, k = ctx.saved_tensors
        g = grad_out.float()
        grad_q = torch.matmul(g, k.float()).to(q.dtype)
        grad_k = torch.matmul(g.transpose(-2, -1), q.float()).to(k.dtype)
        return grad_q, grad_k


class TritonQKFunctionFast(torch.autograd.Function):
    """scores = Q K^T in the input dtype (float32 accumulation, rounded once)."""

    @staticmethod
    def forward(ctx, q, k):
        _guard(q, k, "TritonQKFunctionFast")
        ctx.save_for_backward(q, k)
        return _ops.qk_scores(q, k, out_f32=False)

    @staticmethod
    def backward(ctx, grad_out):
        q, k = ctx.saved_tensors
        g = grad_out.float()
        grad_q = torch.matmul(g, k.float()).to(q.dtype)
        grad_k = torch.matmul(g.transpose(-2, -1), q.float()).to(k.dtype)
        return grad_q, grad_k


def triton_qk(q, k):
    """Q K^T scores (B,H,T,M) in float32 with autograd."""
    return TritonQKFunction.apply(q, k)


def triton_qk_fast(q, k):
    """Q K^T scores (B,H,T,M) in the input dtype with autograd."""
    return TritonQKFunctionFast.apply(q, k)


def triton_qk_softmax(q, k):
    """softmax(Q K^T / sqrt(D)) over the keys, float32 (B,H,T,M); not differentiable in q, k."""
    _guard(q, k, "triton_qk_softmax")
    if not (q.is_contiguous() and k.is_contiguous()):
        raise AssertionError("triton_qk_softmax requires contiguous inputs (v0)")
    if q.shape[-1] > 128:
        raise AssertionError("triton_qk_softmax supports D <= 128")
    with torch.no_grad():
        return _ops.qk_softmax(q, k, 1.0 / (q.shape[-1] ** 0.5))


__all__ = ["TritonQKFunction", "TritonQKFunctionFast", "triton_qk", "triton_qk_fast", "triton_qk_softmax"]
