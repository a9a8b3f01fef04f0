"""Explicit frozen-stats backward and JVP on the HIP kernels, under the reference's public names.

sdpa_bwd_dq / sdpa_bwd_dk / sdpa_bwd_dv (q, k, [v,] dout, m, l, scale) and
sdpa_jvp (q, k, v, dq, dk, dv, m, l, scale) follow theria/attention/triton_sdpa_backward.py:194, 401,
465, 635: P is rebuilt from the saved (m, l) (lse = m + log l), outputs are fresh tensors in q's dtype,
and contract violations raise AssertionError (the reference's guards, :23-103). The reference keeps
three separate kernels that each recompute the softmax row term; here each call runs the one fused
backward kernel (with the row term computed once) and returns the requested gradient.
Widened contract: D <= 128 and any strides with a contiguous last dimension.
"""

from __future__ import annotations

import torch

from .. import _ops

_ALLOWED_DTYPES = _ops.ALLOWED_DTYPES


def _assert_backward_contract(q, k, v, dout, m, l, require_v: bool = True):
    if not (q.is_cuda and k.is_cuda and dout.is_cuda and (not require_v or (v is not None and v.is_cuda))):
        raise AssertionError("explicit backward requires GPU tensors")
    named = [("q", q), ("k", k), ("dout", dout)] + ([("v", v)] if require_v else [])
    for name, t in named:
        if t.dtype not in _ALLOWED_DTYPES:
            raise AssertionError(f"Unsupported dtype for {name}: {t.dtype}")
    B, H, T, D = q.shape
    if k.ndim != 4 or k.shape[0] != B or k.shape[1] != H or k.shape[3] != D:
        raise AssertionError("k must have shape (B,H,M,D) with D matching q")
    if tuple(dout.shape) != (B, H, T, D):
        raise AssertionError("dout shape must be (B,H,T,D)")
    if require_v and (v is None or v.ndim != 4 or v.shape[0] != B or v.shape[1] != H or v.shape[3] != D):
        raise AssertionError("v must have shape (B,H,M,D) with D matching q")
    if tuple(m.shape) != (B, H, T) or tuple(l.shape) != (B, H, T):
        raise AssertionError("m,l must be saved forward stats with shape (B,H,T)")
    if D > _ops.MAX_HEAD_DIM:
        raise AssertionError(f"explicit backward supports D<={_ops.MAX_HEAD_DIM}")


def _assert_jvp_contract(q, k, v, dq, dk, dv, m, l):
    for name, t in (("q", q), ("k", k), ("v", v), ("dq", dq), ("dk", dk), ("dv", dv)):
        if not t.is_cuda:
            raise AssertionError("explicit JVP requires GPU tensors")
        if t.dtype not in _ALLOWED_DTYPES:
            raise AssertionError(f"Unsupported dtype for {name}: {t.dtype}")
    B, H, T, D = q.shape
    if k.ndim != 4 or k.shape[0] != B or k.shape[1] != H or k.shape[3] != D:
        raise AssertionError("k must have shape (B,H,M,D) with D matching q")
    if v.ndim != 4 or v.shape[0] != B or v.shape[1] != H or v.shape[3] != D:
        raise AssertionError("v must have shape (B,H,M,D) with D matching q")
    if dq.shape != q.shape or dk.shape != k.shape or dv.shape != v.shape:
        raise AssertionError("dq, dk, dv must match q, k, v shapes respectively")
    if tuple(m.shape) != (B, H, T) or tuple(l.shape) != (B, H, T):
        raise AssertionError("m,l must be saved forward stats with shape (B,H,T)")
    if D > _ops.MAX_HEAD_DIM:
        raise AssertionError(f"explicit JVP supports D<={_ops.MAX_HEAD_DIM}")
    if torch.any(l <= 0):
        raise AssertionError("frozen-stats JVP requires l > 0 (forward sumexp stats)")


def _lse(m, l, q):
    # the peaked-row flag bits are read by the 16-bit kernels only; a float32 lse stays exactly m + log l
    return _ops.lse_from_stats(m, l, peaked_bits=q.dtype != torch.float32)


def sdpa_bwd_dq(q, k, v, dout, m, l, scale):
    """dQ = scale dS K with P rebuilt from (m, l)."""
    _assert_backward_contract(q, k, v, dout, m, l, require_v=True)
    dq, _, _ = _ops.bwd_from_stats(q, k, v, dout, _lse(m, l, q), scale, False, True, False, False)
    return dq


def sdpa_bwd_dk(q, k, v, dout, m, l, scale):
    """dK = scale dS^T Q with P rebuilt from (m, l)."""
    _assert_backward_contract(q, k, v, dout, m, l, require_v=True)
    _, dk, _ = _ops.bwd_from_stats(q, k, v, dout, _lse(m, l, q), scale, False, False, True, False)
    return dk


def sdpa_bwd_dv(q, k, dout, m, l, scale):
    """dV = P^T dO with P rebuilt from (m, l); needs no v (triton_sdpa_backward.py:194)."""
    _assert_backward_contract(q, k, None, dout, m, l, require_v=False)
    _, _, dv = _ops.bwd_from_stats(q, k, None, dout, _lse(m, l, q), scale, False, False, False, True)
    return dv


def sdpa_bwd(q, k, v, dout, m, l, scale):
    """All three gradients in one backward pass: (dq, dk, dv)."""
    _assert_backward_contract(q, k, v, dout, m, l, require_v=True)
    return _ops.bwd_from_stats(q, k, v, dout, _lse(m, l, q), scale, False, True, True, True)


def sdpa_jvp(q, k, v, dq, dk, dv, m, l, scale):
    """Frozen-stats JVP (docs/phase9.md:30-39): dO = P o (dS - rowsum(dS o P)) V + P dv, with
    P = exp(S - m) / l held exactly as given (triton_sdpa_backward.py:488-503)."""
    _assert_jvp_contract(q, k, v, dq, dk, dv, m, l)
    return _ops.jvp(q, k, v, None, _lse(m, l, q), dq, dk, dv, scale, False, normalize=False)


__all__ = ["sdpa_bwd_dq", "sdpa_bwd_dk", "sdpa_bwd_dv", "sdpa_bwd", "sdpa_jvp"]
