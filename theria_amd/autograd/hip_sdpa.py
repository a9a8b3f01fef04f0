"""autograd wiring of the HIP SDPA operator: exact derivatives of every order, forward-mode JVP.

SDPAOp            O = softmax(scale Q K^T) V (optional causal mask); forward kernel, saves (O, lse).
  .backward       -> SDPABackwardOp.apply(...), itself an autograd.Function, so gradients computed
                     with create_graph=True stay differentiable (MAML's full second order).
  .jvp            -> the frozen-stats JVP kernel (torch.func.jvp / forward-mode AD).
SDPABackwardOp    (dQ, dK, dV) from the backward kernel; its backward is the explicit double-backward
                  kernel set (G_Q, G_K, G_V, G_dO).

The reference's Triton path returns backward outputs with no graph (theria/attention/triton_qk.py:
379-387), which silently drops attention's second-order terms under MAML create_graph=True. Here the
second-order terms are explicit kernels. When the double backward itself must stay differentiable
(create_graph=True while differentiating a create_graph'ed gradient: third order, as in the
meta-gradient probe of experiments/phase10/scripts/run_maml_backend_compare.py:169-199), the double
backward is instead taken by autograd through a float32 PyTorch restatement of the backward map on
the same device (materialised T x M scores), which is exact to any order. Everything up to second
order, including every MAML outer backward, runs on the kernels.
"""

from __future__ import annotations

import torch

from .. import _ops


def _backward_map(q, k, v, dout, scale: float, causal: bool):
    """(dQ, dK, dV) of O = softmax(scale Q K^T) V given dO, as differentiable PyTorch ops (float32 or wider).

    dV = P^T dO, dP = dO V^T, dS = P * (dP - rowsum(dP * P)), dQ = scale dS K, dK = scale dS^T Q
    (reference theria/attention/reference_backward_sdpa.py:31-51). Only used for derivatives of order
    three and higher, which no kernel covers.
    """
    ct = torch.promote_types(q.dtype, torch.float32)
    qf, kf, vf, df = (t.to(ct) for t in (q, k, v, dout))
    s = torch.matmul(qf, kf.transpose(-2, -1)) * scale
    if causal:
        keep = torch.ones(s.shape[-2], s.shape[-1], dtype=torch.bool, device=s.device).tril()
        s = s.masked_fill(~keep, float("-inf"))
    p = torch.softmax(s, dim=-1)
    dp = torch.matmul(df, vf.transpose(-2, -1))
    ds = p * (dp - (dp * p).sum(dim=-1, keepdim=True))
    dq = torch.matmul(ds, kf) * scale
    dk = torch.matmul(ds.transpose(-2, -1), qf) * scale
    dv = torch.matmul(p.transpose(-2, -1), df)
    return dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype)


def _differentiable_double_backward(q, k, v, dout, gq, gk, gv, scale: float, causal: bool):
    """(G_Q, G_K, G_V, G_dO) with a graph: the VJP of _backward_map taken with create_graph=True.

    The map is differentiated through aliases (view_as) of its inputs, so each result is the partial
    derivative with respect to that argument: dO usually depends on q, k, v itself (dO = dL/dO of a
    loss of O), and that path is already carried by G_dO. The aliases keep the results connected to
    the original tensors for the next order.
    """
    prim = tuple(t.view_as(t) if t.requires_grad else t for t in (q, k, v, dout))
    wrt = [t for t in prim if t.requires_grad]
    if not wrt:
        return None, None, None, None
    q, k, v, dout = prim
    outs = _backward_map(q, k, v, dout, scale, causal)
    pairs = [(o, g) for o, g in zip(outs, (gq, gk, gv)) if g is not None]
    grads = iter(torch.autograd.grad([o for o, _ in pairs], wrt, [g for _, g in pairs], create_graph=True,
                                     allow_unused=True))
    return tuple(next(grads) if t.requires_grad else None for t in prim)


class SDPABackwardOp(torch.autograd.Function):
    """(q, k, v, o, lse, dout, scale, causal) -> (dq, dk, dv). o and lse (whose flag bits mark the peaked rows
    of the 16-bit backward) are treated as constants of q, k, v."""

    @staticmethod
    def forward(ctx, q, k, v, o, lse, dout, scale, causal):
        dq, dk, dv, _ = _ops.bwd(q, k, v, o, lse, dout, scale, causal, checked=False)
        ctx.set_materialize_grads(False)  # an absent cotangent stays None (the kernels skip it), not a zero fill
        ctx.save_for_backward(q, k, v, o, lse, dout)
        ctx.scale = scale
        ctx.causal = causal
        return dq, dk, dv

    @staticmethod
    def backward(ctx, gq, gk, gv):
        q, k, v, o, lse, dout = ctx.saved_tensors
        if gq is None and gk is None and gv is None:
            return None, None, None, None, None, None, None, None
        if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (q, k, v, dout, gq, gk, gv)):
            g_q, g_k, g_v, g_do = _differentiable_double_backward(q, k, v, dout, gq, gk, gv, ctx.scale, ctx.causal)
            return g_q, g_k, g_v, None, None, g_do, None, None
        g_q, g_k, g_v, g_do = _ops.bwd_bwd(q, k, v, o, dout, lse, None, gq, gk, gv, ctx.scale, ctx.causal,
                                           checked=False)
        return g_q, g_k, g_v, None, None, g_do.to(dout.dtype), None, None


def _save_forward(ctx, q, k, v, scale, causal, o, lse) -> None:
    ctx.scale = scale
    ctx.causal = causal
    ctx.mark_non_differentiable(lse)
    ctx.set_materialize_grads(False)  # lse's gradient stays None rather than a zero fill on every backward
    ctx.save_for_backward(q, k, v, o, lse)
    ctx.save_for_forward(q, k, v, o, lse)


def _sdpa_backward(ctx, do, _dlse):
    if do is None:
        return None, None, None, None, None, None
    q, k, v, o, lse = ctx.saved_tensors
    dq, dk, dv = SDPABackwardOp.apply(q, k, v, o.detach(), lse, do, ctx.scale, ctx.causal)
    return dq, dk, dv, None, None, None


def _sdpa_jvp(ctx, tq, tk, tv, _ts, _tc, _tf):
    q, k, v, o, lse = ctx.saved_tensors
    to = _ops.jvp(q, k, v, o, lse, tq, tk, tv, ctx.scale, ctx.causal, normalize=True, checked=False)
    if to.dtype != o.dtype:
        to = to.to(o.dtype)
    return to, None


class SDPAOp(torch.autograd.Function):
    """(q, k, v, scale, causal, out_fp32) -> (o, lse). The setup_context form, which torch.func transforms
    (vmap, jvp, grad) require; hip_sdpa takes _SDPAOpEager outside them."""

    @staticmethod
    def forward(q, k, v, scale, causal, out_fp32):
        return _ops.fwd(q, k, v, scale, causal, out_fp32=out_fp32)[:2]

    @staticmethod
    def setup_context(ctx, inputs, output):
        q, k, v, scale, causal, _ = inputs
        _save_forward(ctx, q, k, v, scale, causal, *output)

    backward = staticmethod(_sdpa_backward)
    jvp = staticmethod(_sdpa_jvp)


class _SDPAOpEager(torch.autograd.Function):
    """SDPAOp in the ctx-first form, for calls outside torch.func transforms (which refuse this form).
    torch.autograd.Function.apply binds the arguments of a setup_context-form forward through
    inspect.signature on every call, ~30 us of host time, as much as the forward kernel's own launch path;
    this form skips it. Same kernels, saved tensors, backward and JVP as SDPAOp."""

    @staticmethod
    def forward(ctx, q, k, v, scale, causal, out_fp32):
        o, lse = _ops.fwd(q, k, v, scale, causal, out_fp32=out_fp32)[:2]
        _save_forward(ctx, q, k, v, scale, causal, o, lse)
        return o, lse

    backward = staticmethod(_sdpa_backward)
    jvp = staticmethod(_sdpa_jvp)


# torch's own test for an active torch.func transform (what Function.apply checks); without it, always SDPAOp
_transforms_active = getattr(torch._C, "_are_functorch_transforms_active", lambda: True)


def _sdpa_op(q, k, v, scale: float, causal: bool, out_fp32: bool):
    op = SDPAOp if _transforms_active() else _SDPAOpEager
    return op.apply(q, k, v, scale, causal, out_fp32)


def _common_head_dim(q, k, v):
    """q, k, v zero-padded along the head dim to max(D, Dv) when Dv != D, and Dv.

    Zero columns add nothing to Q K^T and the padded columns of O = P V are sliced off, so the result
    and every derivative (padding and slicing are linear) equal the unpadded operator's; the kernels
    themselves take one head dim for Q, K and V.
    """
    D, Dv = q.shape[-1], v.shape[-1]
    if D == Dv:
        return q, k, v, Dv
    Dp = max(D, Dv)
    if D < Dp:
        q = torch.nn.functional.pad(q, (0, Dp - D))
        k = torch.nn.functional.pad(k, (0, Dp - D))
    else:
        v = torch.nn.functional.pad(v, (0, Dp - Dv))
    return q, k, v, Dv


def hip_sdpa(q, k, v, *, causal: bool = False, scale: float | None = None, out_fp32: bool = False):
    """Differentiable SDPA through the HIP kernels (any order; see the module docstring). Returns O only.

    v may have its own head dim Dv (B, H, M, Dv); scale defaults to 1/sqrt(D) of q and k.
    """
    if scale is None:
        scale = _ops.default_scale(q.shape[-1])
    q, k, v, dv = _common_head_dim(q, k, v)
    o = _sdpa_op(q, k, v, float(scale), bool(causal), bool(out_fp32))[0]
    return o if o.shape[-1] == dv else o[..., :dv]


def hip_sdpa_with_lse(q, k, v, *, causal: bool = False, scale: float | None = None):
    """(O, lse) with lse = log-sum-exp of the scaled scores per query row (not differentiable)."""
    if scale is None:
        scale = _ops.default_scale(q.shape[-1])
    q, k, v, dv = _common_head_dim(q, k, v)
    o, lse = _sdpa_op(q, k, v, float(scale), bool(causal), False)[:2]
    return (o if o.shape[-1] == dv else o[..., :dv]), lse


def hip_sdpa_hvp(q, k, v, vq, vk, vv, *, weight=None, target=None, causal: bool = False, scale: float | None = None):
    """Hessian-vector product of a scalar loss of O = SDPA(q, k, v) along (vq, vk, vv), from the kernels
    directly (no autograd graph): the counterpart of the reference's sdpa_hvp
    (theria/attention/reference_hvp_sdpa.py:46-97), which differentiates sum(O).

    Loss: sum(O) by default; <weight, O> for a constant weight; 0.5 ||O - target||^2 for a target. With
    dO = dL/dO the HVP is the double backward of the backward map with cotangents (vq, vk, vv), plus, for
    the quadratic loss, the Gauss-Newton term J^T (J v) = backward(G_dO), since G_dO = J v.
    Returns (hq, hk, hv) in the input dtype.
    """
    if scale is None:
        scale = _ops.default_scale(q.shape[-1])
    if weight is not None and target is not None:
        raise ValueError("hip_sdpa_hvp: give weight or target, not both")
    with torch.no_grad():
        o, lse, _, _ = _ops.fwd(q, k, v, float(scale), bool(causal))
        if target is not None:
            # the float32 difference rounded once to o's dtype (one kernel when the dtypes agree)
            dout = o - target if target.dtype == o.dtype else (o.float() - target.float()).to(o.dtype)
        elif weight is not None:
            dout = weight.to(o.dtype)
        else:
            dout = torch.ones_like(o)
        if target is None:
            return _ops.bwd_bwd(q, k, v, o, dout, lse, None, vq, vk, vv, float(scale), bool(causal), checked=False)[:3]
        # both results as views of one flat buffer each, so that their sum is one full-grid launch
        B, H, T, D = q.shape
        M = k.shape[2]
        sizes = (B * H * T * D, B * H * M * D, B * H * M * D)
        shapes = ((B, H, T, D), (B, H, M, D), (B, H, M, D))
        flat_h, flat_j = (torch.empty(sum(sizes), dtype=q.dtype, device=q.device) for _ in range(2))
        hs, js = ([f.view(sh) for f, sh in zip(buf.split(sizes), shapes)] for buf in (flat_h, flat_j))
        g_do = _ops.bwd_bwd(q, k, v, o, dout, lse, None, vq, vk, vv, float(scale), bool(causal), out=hs,
                            checked=False)[3]
        _ops.bwd(q, k, v, o, lse, g_do.to(o.dtype), float(scale), bool(causal), out=js, checked=False)
        flat_h.add_(flat_j)
        return tuple(hs)


__all__ = ["SDPAOp", "SDPABackwardOp", "hip_sdpa", "hip_sdpa_with_lse", "hip_sdpa_hvp"]
