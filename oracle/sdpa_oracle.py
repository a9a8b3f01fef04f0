"""CPU oracle for theria's SDPA operator family. TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module, and only
as the checker (or the timed CPU baseline), never as part of the product path.

A plain restatement, on CPU, of the reference's pure-PyTorch path, by closed form:
  * forward            reference_attention (theria/attention/reference_attention.py:9-19) plus the
                       saved statistics m, l of the fused kernel (theria/attention/triton_qk.py:280-304,
                       docs/phase9.md:12-16) and lse = m + log l;
  * backward           sdpa_backward_reference (theria/attention/reference_backward_sdpa.py:24-53);
                       frozen_backward takes P from a given lse like the explicit sdpa_bwd_* kernels
                       (theria/attention/triton_sdpa_backward.py:106-696);
  * jvp                sdpa_jvp_reference (theria/attention/reference_jvp_sdpa.py:21-44), which equals
                       the frozen-stats sdpa_jvp (theria/attention/triton_sdpa_backward.py:465-503) at
                       exact stats; frozen_jvp takes the stats as given like the latter;
  * double_backward    VJP of the backward map (Q,K,V,dO) -> (dQ,dK,dV), closed form. The reference
                       has no closed form (it relies on autograd through SDPACustom,
                       theria/autograd/sdpa_custom_function.py:32-53); this one is pinned against
                       torch.autograd double-backward in tests/test_oracle.py;
  * hvp_sum            analytic HVP of sum(O) (theria/attention/reference_hvp_sdpa.py:46-97);
  * hvp                HVP of a scalar loss L(O) composed from the pieces above.
Everything runs in float64 unless the caller passes another dtype. The causal mask (not in the
reference) is lower-triangular, top-left aligned: key j is visible to query i iff j <= i.

How each function is pinned (tests/test_oracle.py): against torch.autograd / torch.func in float64
(grad, double backward, forward-mode jvp, gradcheck), central finite differences, closed-form special
cases (M = 1 gives O = V and dQ = dK = 0; a constant K gives uniform P), torch.logsumexp for lse,
and invariants (rows of P sum to 1; delta = rowsum(dP * P) = rowsum(dO * O); G_dO equals the JVP with
the cotangents as tangents; HVP symmetry). Every function here has at least one such check.
"""

from __future__ import annotations

import math

import torch


def _f64(*ts, dtype=torch.float64):
    return tuple(None if t is None else t.detach().to("cpu", dtype) for t in ts)


def _scale(q, scale):
    return 1.0 / math.sqrt(q.shape[-1]) if scale is None else float(scale)


def _mask(T: int, M: int, causal: bool):
    if not causal:
        return None
    return torch.ones(T, M, dtype=torch.bool).tril()


def probs(q, k, scale=None, causal=False):
    """P = softmax(scale Q K^T) with the optional causal mask; rows without a visible key are 0."""
    s = _scale(q, scale)
    S = (q @ k.transpose(-2, -1)) * s
    msk = _mask(q.shape[-2], k.shape[-2], causal)
    if msk is not None:
        S = S.masked_fill(~msk, float("-inf"))
    P = torch.softmax(S, dim=-1)
    return torch.nan_to_num(P, nan=0.0)


def forward(q, k, v, scale=None, causal=False, dtype=torch.float64):
    """(O, lse, m, l) in float64 (or `dtype`). m = row max of scaled scores, l = sum exp(S - m), lse = m + log l."""
    q, k, v = _f64(q, k, v, dtype=dtype)
    s = _scale(q, scale)
    S = (q @ k.transpose(-2, -1)) * s
    msk = _mask(q.shape[-2], k.shape[-2], causal)
    if msk is not None:
        S = S.masked_fill(~msk, float("-inf"))
    m = S.max(dim=-1).values if S.shape[-1] > 0 else torch.full(S.shape[:-1], float("-inf"), dtype=S.dtype)
    l = torch.exp(S - m.unsqueeze(-1)).nan_to_num(nan=0.0).sum(-1)
    lse = m + torch.log(l)
    P = torch.exp(S - lse.unsqueeze(-1)).nan_to_num(nan=0.0)
    O = P @ v
    return O, lse, m, l


def backward(q, k, v, dout, scale=None, causal=False, dtype=torch.float64):
    """(dQ, dK, dV): dV = P^T dO, dP = dO V^T, z = rowsum(dP P), dS = P (dP - z), dQ = s dS K, dK = s dS^T Q."""
    q, k, v, dout = _f64(q, k, v, dout, dtype=dtype)
    s = _scale(q, scale)
    P = probs(q, k, s, causal)
    dv = P.transpose(-2, -1) @ dout
    dP = dout @ v.transpose(-2, -1)
    z = (dP * P).sum(-1, keepdim=True)
    dS = P * (dP - z)
    return s * (dS @ k), s * (dS.transpose(-2, -1) @ q), dv


def frozen_backward(q, k, v, dout, lse, scale=None, causal=False, dtype=torch.float64):
    """(dQ, dK, dV) of the frozen-stats backward: the gradient formula of backward() evaluated with
    P = exp(S - lse) held as given (the reference's sdpa_bwd_dq / _dk / _dv with saved (m, l), lse = m + log l,
    theria/attention/triton_sdpa_backward.py:106-266, 269-462, 505-696): z = rowsum(dP P), dS = P (dP - z)."""
    q, k, v, dout, lse = _f64(q, k, v, dout, lse, dtype=dtype)
    s = _scale(q, scale)
    S = (q @ k.transpose(-2, -1)) * s
    msk = _mask(q.shape[-2], k.shape[-2], causal)
    if msk is not None:
        S = S.masked_fill(~msk, float("-inf"))
    P = torch.exp(S - lse.unsqueeze(-1)).nan_to_num(nan=0.0)
    dv = P.transpose(-2, -1) @ dout
    dP = dout @ v.transpose(-2, -1)
    z = (dP * P).sum(-1, keepdim=True)
    dS = P * (dP - z)
    return s * (dS @ k), s * (dS.transpose(-2, -1) @ q), dv


def jvp(q, k, v, tq, tk, tv, scale=None, causal=False):
    """Tangent of O: dS = s (tQ K^T + Q tK^T); dP = P (dS - rowsum(dS P)); tO = dP V + P tV."""
    q, k, v, tq, tk, tv = _f64(q, k, v, tq, tk, tv)
    s = _scale(q, scale)
    P = probs(q, k, s, causal)
    G = torch.zeros_like(P)
    if tq is not None:
        G = G + tq @ k.transpose(-2, -1)
    if tk is not None:
        G = G + q @ tk.transpose(-2, -1)
    G = G * s
    dP = P * (G - (G * P).sum(-1, keepdim=True))
    out = dP @ v
    if tv is not None:
        out = out + P @ tv
    return out


def frozen_jvp(q, k, v, tq, tk, tv, m, l, scale):
    """Frozen-stats JVP with P = exp(S - m) / l rebuilt from the given (m, l)."""
    q, k, v, tq, tk, tv, m, l = _f64(q, k, v, tq, tk, tv, m, l)
    S = (q @ k.transpose(-2, -1)) * scale
    P = torch.exp(S - m.unsqueeze(-1)) / l.unsqueeze(-1)
    G = (tq @ k.transpose(-2, -1) + q @ tk.transpose(-2, -1)) * scale
    Gc = G - (G * P).sum(-1, keepdim=True)
    return (P * Gc) @ v + P @ tv


def double_backward(q, k, v, dout, gq, gk, gv, scale=None, causal=False):
    """VJP of (Q,K,V,dO) -> (dQ,dK,dV) with cotangents (gq, gk, gv): returns (G_Q, G_K, G_V, G_dO).

    Gam = s (gQ K^T + Q gK^T), r = rowsum(P Gam), z = rowsum(P dP), W = dO gV^T,
    Gbar_dP = P (Gam - r), Gbar_P = Gam (dP - z) - r dP + W, srow = rowsum(P Gbar_P),
    Gbar_S = P (Gbar_P - srow), dS = P (dP - z);
    G_dO = Gbar_dP V + P gV, G_V = Gbar_dP^T dO, G_Q = s (Gbar_S K + dS gK), G_K = s (Gbar_S^T Q + dS^T gQ).
    """
    q, k, v, dout, gq, gk, gv = _f64(q, k, v, dout, gq, gk, gv)
    s = _scale(q, scale)
    z0 = lambda x, like: torch.zeros_like(like) if x is None else x  # noqa: E731
    gq, gk, gv = z0(gq, q), z0(gk, k), z0(gv, v)
    P = probs(q, k, s, causal)
    dP = dout @ v.transpose(-2, -1)
    z = (P * dP).sum(-1, keepdim=True)
    dS = P * (dP - z)
    Gam = s * (gq @ k.transpose(-2, -1) + q @ gk.transpose(-2, -1))
    r = (P * Gam).sum(-1, keepdim=True)
    W = dout @ gv.transpose(-2, -1)
    Gbar_dP = P * (Gam - r)
    Gbar_P = Gam * (dP - z) - r * dP + W
    srow = (P * Gbar_P).sum(-1, keepdim=True)
    Gbar_S = P * (Gbar_P - srow)
    G_dO = Gbar_dP @ v + P @ gv
    G_V = Gbar_dP.transpose(-2, -1) @ dout
    G_Q = s * (Gbar_S @ k + dS @ gk)
    G_K = s * (Gbar_S.transpose(-2, -1) @ q + dS.transpose(-2, -1) @ gq)
    return G_Q, G_K, G_V, G_dO


def hvp_sum(q, k, v, vq, vk, vv):
    """HVP of L = sum(reference_attention(q, k, v)) along (vq, vk, vv) (scale 1/sqrt(D), no mask).

    dL/dO is the constant all-ones tensor, so the HVP is exactly the double backward's (G_Q, G_K, G_V)
    with dO = 1 and cotangents (vq, vk, vv).
    """
    q, k, v, vq, vk, vv = _f64(q, k, v, vq, vk, vv)
    ones = torch.ones(q.shape[:-1] + (v.shape[-1],), dtype=torch.float64)
    G_Q, G_K, G_V, _ = double_backward(q, k, v, ones, vq, vk, vv)
    return G_Q, G_K, G_V


def hvp_quadratic(q, k, v, target, vq, vk, vv, scale=None, causal=False):
    """HVP of L = 0.5 ||O - target||^2 along (vq, vk, vv).

    grad L = backward(dO = O - T). Differentiating <grad L, v> gives the double backward with dO held
    fixed, plus the path through dO = O - T: backward(dO = J v) where J v = jvp(vq, vk, vv) (the
    Gauss-Newton term J^T J v).
    """
    q, k, v, target, vq, vk, vv = _f64(q, k, v, target, vq, vk, vv)
    O, _, _, _ = forward(q, k, v, scale, causal)
    dO = O - target
    G_Q, G_K, G_V, G_dO = double_backward(q, k, v, dO, vq, vk, vv, scale, causal)
    gn_q, gn_k, gn_v = backward(q, k, v, G_dO, scale, causal)
    return G_Q + gn_q, G_K + gn_k, G_V + gn_v


def hvp_weighted_sum(q, k, v, w, vq, vk, vv, scale=None, causal=False):
    """HVP of L = sum(O * W) along (vq, vk, vv): dO = W is constant, so only the double backward remains."""
    q, k, v, w, vq, vk, vv = _f64(q, k, v, w, vq, vk, vv)
    G_Q, G_K, G_V, _ = double_backward(q, k, v, w, vq, vk, vv, scale, causal)
    return G_Q, G_K, G_V


def autograd_attention(q, k, v, scale=None, causal=False):
    """Textbook SDPA as a differentiable torch expression (the object the oracle is pinned against)."""
    s = _scale(q, scale)
    S = (q @ k.transpose(-2, -1)) * s
    msk = _mask(q.shape[-2], k.shape[-2], causal)
    if msk is not None:
        S = S.masked_fill(~msk, float("-inf"))
    return torch.softmax(S, dim=-1) @ v


__all__ = [
    "probs",
    "forward",
    "backward",
    "jvp",
    "frozen_jvp",
    "double_backward",
    "hvp_sum",
    "hvp_quadratic",
    "hvp_weighted_sum",
    "autograd_attention",
]
