"""The autograd Hessian-vector product of an SDPA loss, captured once in a HIP graph and replayed.

The HVP is taken as the reference takes it through its differentiable backward (theria/autograd/
sdpa_custom_function.py:32-53; tests/test_reference_attention_hvp.py:53-60): the gradient with
create_graph=True, then its vector-Jacobian product with v.
At small shapes (B8 H8 S512 D64) one such HVP issues ~20 kernel launches whose GPU time (~0.13 ms) is
shorter than the host time PyTorch's autograd engine spends issuing them, so the eager HVP is bound by
the host. A captured graph replays the same launches in the same order without the engine or Python;
the kernels are deterministic, so every replay returns what the eager autograd HVP returns for the same
inputs, bit for bit.

Shapes, dtypes, the loss form, the mask and the scale are fixed at capture. Each call copies the given
inputs into the graph's static buffers and replays; the returned tensors are those static outputs,
overwritten by the next call (clone them to keep them).
"""

from __future__ import annotations

import torch

from .. import _ops
from .hip_sdpa import hip_sdpa


class GraphedSDPAHVP:
    """H (vq, vk, vv) for the loss L(O), O = SDPA(q, k, v), through autograd's double backward, one graph replay
    per call.

    Loss: sum(O) by default; <weight, O> for a weight; 0.5 ||O - target||^2 for a target (as hip_sdpa_hvp,
    dL/dO = O - target formed in O's dtype). The tensors given here are the capture's examples: their
    values are copied in, and every later call may replace any of them (same shape and dtype).
    """

    _NAMES = ("q", "k", "v", "vq", "vk", "vv", "target", "weight")

    def __init__(self, q, k, v, vq, vk, vv, *, target=None, weight=None, causal: bool = False,
                 scale: float | None = None, warmup: int = 2):
        if weight is not None and target is not None:
            raise ValueError("GraphedSDPAHVP: give weight or target, not both")
        if not q.is_cuda:
            raise ValueError("GraphedSDPAHVP captures a HIP graph: the inputs must be on a GPU")
        self.causal = bool(causal)
        self.scale = float(_ops.default_scale(q.shape[-1]) if scale is None else scale)
        # static buffers: q, k, v are leaves that require grad; the rest are plain tensors
        self.q, self.k, self.v = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
        self.vq, self.vk, self.vv = (t.detach().clone() for t in (vq, vk, vv))
        self.target = None if target is None else target.detach().clone()
        self.weight = None if weight is None else weight.detach().clone()
        side = torch.cuda.Stream(device=q.device)
        side.wait_stream(torch.cuda.current_stream(q.device))
        with torch.cuda.stream(side):  # warm-up outside the graph (allocator pools, lazy library state)
            for _ in range(max(1, warmup)):
                self._body()
        torch.cuda.current_stream(q.device).wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.out = self._body()

    def _body(self):
        q, k, v = self.q, self.k, self.v
        o = hip_sdpa(q, k, v, causal=self.causal, scale=self.scale)
        if self.target is not None:
            t = self.target
            dout = o - t if t.dtype == o.dtype else (o.float() - t.float()).to(o.dtype)
        elif self.weight is not None:
            dout = self.weight if self.weight.dtype == o.dtype else self.weight.to(o.dtype)
        else:
            dout = torch.ones_like(o)
        g = torch.autograd.grad(o, (q, k, v), grad_outputs=dout, create_graph=True)
        return torch.autograd.grad(g, (q, k, v), grad_outputs=(self.vq, self.vk, self.vv))

    def __call__(self, **inputs):
        """Replay with the given inputs (keywords q, k, v, vq, vk, vv, target, weight); returns (hq, hk, hv)."""
        with torch.no_grad():
            for name, src in inputs.items():
                if name not in self._NAMES:
                    raise TypeError(f"GraphedSDPAHVP: unknown input {name!r}")
                dst = getattr(self, name)
                if dst is None:
                    raise ValueError(f"GraphedSDPAHVP: {name} was not part of the captured loss")
                if src.shape != dst.shape or src.dtype != dst.dtype or src.device != dst.device:
                    raise ValueError(f"GraphedSDPAHVP: {name} is {tuple(src.shape)} {src.dtype} on {src.device}, "
                                     f"the capture used {tuple(dst.shape)} {dst.dtype} on {dst.device}")
                dst.copy_(src)
        self.graph.replay()
        return self.out


__all__ = ["GraphedSDPAHVP"]
