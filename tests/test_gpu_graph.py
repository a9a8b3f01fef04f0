"""HIP-graph capture of the operator: replays must reproduce the eager results exactly.

The kernels are deterministic (no atomics) and the library allocates nothing, so a captured forward +
backward replays to bit-identical outputs. Each graph is replayed several times with eager work and
synchronisations between the replays, and every replay is checked.
"""

import math

import pytest
import torch

from theria_amd import _ops

pytestmark = pytest.mark.gpu

CASES = [
    # dtype, B, H, T, M, D, causal   (16-bit D=64 / D=128: pipelined kernels; fp32 and D=40: general kernels)
    (torch.bfloat16, 2, 4, 512, 512, 64, False),
    (torch.float16, 1, 2, 384, 384, 128, True),
    (torch.float32, 1, 2, 96, 80, 40, False),
]


def _make(shape, dtype, dev, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dtype).to(dev)


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}-T{c[3]}-D{c[5]}{'-causal' if c[6] else ''}" for c in CASES])
def test_graph_replay_matches_eager(case, hip_device):
    dt, B, H, T, M, D, causal = case
    dev = hip_device
    print(f"[graph] {case}", flush=True)
    q, do = _make((B, H, T, D), dt, dev, 1), _make((B, H, T, D), dt, dev, 4)
    k, v = _make((B, H, M, D), dt, dev, 2), _make((B, H, M, D), dt, dev, 3)
    s = 1.0 / math.sqrt(D)

    def step():
        o, lse, _, _ = _ops.fwd(q, k, v, s, causal)
        dq, dk, dv, delta = _ops.bwd(q, k, v, o, lse, do, s, causal)
        return o, lse, dq, dk, dv, delta

    ref = [t.clone() for t in step()]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = step()
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for name, a, b in zip(("o", "lse", "dq", "dk", "dv", "delta"), outs, ref):
            assert torch.equal(a, b), f"replay {rep}: {name} differs from the eager result"
        # eager work between replays (allocations and launches outside the graph)
        step()
        torch.cuda.synchronize()


HVP_CASES = [
    # dtype, B, H, T, M, D, causal, loss
    (torch.bfloat16, 2, 2, 256, 256, 64, False, "target"),
    (torch.float16, 1, 2, 200, 200, 128, True, "weight"),
    (torch.float32, 1, 2, 96, 80, 40, False, "sum"),
]


@pytest.mark.parametrize("case", HVP_CASES, ids=[f"{c[0]}-T{c[3]}-D{c[5]}-{c[7]}{'-causal' if c[6] else ''}"
                                                 for c in HVP_CASES])
def test_graphed_hvp_matches_eager_autograd(case, hip_device):
    """GraphedSDPAHVP replays return the eager autograd HVP (gradient with create_graph, then its VJP with v) bit for
    bit, for new inputs on every replay, with eager work between the replays."""
    from theria_amd.autograd import GraphedSDPAHVP, hip_sdpa

    dt, B, H, T, M, D, causal, loss = case
    dev = hip_device
    print(f"[graphed hvp] {case}", flush=True)

    def inputs(seed):
        x = {"q": _make((B, H, T, D), dt, dev, seed), "k": _make((B, H, M, D), dt, dev, seed + 1),
             "v": _make((B, H, M, D), dt, dev, seed + 2), "vq": _make((B, H, T, D), dt, dev, seed + 3),
             "vk": _make((B, H, M, D), dt, dev, seed + 4), "vv": _make((B, H, M, D), dt, dev, seed + 5)}
        if loss != "sum":
            x[loss] = _make((B, H, T, D), dt, dev, seed + 6)
        return x

    def eager(x):
        q, k, v = (x[n].clone().requires_grad_(True) for n in ("q", "k", "v"))
        o = hip_sdpa(q, k, v, causal=causal)
        dout = {"target": lambda: o - x.get("target"), "weight": lambda: x.get("weight"),
                "sum": lambda: torch.ones_like(o)}[loss]()
        g = torch.autograd.grad(o, (q, k, v), grad_outputs=dout, create_graph=True)
        return torch.autograd.grad(g, (q, k, v), grad_outputs=(x["vq"], x["vk"], x["vv"]))

    x0 = inputs(10)
    graphed = GraphedSDPAHVP(causal=causal, **x0)
    for rep in range(3):
        x = inputs(20 + 10 * rep)
        out = graphed(**x)
        torch.cuda.synchronize()
        ref = eager(x)
        torch.cuda.synchronize()
        for name, a, b in zip(("hq", "hk", "hv"), out, ref):
            assert torch.isfinite(b).all(), f"{name}: eager HVP not finite"
            assert torch.equal(a, b), f"replay {rep}: {name} differs from the eager autograd HVP"
    with pytest.raises(ValueError):
        graphed(q=torch.zeros(1, device=dev, dtype=dt))
