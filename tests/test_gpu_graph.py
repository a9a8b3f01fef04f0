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
