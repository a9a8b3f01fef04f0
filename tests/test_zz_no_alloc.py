"""theria_sdpa_bwd_bwd_noalloc (static device scratch instead of a workspace argument) against
theria_sdpa_bwd_bwd through the C ABI: bit-identical outputs on two calls in a row, the second on a smaller
problem (the scratch keeps the first call's contents), and the size limit rejected on the host."""

import math

import pytest
import torch

from theria_amd import _ops

pytestmark = pytest.mark.gpu


def _problem(dev, dt, B, H, T, M, D, seed):
    g = torch.Generator().manual_seed(seed)
    shapes = [(B, H, T, D), (B, H, M, D), (B, H, M, D), (B, H, T, D), (B, H, T, D), (B, H, M, D), (B, H, M, D)]
    return [torch.randn(*sh, generator=g).to(dt).to(dev) for sh in shapes]


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_noalloc_double_backward_equals_the_workspace_entry_point(dt, hip_device):
    for B, H, T, M, D, causal in [(2, 4, 512, 384, 64, False), (1, 2, 130, 200, 64, True)]:
        print(f"[noalloc] {dt} B{B} H{H} T{T} M{M} D{D} causal={causal}", flush=True)
        q, k, v, do, gq, gk, gv = _problem(hip_device, dt, B, H, T, M, D, seed=T)
        s = 1 / math.sqrt(D)
        o, lse, _, _ = _ops.fwd(q, k, v, s, causal)
        _, _, _, delta = _ops.bwd(q, k, v, o, lse, do, s, causal)
        ref = _ops.bwd_bwd(q, k, v, o, do, lse, delta, gq, gk, gv, s, causal)
        got = _ops.bwd_bwd(q, k, v, o, do, lse, delta, gq, gk, gv, s, causal, noalloc=True)
        torch.cuda.synchronize()
        for name, a, b in zip(("G_Q", "G_K", "G_V", "G_dO"), got, ref):
            assert torch.equal(a, b), f"{name} differs from theria_sdpa_bwd_bwd ({dt}, T={T})"


def test_noalloc_rejects_problems_beyond_the_static_scratch(hip_device):
    """5 * B * H * T > 5 * 2^20 is refused before any launch (a contract error, not a fault)."""
    B, H, T, M, D = 1, 1, (1 << 20) + 1, 8, 8
    q = torch.zeros(B, H, T, D, dtype=torch.bfloat16, device=hip_device)
    k = torch.zeros(B, H, M, D, dtype=torch.bfloat16, device=hip_device)
    lse = torch.zeros(B, H, T, device=hip_device)
    with pytest.raises(AssertionError, match="static scratch"):
        _ops.bwd_bwd(q, k, k, q, q, lse, lse, None, k, None, 0.25, False, noalloc=True)


def test_noalloc_double_backward_replays_in_a_graph(hip_device):
    """Captured in a HIP graph (after one eager call, which looks up the device's scratch address), the
    allocation-free double backward replays bit for bit equal to the eager result, also when an eager call on
    other inputs has rewritten the shared scratch in between (the kernels rewrite every element they read)."""
    dt, B, H, T, M, D = torch.bfloat16, 2, 2, 256, 192, 64
    print("[noalloc graph] capture + replays", flush=True)
    args = _problem(hip_device, dt, B, H, T, M, D, seed=7)
    other = _problem(hip_device, dt, B, H, T, M, D, seed=8)
    s = 1 / math.sqrt(D)

    def call(q, k, v, do, gq, gk, gv):
        o, lse, _, _ = _ops.fwd(q, k, v, s, False)
        return _ops.bwd_bwd(q, k, v, o, do, lse, None, gq, gk, gv, s, False, noalloc=True)

    ref = [t.clone() for t in call(*args)]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up on a side stream, as torch's graph capture recommends
        call(*args)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = call(*args)
    for i in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for name, a, b in zip(("G_Q", "G_K", "G_V", "G_dO"), out, ref):
            assert torch.equal(a, b), f"replay {i}: {name} differs from the eager result"
        call(*other)  # eager work on the same scratch between replays
        torch.cuda.synchronize()
