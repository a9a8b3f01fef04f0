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
