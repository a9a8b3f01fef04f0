"""Seeded inputs for the precision tests: rows whose softmax is peaked, and rows whose maximum score sits in
a late key tile far above the scores of the earlier tiles.

Shared by the CPU emulation test of the forward's online-softmax rescaling (test_online_softmax_emulation.py)
and the GPU parity tests (test_gpu_precision.py), so both look at exactly the same values. Every tensor is
generated on the CPU in float32 and rounded to the compute dtype; callers give the oracle the rounded values.
"""

from __future__ import annotations

import torch


def randn(shape, seed: int, std: float = 1.0, dtype=torch.float32) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * std).to(dtype)


def planted_late_key(B, H, T, M, D, dtype, seed: int, key: int, gap: float, scale: float):
    """(q, k, v) where, on every query row with a positive planted sign, key `key` scores about `gap` nats
    above every other key; rows with a negative sign score it about `gap` nats below the rest.

    Component 0 of every query is +-a and component 0 of every other key is small, so the planted key
    (component 0 = b) adds +-scale a b to the row's score: a, b are chosen so that scale a b = gap, with a
    and b exactly representable in 16 bits. Query signs alternate in blocks of 7 rows, so that a wave of
    32 queries mixes rows whose maximum moves with rows whose maximum does not.
    """
    q = randn((B, H, T, D), seed)
    k = randn((B, H, M, D), seed + 1)
    v = randn((B, H, M, D), seed + 2)
    a = 8.0
    b = float(torch.tensor(gap / (scale * a)).to(dtype).float())
    sign = torch.tensor([1.0 if (i // 7) % 2 == 0 else -1.0 for i in range(T)])
    q[..., 0] = a * sign
    k[..., 0] = 0.25 * k[..., 0]
    k[..., key, 0] = b
    return q.to(dtype), k.to(dtype), v.to(dtype)


def peaked(B, H, T, M, D, dtype, seed: int, std: float):
    """(q, k, v, dout): q, k ~ N(0, std^2), so that scaled scores have a standard deviation of about std^2;
    v, dout ~ N(0, 1)."""
    return (
        randn((B, H, T, D), seed, std, dtype),
        randn((B, H, M, D), seed + 1, std, dtype),
        randn((B, H, M, D), seed + 2, 1.0, dtype),
        randn((B, H, T, D), seed + 3, 1.0, dtype),
    )
