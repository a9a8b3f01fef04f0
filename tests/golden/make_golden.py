"""Regenerate tests/golden/c1_fp32.npz: config 1 inputs and oracle outputs.

Config 1: Q, K, V ~ N(0,1), B=2, H=2, S=16, D=8, float32, non-causal, scale 1/sqrt(D); upstream dO,
tangents (tq, tk, tv), weight W and HVP direction (vq, vk, vv) all ~ N(0,1). Expected values come
from oracle/sdpa_oracle.py in float64 (the oracle itself is pinned by tests/test_oracle.py):
O, lse, m, l; dQ, dK, dV for dO; the JVP along (tq, tk, tv); the HVP of sum(O * W) along (vq, vk, vv).
Inputs are stored in float32 (exactly what the GPU receives), expected outputs in float64.

Run: python tests/golden/make_golden.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import sdpa_oracle as O  # noqa: E402

OUT = Path(__file__).resolve().parent / "c1_fp32.npz"


def make():
    g = torch.Generator().manual_seed(1)
    B, H, S, D = 2, 2, 16, 8
    names = ["q", "k", "v", "dout", "tq", "tk", "tv", "w", "vq", "vk", "vv"]
    inp = {n: torch.randn(B, H, S, D, generator=g, dtype=torch.float32) for n in names}
    q, k, v = inp["q"], inp["k"], inp["v"]
    o, lse, m, l = O.forward(q, k, v)
    dq, dk, dv = O.backward(q, k, v, inp["dout"])
    jvp = O.jvp(q, k, v, inp["tq"], inp["tk"], inp["tv"])
    hq, hk, hv = O.hvp_weighted_sum(q, k, v, inp["w"], inp["vq"], inp["vk"], inp["vv"])
    exp = dict(o=o, lse=lse, m=m, l=l, dq=dq, dk=dk, dv=dv, jvp=jvp, hvp_q=hq, hvp_k=hk, hvp_v=hv)
    arrays = {f"in_{n}": t.numpy() for n, t in inp.items()}
    arrays.update({f"out_{n}": t.numpy() for n, t in exp.items()})
    np.savez_compressed(OUT, **arrays)
    return OUT


if __name__ == "__main__":
    print(make())
