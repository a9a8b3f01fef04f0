"""CPU emulation (float64) of the forward kernels' online-softmax rescaling, with planted mistakes.

The two forward kernels accumulate O and the row sum l against a running offset and rescale them when the
offset moves:
* the pipelined kernel (sdpa_fwd_pipe.hip): tile 0 sets the offset to its row max; a later 64-key tile keeps
  the offset unless a lane's partial row sum of the tile exceeds 2^20 (for any lane of the wave), and then
  moves the offset to the exact running max and rescales O and l by alpha = 2^(m_old - m_new);
* the general kernel (sdpa_fwd.hip): the offset moves lazily, only when a tile's row max exceeds it by more
  than 8 (log2 units), with the same rescale.
This file restates both schedules in float64 (no 16-bit rounding), checks them against the oracle, and shows
that a wrong alpha (1, or O or l left unscaled) is invisible on N(0, 1) inputs -- the rescale never runs
after tile 0 there -- but fails the planted late-maximum inputs that tests/test_gpu_precision.py gives the
GPU kernels. Reference: the online softmax of theria/attention/triton_qk.py:280-290.
"""

import math

import numpy as np
import pytest
import torch

from inputs_planted import planted_late_key
from oracle import sdpa_oracle as O

LOG2E = 1.4426950408889634


def emulate(q, k, v, scale, kernel: str, mistake: str | None = None, causal: bool = False, wave_rows: int = 32):
    """(O, lse, number of rescales after the first tile) of one head, q (T, D), k, v (M, D) as float64."""
    T, M = q.shape[0], k.shape[0]
    c2 = scale * LOG2E
    S = (q @ k.T) * c2  # log2 domain
    if causal:
        S = np.where(np.tri(T, M, dtype=bool), S, -np.inf)
    m_use = np.full(T, -np.inf)
    l = np.zeros(T)
    o = np.zeros((T, v.shape[1]))
    late = 0
    for t0 in range(0, M, 64):
        st = S[:, t0 : t0 + 64]
        mx = st.max(axis=1)
        if kernel == "pipe":
            if t0 == 0:
                move = np.ones(T, dtype=bool)
            else:
                with np.errstate(invalid="ignore", over="ignore"):
                    p = np.exp2(st - m_use[:, None])
                # lane partial sums: a lane holds 32 of the tile's 64 keys
                lane = np.maximum(p[:, :32].sum(axis=1), p[:, 32:].sum(axis=1))
                bad = ~(lane <= 2.0**20)
                # the exact path runs for the whole wave when any of its rows fails the check
                per_wave = np.pad(bad, (0, -T % wave_rows)).reshape(-1, wave_rows).any(axis=1)
                move = np.repeat(per_wave, wave_rows)[:T]
                late += int(bad.any())
        else:  # general kernel: lazy move by more than 8 (log2)
            move = mx > m_use + 8.0
            if t0 > 0:
                late += int(move.any())
        m_new = np.where(move, np.maximum(m_use, mx), m_use)
        with np.errstate(invalid="ignore"):
            alpha = np.where(np.isneginf(m_new), 1.0, np.exp2(m_use - m_new))
        if mistake == "alpha_one":
            alpha = np.ones(T)
        if mistake != "l_unscaled":
            l = l * alpha
        if mistake != "o_unscaled":
            o = o * alpha[:, None]
        m_use = m_new
        off = np.where(np.isneginf(m_use), 0.0, m_use)
        p = np.exp2(st - off[:, None])
        l = l + p.sum(axis=1)
        o = o + p @ v[t0 : t0 + 64]
    with np.errstate(divide="ignore", invalid="ignore"):
        return o / l[:, None], (m_use + np.log2(l)) / LOG2E, late


def _head(t):
    return t[0, 0].double().numpy()


def _planted(T, M, D, key, gap, dt=torch.bfloat16):
    s = 1 / math.sqrt(D)
    q, k, v = planted_late_key(1, 1, T, M, D, dt, 60, key, gap, s)
    return _head(q), _head(k), _head(v), s


def _normal(T, M, D, seed=3):
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(1, 1, n, D, generator=g).to(torch.bfloat16) for n in (T, M, M))
    return _head(q), _head(k), _head(v), 1 / math.sqrt(D)


def _oracle(q, k, v, s, causal=False):
    o, lse, _, _ = O.forward(torch.from_numpy(q)[None, None], torch.from_numpy(k)[None, None],
                             torch.from_numpy(v)[None, None], s, causal)
    return o[0, 0].numpy(), lse[0, 0].numpy()


@pytest.mark.parametrize("kernel", ["pipe", "general"])
@pytest.mark.parametrize("causal", [False, True])
def test_emulation_matches_the_oracle_on_planted_inputs(kernel, causal):
    q, k, v, s = _planted(320, 320, 64, 290 if not causal else 100, 24.0)
    o, lse, late = emulate(q, k, v, s, kernel, causal=causal)
    ro, rlse = _oracle(q, k, v, s, causal)
    assert late > 0, "the planted key must move the offset after the first tile"
    np.testing.assert_allclose(o, ro, rtol=0, atol=1e-12)
    np.testing.assert_allclose(lse, rlse, rtol=0, atol=1e-12)


@pytest.mark.parametrize("kernel", ["pipe", "general"])
@pytest.mark.parametrize("mistake", ["alpha_one", "o_unscaled", "l_unscaled"])
def test_planted_mistakes_fail_on_planted_inputs_only(kernel, mistake):
    # N(0, 1) inputs (config-2 statistics): the offset never moves after tile 0, so a wrong rescale is invisible
    q, k, v, s = _normal(256, 512, 64)
    o, lse, late = emulate(q, k, v, s, kernel, mistake=mistake)
    ro, rlse = _oracle(q, k, v, s)
    assert late == 0
    np.testing.assert_allclose(o, ro, rtol=0, atol=1e-12)
    # the planted late maximum exposes it: far beyond the 2e-2 bar of the GPU tests
    q, k, v, s = _planted(320, 320, 64, 290, 24.0)
    o, lse, late = emulate(q, k, v, s, kernel, mistake=mistake)
    ro, rlse = _oracle(q, k, v, s)
    assert late > 0
    err = max(np.nanmax(np.abs(o - ro)), np.nanmax(np.abs(lse - rlse)) if mistake != "o_unscaled" else 0.0)
    assert not np.isfinite(err) or err > 0.1, f"{mistake} should be visible ({err})"
