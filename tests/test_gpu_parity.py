"""GPU parity of the HIP kernels (through the C ABI) against the CPU oracle.

Bars (tests/bars.py): float32 within 1e-5 abs/rel; float16/bfloat16 outputs within 2e-2 abs plus one rounding
unit of the output dtype (2^-8 bfloat16, 2^-11 float16) relative. Inputs are
generated on the CPU with a seeded generator, rounded to the compute dtype, and the oracle receives
exactly those rounded values in float64 (as the reference's GPU tests do, test_triton_sdpa_dq.py:30-31).
Full-size configs are checked on sampled heads plus size-independent invariants:
  sum_j dV_j = sum_i dO_i (rows of P sum to 1), sum_j dK_j = 0 (rows of dS sum to 0),
  O(q, k + c, v) = O(q, k, v) (softmax shift invariance), O(q, k, v + c) = O(q, k, v) + c.
"""

import math
import random
from pathlib import Path

import numpy as np
import pytest
import torch

import bars
from oracle import sdpa_oracle as O
from theria_amd import _ops

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden" / "c1_fp32.npz"


tol = bars.tol


def stat_tol(dtype):
    """Row statistics (lse, l). float32: 1e-5. 16-bit inputs: the row sum is accumulated from the
    16-bit-rounded probabilities that also feed the PV product (so the weights of O sum to one exactly);
    each carries a relative rounding error below 2^-8 (bfloat16; 2^-11 for float16), so l is within a
    relative 2^-8 of the float32 sum and lse within 2^-8 absolute: 4e-3."""
    return dict(rtol=1e-5, atol=1e-5) if dtype == torch.float32 else dict(rtol=4e-3, atol=4e-3)


def close(gpu, ref, dtype, what):
    _close(gpu, ref, dtype, what)


def _close(gpu, ref, dtype, what):
    bars.close(gpu, ref, what=what, **tol(dtype))


def make(shape, dtype, dev, seed, std=1.0):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(*shape, generator=g) * std).to(dtype)
    return x.to(dev), x.double()


CASES = [
    # dtype, B, H, T, M, D, causal
    (torch.float32, 2, 2, 16, 16, 8, False),
    (torch.float32, 1, 2, 37, 53, 24, False),
    (torch.float32, 1, 1, 1, 32, 64, False),
    (torch.float32, 2, 1, 9, 1, 4, False),
    (torch.float32, 1, 2, 70, 70, 32, True),
    (torch.float32, 1, 1, 64, 96, 128, False),
    (torch.float16, 1, 1, 32, 32, 32, False),
    (torch.float16, 2, 4, 128, 128, 64, False),
    (torch.bfloat16, 2, 3, 130, 200, 64, False),
    (torch.bfloat16, 1, 2, 150, 150, 64, True),
    (torch.bfloat16, 1, 2, 96, 80, 128, False),
    (torch.bfloat16, 1, 1, 1, 17, 16, False),
    (torch.float16, 1, 2, 200, 200, 128, True),
    # several full 128-row tiles plus ragged ends (head dim 128 runs the backward on 128-row tiles)
    (torch.bfloat16, 1, 2, 600, 600, 128, True),
    (torch.float16, 1, 1, 520, 777, 128, False),
    # causal blocks run in mirrored pairs: odd block counts (a middle block that runs alone) and T != M
    (torch.bfloat16, 1, 2, 300, 300, 64, True),
    (torch.float16, 2, 1, 390, 390, 128, True),
    (torch.bfloat16, 1, 2, 200, 330, 64, True),
    (torch.bfloat16, 1, 1, 330, 200, 64, True),
    # head dims below the pipelined kernels' 64 / 128 (multiples of 8): zero-filled columns past D
    (torch.bfloat16, 1, 2, 300, 260, 80, False),
    (torch.float16, 1, 2, 200, 200, 96, True),
    (torch.bfloat16, 2, 1, 257, 257, 48, True),
    (torch.bfloat16, 1, 1, 333, 129, 120, False),
    (torch.float16, 1, 2, 150, 170, 40, False),
    (torch.bfloat16, 1, 2, 260, 260, 72, True),
    # head dims 8..32 (multiples of 8) in the pipelined kernels at DP = 32: 64-byte tile rows, four- and two-wave
    # workgroups, zero-filled columns past D
    (torch.bfloat16, 2, 2, 300, 260, 32, False),
    (torch.float16, 1, 3, 257, 190, 32, True),
    (torch.bfloat16, 1, 2, 520, 520, 16, True),
    (torch.bfloat16, 2, 2, 200, 333, 24, False),
    (torch.float16, 1, 1, 700, 700, 8, False),
    (torch.bfloat16, 4, 4, 1030, 1030, 16, True),
]


def _ids(c):
    dt, B, H, T, M, D, causal = c
    return f"{str(dt).split('.')[-1]}-B{B}H{H}T{T}M{M}D{D}{'-causal' if causal else ''}"


@pytest.mark.parametrize("case", CASES, ids=[_ids(c) for c in CASES])
def test_kernels_match_oracle(case, hip_device):
    print(f"[parity] {_ids(case)}", flush=True)
    _check_all_entry_points(case, hip_device, seed=1)


def _random_cases(n: int = 120, seed: int = 2024):
    """Seeded random configurations: dtype, head dim 8-128, 1-700 query / key rows, T != M, causal."""
    rng = random.Random(seed)
    cases = []
    for _ in range(n):
        dt = rng.choice([torch.float32, torch.float16, torch.bfloat16])
        D = rng.choice([8, 16, 24, 32, 40, 64, 64, 96, 128, 128])
        T = rng.choice([1, rng.randint(2, 100), rng.randint(100, 700)])
        M = rng.choice([T, rng.randint(1, 100), rng.randint(100, 700)])
        B, H = rng.choice([(1, 1), (1, 2), (2, 1), (2, 2)])
        cases.append((dt, B, H, T, M, D, rng.random() < 0.4))
    return cases


RANDOM_CASES = _random_cases()


@pytest.mark.parametrize("case", RANDOM_CASES, ids=[f"r{i}-" + _ids(c) for i, c in enumerate(RANDOM_CASES)])
def test_random_configurations_match_oracle(case, hip_device):
    print(f"[parity random] {_ids(case)}", flush=True)
    _check_all_entry_points(case, hip_device, seed=100)


def test_row_term_of_a_long_head(hip_device):
    """bf16 at head dim 128: the row term dO . O over 128 columns of the 16-bit O is off by its rounding (here
    0.022 on |delta| = 7.2, over the 2e-2 absolute bar alone), so the 16-bit row term is held to the 16-bit bar.
    Found by a random sweep (the generator of _random_cases, seed 21, case 721)."""
    _check_all_entry_points((torch.bfloat16, 2, 2, 82, 82, 128, False), hip_device, seed=1021)


def _check_all_entry_points(case, dev, seed: int):
    """Forward (O, lse, m, l), backward (with O, from stats, dV only), JVP (saved / rebuilt O, one tangent)
    and the double backward (all cotangents, one) against the float64 oracle on the same inputs."""
    dt, B, H, T, M, D, causal = case
    shapes = [(B, H, T, D), (B, H, M, D), (B, H, M, D), (B, H, T, D), (B, H, T, D), (B, H, M, D), (B, H, M, D)]
    g = [torch.Generator().manual_seed(seed + i) for i in range(7)]
    ts = [torch.randn(*sh, generator=gi).to(dt) for sh, gi in zip(shapes, g)]
    check_entry_points_on(dev, dt, causal, *ts)


def flag_all(lse):
    """lse with the peaked-row flag set on every finite entry (the backward's exact path everywhere)."""
    bits = lse.view(torch.int32)
    return torch.where(torch.isfinite(lse), bits | 1, bits).view(torch.float32)


def check_entry_points_on(dev, dt, causal, q, k, v, do, tq, tk, tv, scale=None, fp32_ref_err=None, orders=(1, 2)):
    """Every entry point on the given CPU inputs (already rounded to dt) against the float64 oracle.

    Bars: tol(dt) for outputs in the input dtype; float32 outputs of 16-bit inputs (O with a float32
    output, lse) carry no output rounding, so they are held to an absolute bound alone: 2e-2 for O (the
    north star's bar), 4e-3 for lse (the row sum is accumulated from probabilities rounded to 16 bits,
    each within a relative 2^-8 of its float32 value, so log l is within 2^-8 absolute).
    fp32_ref_err (float32 only): {quantity: largest error of theria's float32 PyTorch path against the
    oracle on these inputs}; a quantity listed there may be off by up to twice that error (when it exceeds
    1e-5), since float32 arithmetic itself cannot reach 1e-5 there.
    orders: 1 checks the forward, backward and JVP entry points, 2 the double backward (the forward is checked
    either way)."""
    qc, kc, vc, doc, tqc, tkc, tvc = (t.double() for t in (q, k, v, do, tq, tk, tv))
    q, k, v, do, tq, tk, tv = (t.to(dev) for t in (q, k, v, do, tq, tk, tv))
    s = 1 / math.sqrt(q.shape[-1]) if scale is None else scale
    f32_out = dict(rtol=1e-5, atol=1e-5) if dt == torch.float32 else dict(rtol=0, atol=2e-2)
    lse_tol = dict(rtol=1e-5, atol=1e-5) if dt == torch.float32 else dict(rtol=0, atol=4e-3)

    def close(gpu, ref, dtype, what):
        base = what if fp32_ref_err and what in fp32_ref_err else what.split("(")[0]
        if dtype == torch.float32 and fp32_ref_err and base in fp32_ref_err:
            atol = max(1e-5, 2 * fp32_ref_err[base])
            bars.close(gpu, ref, rtol=1e-5, atol=atol, what=f"{what} (float32 reference error {fp32_ref_err[base]:.2e})")
        else:
            _close(gpu, ref, dtype, what)

    o, lse, m, l = _ops.fwd(q, k, v, s, causal, stats=True)
    o32, lse32, _, _ = _ops.fwd(q, k, v, s, causal, out_fp32=True)
    Or, lser, mr, lr = O.forward(qc, kc, vc, s, causal)
    close(o, Or, dt, "O")
    torch.testing.assert_close(o32.double().cpu(), Or, **f32_out, msg=lambda m_: f"O(fp32 out): {m_}")
    torch.testing.assert_close(lse.double().cpu(), lser, **lse_tol, msg=lambda m_: f"lse: {m_}")
    torch.testing.assert_close(lse32.double().cpu(), lser, **lse_tol, msg=lambda m_: f"lse(fp32 out): {m_}")
    torch.testing.assert_close(m.double().cpu(), mr, rtol=1e-5, atol=1e-5, msg=lambda m_: f"m: {m_}")
    torch.testing.assert_close(l.double().cpu(), lr, **stat_tol(dt), msg=lambda m_: f"l: {m_}")

    def second_order(delta):
        G = _ops.bwd_bwd(q, k, v, o, do, lse, delta, tq, tk, tv, s, causal)
        Gr = O.double_backward(qc, kc, vc, doc, tqc, tkc, tvc, s, causal)
        for name, a, b in zip(("G_Q", "G_K", "G_V", "G_dO"), G, Gr):
            close(a, b, dt, name)
        G2 = _ops.bwd_bwd(q, k, v, o, do, lse, delta, None, tk, None, s, causal)
        G2r = O.double_backward(qc, kc, vc, doc, None, tkc, None, s, causal)
        for name, a, b in zip(("G_Q(gk)", "G_K(gk)", "G_V(gk)", "G_dO(gk)"), G2, G2r):
            close(a, b, dt, name)

    if 1 not in orders:
        if 2 in orders:
            second_order(_ops.bwd(q, k, v, o, lse, do, s, causal)[3])
        return

    if dt != torch.float32:
        # the forward flags every row whose largest probability exceeds 1/4 (its bound may flag a few more)
        flagged = (lse.cpu().view(torch.int32) & 1).bool()
        pmax = (mr - lser).exp()
        missed = (pmax > 0.25 * (1 + 1e-3)) & ~flagged
        assert not missed.any(), f"peaked rows not flagged in lse: {int(missed.sum())}"
    else:
        assert torch.equal(lse.cpu(), lse32.cpu()), "float32 lse carries no flags"

    # the backward as the autograd operator runs it: the forward's lse with its peaked-row flags
    dq, dk, dv, delta = _ops.bwd(q, k, v, o, lse, do, s, causal)
    ref = O.backward(qc, kc, vc, doc, s, causal)
    for name, a, b in zip(("dQ", "dK", "dV"), (dq, dk, dv), ref):
        close(a, b, dt, name)
    # the row term: dO . O, or its exact form sum_j P_ij dP_ij / sum_j P_ij on query blocks holding a peaked
    # row; both equal the oracle's dO . O_exact within the 16-bit bar (dO . O reads the forward's 16-bit O, whose
    # rounding, 2^-9 relative per element, carries into the sum: one rounding unit of |delta| on top of 2e-2)
    delta_tol = f32_out if dt == torch.float32 else bars.tol(dt)
    torch.testing.assert_close(delta.double().cpu(), (doc * Or).sum(-1), **delta_tol, msg=lambda m_: f"delta: {m_}")
    # every 16-bit row flagged peaked: two-term operands and the exact row term everywhere
    aq, ak, av, adelta = _ops.bwd(q, k, v, o, flag_all(lse) if dt != torch.float32 else lse, do, s, causal)
    torch.testing.assert_close(adelta.double().cpu(), (doc * Or).sum(-1), **delta_tol,
                               msg=lambda m_: f"delta(all peaked): {m_}")
    for name, a, b in zip(("dQ(all split)", "dK(all split)", "dV(all split)"), (aq, ak, av), ref):
        close(a, b, dt, name)

    # the reference's explicit frozen-stats backward: P = exp(S - lse) for exactly the lse it is given
    fref = O.frozen_backward(qc, kc, vc, doc, lse.double().cpu(), s, causal)
    if dt == torch.float32 and fp32_ref_err is not None:
        # the same formula in float32 arithmetic (exp(S - lse) with S, lse ~ 30 loses ~2^-24 * 30 relative)
        f32 = O.frozen_backward(qc, kc, vc, doc, lse.double().cpu(), s, causal, dtype=torch.float32)
        for name, a_, b_ in zip(("dQ(stats)", "dK(stats)", "dV(stats)"), f32, fref):
            fp32_ref_err[name] = float((a_.double() - b_).abs().max())
        fp32_ref_err["dV(no v)"] = fp32_ref_err["dV(stats)"]
    sq, sk, sv = _ops.bwd_from_stats(q, k, v, do, lse, s, causal, True, True, True)
    for name, a, b in zip(("dQ(stats)", "dK(stats)", "dV(stats)"), (sq, sk, sv), fref):
        close(a, b, dt, name)
    _, _, dv_only = _ops.bwd_from_stats(q, k, None, do, lse, s, causal, False, False, True)
    close(dv_only, fref[2], dt, "dV(no v)")
    # normalised row term: the exact softmax gradient from the operator's own lse
    nq, nk, nv = _ops.bwd_from_stats(q, k, v, do, lse, s, causal, True, True, True, normalize=True)
    for name, a, b in zip(("dQ(stats, normalised)", "dK(stats, normalised)", "dV(stats, normalised)"), (nq, nk, nv), ref):
        close(a, b, dt, name)

    jr = O.jvp(qc, kc, vc, tqc, tkc, tvc, s, causal)
    close(_ops.jvp(q, k, v, o, lse, tq, tk, tv, s, causal), jr, dt, "JVP(saved O)")
    close(_ops.jvp(q, k, v, None, lse, tq, tk, tv, s, causal), jr, dt, "JVP(rebuilt O)")
    close(_ops.jvp(q, k, v, o, lse, tq, None, None, s, causal), O.jvp(qc, kc, vc, tqc, None, None, s, causal), dt, "JVP(tq only)")
    if 2 in orders:
        second_order(delta)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_double_backward_single_visible_key_row(dt, hip_device):
    """Causal query 0 sees one key, so P = 1 on that row and dS, r - Gam and every second-order term of the
    row vanish: G_Q[..., 0, :] = 0 in exact arithmetic. The G_Q expression subtracts the products
    sum_j (P o E1)_ij K_j and t_i sum_j P_ij K_j; with 16-bit operands they cancel only if t is summed from
    the same rounded P o E1 values (otherwise the row is left with the rounding of E1, ~1e-2 here)."""
    B, H, T, D = 2, 2, 300, 64
    q, _ = make((B, H, T, D), dt, hip_device, 21)
    k, _ = make((B, H, T, D), dt, hip_device, 22)
    v, _ = make((B, H, T, D), dt, hip_device, 23)
    do, _ = make((B, H, T, D), dt, hip_device, 24)
    tq, tk, tv = (make((B, H, T, D), dt, hip_device, 25 + i)[0] for i in range(3))
    s = 1 / math.sqrt(D)
    print(f"[single-key row] {dt}", flush=True)
    o, lse, _, _ = _ops.fwd(q, k, v, s, True)
    _, _, _, delta = _ops.bwd(q, k, v, o, lse, do, s, True)
    G = _ops.bwd_bwd(q, k, v, o, do, lse, delta, tq, tk, tv, s, True)
    row0 = G[0][:, :, 0].float().abs().max().item()
    assert row0 <= 1e-3, f"G_Q of the single-key row: {row0}"


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16, torch.float32])
def test_double_backward_ignores_delta(dt, hip_device):
    """The double backward forms its own row term (and, for 16-bit inputs, the row normaliser; for float32, the
    rows' own max and sum) in a pass over the keys, so the delta argument is not read: None, the backward's delta
    and a wrong delta give the same bits."""
    B, H, T, M, D = 1, 2, 200, 180, 64
    q, _ = make((B, H, T, D), dt, hip_device, 31)
    k, _ = make((B, H, M, D), dt, hip_device, 32)
    v, _ = make((B, H, M, D), dt, hip_device, 33)
    do, _ = make((B, H, T, D), dt, hip_device, 34)
    tq, tk, tv = (make(t.shape, dt, hip_device, 35 + i)[0] for i, t in enumerate((q, k, v)))
    s = 1 / math.sqrt(D)
    print(f"[bwd_bwd without delta] {dt}", flush=True)
    o, lse, _, _ = _ops.fwd(q, k, v, s, False)
    delta = _ops.bwd(q, k, v, o, lse, do, s, False)[3]
    ref = _ops.bwd_bwd(q, k, v, o, do, lse, delta, tq, tk, tv, s, False)
    for d in (None, delta + 5.0):
        got = _ops.bwd_bwd(q, k, v, o, do, lse, d, tq, tk, tv, s, False)
        for name, a, b in zip(("G_Q", "G_K", "G_V", "G_dO"), got, ref):
            assert torch.equal(a, b), f"{name} depends on delta ({dt})"


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_double_backward_every_cotangent_subset(dt, causal, hip_device):
    """Every non-empty subset of (gQ, gK, gV) against the oracle at 16-bit head dim 64 (the key-split row kernel
    and the query-split column kernel with their presence tests at run time; all three given takes the
    variant where they are constants). Ragged sizes: T and M are not multiples of the tiles."""
    B, H, T, M, D = 2, 2, 301, 275, 64
    q, qc = make((B, H, T, D), dt, hip_device, 61)
    k, kc = make((B, H, M, D), dt, hip_device, 62)
    v, vc = make((B, H, M, D), dt, hip_device, 63)
    do, doc = make((B, H, T, D), dt, hip_device, 64)
    gs = [make(t.shape, dt, hip_device, 65 + i, std=0.5) for i, t in enumerate((q, k, v))]
    s = 1 / math.sqrt(D)
    o, lse, _, _ = _ops.fwd(q, k, v, s, causal)
    for mask in range(1, 8):
        pick = [gs[i] if mask >> i & 1 else (None, None) for i in range(3)]
        tag = "".join(n for i, n in enumerate(("q", "k", "v")) if mask >> i & 1)
        print(f"[bwd_bwd cotangents g{tag}] {dt} causal={causal}", flush=True)
        G = _ops.bwd_bwd(q, k, v, o, do, lse, None, *(p[0] for p in pick), s, causal)
        Gr = O.double_backward(qc, kc, vc, doc, *(p[1] for p in pick), s, causal)
        for name, a, b in zip(("G_Q", "G_K", "G_V", "G_dO"), G, Gr):
            close(a, b, dt, f"{name}(g{tag})")


# bfloat16 causal cases whose G_Q on the first rows (two to ten visible keys) missed the bar by up to 0.044
# while the rows kernel formed G_Q from uncentred products; (case, seed) as a random sweep drew them.
CENTRED_GQ_CASES = [
    ((torch.bfloat16, 2, 2, 769, 191, 64, True), 1520),
    ((torch.bfloat16, 1, 2, 191, 191, 88, True), 1254),
    ((torch.bfloat16, 2, 2, 864, 702, 40, True), 1077),
    ((torch.bfloat16, 2, 2, 53, 53, 112, True), 1992),
]


@pytest.mark.parametrize("case,seed", CENTRED_GQ_CASES, ids=[_ids(c) for c, _ in CENTRED_GQ_CASES])
def test_double_backward_few_key_rows(case, seed, hip_device):
    print(f"[few-key G_Q] {_ids(case)} seed {seed}", flush=True)
    dt, B, H, T, M, D, causal = case
    q, qc = make((B, H, T, D), dt, hip_device, seed)
    k, kc = make((B, H, M, D), dt, hip_device, seed + 1)
    v, vc = make((B, H, M, D), dt, hip_device, seed + 2)
    do, doc = make((B, H, T, D), dt, hip_device, seed + 3)
    tq, tqc = make((B, H, T, D), dt, hip_device, seed + 4)
    tk, tkc = make((B, H, M, D), dt, hip_device, seed + 5)
    tv, tvc = make((B, H, M, D), dt, hip_device, seed + 6)
    s = 1 / math.sqrt(D)
    o, lse, _, _ = _ops.fwd(q, k, v, s, causal)
    _, _, _, delta = _ops.bwd(q, k, v, o, lse, do, s, causal)
    G = _ops.bwd_bwd(q, k, v, o, do, lse, delta, tq, tk, tv, s, causal)
    Gr = O.double_backward(qc, kc, vc, doc, tqc, tkc, tvc, s, causal)
    close(G[0], Gr[0], dt, "G_Q")


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_dv_only_backward_float32(D, causal, hip_device):
    """The dV-only backward (no V: the reference's sdpa_bwd_dv) in float32 at head dims 64 and 128 with
    several query tiles, the regime where an earlier runtime-flag form of it returned wrong dV; here the
    DV_ONLY variant of the dK/dV kernel, through the explicit API, against the frozen-stats oracle."""
    from theria_amd.attention import explicit

    print(f"[dv only] fp32 D{D} causal={causal}", flush=True)
    B, H, T, M = 1, 2, 200, 170 if not causal else 200
    g = torch.Generator().manual_seed(7 + D)
    q, k, v, do = (torch.randn(B, H, n, D, generator=g) for n in (T, M, M, T))
    s = 1 / math.sqrt(D)
    dev = hip_device
    _, lse, m, l = _ops.fwd(q.to(dev), k.to(dev), v.to(dev), s, causal, stats=True)
    ref = O.frozen_backward(q.double(), k.double(), v.double(), do.double(), lse.double().cpu(), s, causal)[2]
    _, _, dv = _ops.bwd_from_stats(q.to(dev), k.to(dev), None, do.to(dev), lse, s, causal, False, False, True)
    _close(dv, ref, torch.float32, "dV(no v)")
    if not causal:  # the reference's sdpa_bwd_dv(q, k, dout, m, l, scale) takes no causal flag
        dv2 = explicit.sdpa_bwd_dv(q.to(dev), k.to(dev), do.to(dev), m, l, s)
        lse_ml = (m.double() + torch.log(l.double())).cpu()
        ref2 = O.frozen_backward(q.double(), k.double(), v.double(), do.double(), lse_ml, s, causal)[2]
        _close(dv2, ref2, torch.float32, "sdpa_bwd_dv")


def test_config1_golden_fixture_fp32(hip_device):
    """Config 1 (B2 H2 S16 D8, float32) against the committed fixture, 1e-5."""
    z = np.load(GOLDEN, allow_pickle=False)
    t = {k: torch.from_numpy(z[k]) for k in z.files}
    dev = hip_device
    q, k, v, do = (t[f"in_{n}"].to(dev) for n in ("q", "k", "v", "dout"))
    s = 1 / math.sqrt(8)
    o, lse, m, l = _ops.fwd(q, k, v, s, False, stats=True)
    for name, a in dict(o=o, lse=lse, m=m, l=l).items():
        close(a, t[f"out_{name}"], torch.float32, name)
    dq, dk, dv, delta = _ops.bwd(q, k, v, o, lse, do, s, False)
    for name, a in dict(dq=dq, dk=dk, dv=dv).items():
        close(a, t[f"out_{name}"], torch.float32, name)
    tq, tk, tv = (t[f"in_{n}"].to(dev) for n in ("tq", "tk", "tv"))
    close(_ops.jvp(q, k, v, o, lse, tq, tk, tv, s, False), t["out_jvp"], torch.float32, "jvp")
    w, vq, vk, vv = (t[f"in_{n}"].to(dev) for n in ("w", "vq", "vk", "vv"))
    _, _, _, delta_w = _ops.bwd(q, k, v, o, lse, w, s, False)
    G = _ops.bwd_bwd(q, k, v, o, w, lse, delta_w, vq, vk, vv, s, False)
    for name, a in zip(("hvp_q", "hvp_k", "hvp_v"), G[:3]):
        close(a, t[f"out_{name}"], torch.float32, name)


def test_empty_and_degenerate_shapes(hip_device):
    dev = hip_device
    # no keys: O = 0, lse = -inf (a softmax over nothing contributes nothing)
    q = torch.randn(1, 2, 5, 16, device=dev)
    k = torch.randn(1, 2, 0, 16, device=dev)
    o, lse, _, _ = _ops.fwd(q, k, k, 0.25, False)
    assert torch.equal(o, torch.zeros_like(o)) and torch.isneginf(lse).all()
    dq, dk, dv, _ = _ops.bwd(q, k, k, o, lse, torch.randn_like(q), 0.25, False)
    assert torch.equal(dq, torch.zeros_like(dq)) and dk.numel() == 0 and dv.numel() == 0
    # no queries: nothing to compute, dK = dV = 0
    q0 = torch.randn(1, 2, 0, 16, device=dev)
    k1 = torch.randn(1, 2, 7, 16, device=dev)
    o0, lse0, _, _ = _ops.fwd(q0, k1, k1, 0.25, False)
    assert o0.numel() == 0
    _, dk0, dv0, _ = _ops.bwd(q0, k1, k1, o0, lse0, o0, 0.25, False)
    assert torch.equal(dk0, torch.zeros_like(dk0)) and torch.equal(dv0, torch.zeros_like(dv0))


def test_strided_inputs(hip_device):
    """Non-contiguous (B,H,T,D) views with a contiguous last dimension (e.g. a fused qkv projection)."""
    dev = hip_device
    B, T, H, D = 2, 40, 3, 32
    g = torch.Generator().manual_seed(0)
    qkv = torch.randn(B, T, 3, H, D, generator=g).to(torch.bfloat16)
    q, k, v = qkv.to(dev).permute(2, 0, 3, 1, 4)
    qc, kc, vc = qkv.double().permute(2, 0, 3, 1, 4)
    assert not q.is_contiguous()
    o, lse, _, _ = _ops.fwd(q, k, v, 1 / math.sqrt(D), False)
    close(o, O.forward(qc, kc, vc)[0], torch.bfloat16, "O(strided)")
    do = torch.randn(B, H, T, D, generator=g).to(torch.bfloat16)
    dq, dk, dv, _ = _ops.bwd(q, k, v, o, lse, do.to(dev).transpose(2, 3).contiguous().transpose(2, 3), 1 / math.sqrt(D), False)
    for name, a, b in zip(("dQ", "dK", "dV"), (dq, dk, dv), O.backward(qc, kc, vc, do.double())):
        close(a, b, torch.bfloat16, name)


@pytest.mark.parametrize("D", [16, 48, 64])
def test_split_second_order_kernels_on_strided_views(D, hip_device):
    """The key-split JVP and the split double-backward kernels read their LDS-DMA tiles with the views' row strides
    (here (B, T, H, D) storage, row stride H * D) and, below head dim 64, zero-filled columns past D: the results
    equal those of contiguous copies bit for bit, and the oracle's."""
    dev = hip_device
    B, T, H = 2, 300, 3
    print(f"[parity] split kernels, strided views, D={D}", flush=True)
    g = torch.Generator().manual_seed(D)
    raw = torch.randn(7, B, T, H, D, generator=g).to(torch.bfloat16)
    views = [x.to(dev).transpose(1, 2) for x in raw]  # (B, H, T, D), row stride H * D
    assert not views[0].is_contiguous()
    q, k, v, do, tq, tk, tv = views
    qc, kc, vc, doc, tqc, tkc, tvc = (x.transpose(1, 2).double() for x in raw)
    s = 1 / math.sqrt(D)
    o, lse, _, _ = _ops.fwd(q, k, v, s, False)
    cont = [x.contiguous() for x in (q, k, v, do, tq, tk, tv)]
    jv = _ops.jvp(q, k, v, o, lse, tq, tk, tv, s, False)
    jvc = _ops.jvp(*cont[:3], o, lse, *cont[4:], s, False)
    assert torch.equal(jv, jvc), "JVP: strided and contiguous inputs differ"
    close(jv, O.jvp(qc, kc, vc, tqc, tkc, tvc, s, False), torch.bfloat16, "JVP(strided)")
    G = _ops.bwd_bwd(q, k, v, o, do, lse, None, tq, tk, tv, s, False)
    Gc = _ops.bwd_bwd(*cont[:3], o, cont[3], lse, None, *cont[4:], s, False)
    for name, a, b, r in zip(("G_Q", "G_K", "G_V", "G_dO"), G, Gc, O.double_backward(qc, kc, vc, doc, tqc, tkc, tvc, s, False)):
        assert torch.equal(a, b), f"{name}: strided and contiguous inputs differ"
        close(a, r, torch.bfloat16, f"{name}(strided)")


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_config2_full_size(dt, hip_device):
    """Config 2: B4 H16 S2048 D64, fwd+bwd; two heads vs the oracle, all heads via invariants."""
    dev = hip_device
    B, H, S, D = 4, 16, 2048, 64
    print(f"[parity] config2 {dt}", flush=True)
    q, qc = make((B, H, S, D), dt, dev, 11)
    k, kc = make((B, H, S, D), dt, dev, 12)
    v, vc = make((B, H, S, D), dt, dev, 13)
    do, doc = make((B, H, S, D), dt, dev, 14)
    s = 1 / 8.0
    o, lse, _, _ = _ops.fwd(q, k, v, s, False)
    dq, dk, dv, _ = _ops.bwd(q, k, v, o, lse, do, s, False)
    for b, h in ((0, 0), (3, 15)):
        sl = (slice(b, b + 1), slice(h, h + 1))
        Or, lser, _, _ = O.forward(qc[sl], kc[sl], vc[sl], s)
        close(o[sl], Or, dt, f"O[{b},{h}]")
        torch.testing.assert_close(lse[sl].double().cpu(), lser, **stat_tol(dt))
        for name, a, r in zip(("dQ", "dK", "dV"), (dq[sl], dk[sl], dv[sl]), O.backward(qc[sl], kc[sl], vc[sl], doc[sl], s)):
            close(a, r, dt, f"{name}[{b},{h}]")
    # invariants over every head
    torch.testing.assert_close(dv.double().sum(2), do.double().sum(2), rtol=0, atol=0.5)
    assert float(dk.double().sum(2).abs().max()) < 0.5
    c = torch.randn(1, 1, 1, D, device=dev).to(dt)
    o_shift, _, _, _ = _ops.fwd(q, k + c, v, s, False)
    torch.testing.assert_close(o_shift.float(), o.float(), rtol=0, atol=3e-2)
    o_vc, _, _, _ = _ops.fwd(q, k, v + c, s, False)
    torch.testing.assert_close(o_vc.float(), (o.float() + c.float()), rtol=0, atol=3e-2)


def test_config3_causal_long_sequence(hip_device):
    """Config 3: B1 H32 S8192 D128 causal bf16, inputs 0.5*N(0,1); one head vs the oracle."""
    dev = hip_device
    B, H, S, D = 1, 32, 8192, 128
    dt = torch.bfloat16
    print("[parity] config3", flush=True)
    q, qc = make((B, H, S, D), dt, dev, 21, std=0.5)
    k, kc = make((B, H, S, D), dt, dev, 22, std=0.5)
    v, vc = make((B, H, S, D), dt, dev, 23, std=0.5)
    do, doc = make((B, H, S, D), dt, dev, 24)
    s = 1 / math.sqrt(D)
    o, lse, _, _ = _ops.fwd(q, k, v, s, True)
    dq, dk, dv, _ = _ops.bwd(q, k, v, o, lse, do, s, True)
    h = 7
    sl = (slice(0, 1), slice(h, h + 1))
    Or, _, _, _ = O.forward(qc[sl], kc[sl], vc[sl], s, True)
    close(o[sl], Or, dt, "O[h7]")
    for name, a, r in zip(("dQ", "dK", "dV"), (dq[sl], dk[sl], dv[sl]), O.backward(qc[sl], kc[sl], vc[sl], doc[sl], s, True)):
        close(a, r, dt, f"{name}[h7]")
    torch.testing.assert_close(dv.double().sum(2), do.double().sum(2), rtol=0, atol=0.5)
    # causal: the first query sees only key 0
    torch.testing.assert_close(o[:, :, 0].float(), v[:, :, 0].float(), rtol=0, atol=1e-2)


@pytest.mark.parametrize("S,H,causal", [(1999, 16, False), (1040, 32, True)])
def test_large_grids_ragged(S, H, causal, hip_device):
    """Grids large enough that the head-dim-64 dK/dV launcher picks eight-wave workgroups (at least one
    workgroup per CU), with a ragged sequence length; causal with an odd number of key blocks per head, so
    one workgroup of each head runs the middle block alone. Two heads vs the oracle, every head via the
    dV column-sum invariant."""
    dev = hip_device
    B, D, dt = 4, 64, torch.bfloat16
    print(f"[parity] large grid S{S} H{H} causal={causal}", flush=True)
    q, qc = make((B, H, S, D), dt, dev, 31)
    k, kc = make((B, H, S, D), dt, dev, 32)
    v, vc = make((B, H, S, D), dt, dev, 33)
    do, doc = make((B, H, S, D), dt, dev, 34)
    s = 1 / 8.0
    o, lse, _, _ = _ops.fwd(q, k, v, s, causal)
    dq, dk, dv, _ = _ops.bwd(q, k, v, o, lse, do, s, causal)
    for b, h in ((0, 1), (B - 1, H - 1)):
        sl = (slice(b, b + 1), slice(h, h + 1))
        for name, a, r in zip(("dQ", "dK", "dV"), (dq[sl], dk[sl], dv[sl]),
                              O.backward(qc[sl], kc[sl], vc[sl], doc[sl], s, causal)):
            close(a, r, dt, f"{name}[{b},{h}]")
    torch.testing.assert_close(dv.double().sum(2), do.double().sum(2), rtol=0, atol=0.5)


def test_caller_given_outputs_are_checked(hip_device):
    """bwd / bwd_bwd write into caller-given outputs only of the exact shape, dtype and row layout (the torch
    binding checks them before any launch), and results written there equal fresh ones."""
    dt, B, H, T, M, D = torch.bfloat16, 1, 2, 70, 90, 64
    q, k, v, do, gq, gk, gv = (make(sh, dt, hip_device, 200 + i)[0] for i, sh in
                               enumerate([(B, H, T, D), (B, H, M, D), (B, H, M, D), (B, H, T, D), (B, H, T, D),
                                          (B, H, M, D), (B, H, M, D)]))
    s = 1 / math.sqrt(D)
    print("[caller-given outputs]", flush=True)
    o, lse, _, _ = _ops.fwd(q, k, v, s, False)
    ref = _ops.bwd(q, k, v, o, lse, do, s, False)
    # a row-strided output (row stride 2 D, last dimension contiguous) is accepted
    dk_strided = torch.empty(B, H, M, 2 * D, dtype=dt, device=hip_device)[..., :D]
    outs = (torch.empty_like(q), dk_strided, torch.empty_like(v))
    got = _ops.bwd(q, k, v, o, lse, do, s, False, out=outs)
    for name, a, b in zip(("dQ", "dK", "dV"), got[:3], ref[:3]):
        assert torch.equal(a, b), f"{name} written to a caller-given output differs"
    assert got[1].data_ptr() == dk_strided.data_ptr()
    for bad in (torch.empty(B, H, M - 1, D, dtype=dt, device=hip_device),            # wrong rows
                torch.empty(B, H, M, D, dtype=torch.float32, device=hip_device),    # wrong dtype
                torch.empty(B, H, D, M, dtype=dt, device=hip_device).transpose(-1, -2)):  # last dim strided
        with pytest.raises(AssertionError):
            _ops.bwd(q, k, v, o, lse, do, s, False, out=(torch.empty_like(q), bad, torch.empty_like(v)))
        with pytest.raises(AssertionError):
            _ops.bwd_bwd(q, k, v, o, do, lse, None, gq, gk, gv, s, False,
                         out=(torch.empty_like(q), bad, torch.empty_like(v)))
    with pytest.raises(AssertionError, match="dout"):
        _ops.bwd(q, k, v, o, lse, do[:, :, :-1], s, False)


@pytest.mark.parametrize("causal", [False, True])
def test_tile_counting_build(causal, hip_device):
    """The counter-enabled build (libtheria_sdpa_tiles.so) gives the production library's results bit for bit and
    counts the 32 x 32 units its pipelined kernels run: every unit without a mask; with the causal mask at least
    every unit holding an unmasked element (key <= query) and fewer than all."""
    import ctypes

    from theria_amd import _lib

    dt, B, H, T, D = torch.bfloat16, 1, 2, 512, 128
    q, k, v, do = (make((B, H, T, D), dt, hip_device, 300 + i)[0] for i in range(4))
    s = 1 / math.sqrt(D)
    print(f"[tile counts] causal={causal}", flush=True)
    o, lse, _, _ = _ops.fwd(q, k, v, s, causal)
    dq, dk, dv, _ = _ops.bwd(q, k, v, o, lse, do, s, causal)
    lib = _lib.load(_lib.TILES_LIB_PATH)
    counts = (ctypes.c_uint64 * 3)()
    torch.cuda.synchronize()
    assert lib.theria_debug_tile_counts(counts, 1) == _lib.OK
    o2, lse2 = torch.empty_like(o), torch.empty_like(lse)
    dq2, dk2, dv2, delta2 = torch.empty_like(dq), torch.empty_like(dk), torch.empty_like(dv), torch.empty_like(lse)
    prob = _ops._problem(q, k, s, causal)
    st = _ops._stream(q.device)
    tv = _ops._tv
    assert lib.theria_sdpa_fwd(ctypes.byref(prob), tv(q), tv(k), tv(v), tv(o2), 0, lse2.data_ptr(), None, None,
                               st) == _lib.OK
    assert lib.theria_sdpa_bwd(ctypes.byref(prob), tv(q), tv(k), tv(v), tv(o2), 0, tv(do), lse2.data_ptr(),
                               delta2.data_ptr(), tv(dq2), tv(dk2), tv(dv2), st) == _lib.OK
    torch.cuda.synchronize()
    assert lib.theria_debug_tile_counts(counts, 1) == _lib.OK
    for name, a, b in (("O", o2, o), ("lse", lse2, lse), ("dQ", dq2, dq), ("dK", dk2, dk), ("dV", dv2, dv)):
        assert torch.equal(a, b), f"{name} of the counting build differs"
    n = T // 32
    total, needed = B * H * n * n, B * H * n * (n + 1) // 2
    for name, c in zip(("fwd", "dq", "dkdv"), counts):
        if causal:
            assert needed <= c < total, f"{name}: {c} units executed, {needed} needed, {total} in all"
        else:
            assert c == total, f"{name}: {c} units executed, {total} in the grid"
