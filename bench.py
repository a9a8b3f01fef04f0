#!/usr/bin/env python
"""Benchmark of theria_amd's HIP SDPA operator on one MI355X.

Metric: SDPA fwd+bwd TFLOP/s and share of the bf16 MFMA peak at B4 H16 S2048 D64; JVP/HVP ms.

A "step" is one forward + backward pass of the SDPA operator over config 2
(B4 H16 S2048 D64, bfloat16, non-causal, scale 1/8, Q, K, V, dO ~ N(0,1), synthetic, resident in HBM):
forward kernel (O, lse), then the backward's two kernels (dQ with the row term, then dK/dV); query blocks /
tiles holding peaked rows (flagged in lse; none at config 2) take an exact path inside the same launches. Throughput counts algorithmic FLOPs, FlashAttention convention: 4*B*H*S^2*D forward,
10*B*H*S^2*D backward (the recomputed QK^T included), 14*B*H*S^2*D per step.

Printed as ONE JSON line (rank 0): value = TFLOP/s of the whole step, plus
  roofline     the dominant kernel (the backward's dK/dV kernel), its algorithmic FLOPs per launch over the
               average HIP-event duration of theria_sdpa_bwd_dkdv (one launch), against the dense bf16 MFMA peak; traffic = HBM bytes
               per launch from the rocprofv3 FETCH_SIZE / WRITE_SIZE runs (profiles/traffic.json);
  cpu_baseline the CPU oracle (oracle/sdpa_oracle.py, the reference's pure-PyTorch math, float32)
               timed on a bounded sample of heads of the same workload on this host's cores;
  extra        the other configs: C3 causal long sequence, C4 JVP / HVP ms, C5 MAML.
One GPU only: --gpus N with N > 1 exits with a message.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "SDPA fwd+bwd TFLOP/s & % MFMA peak, B4 H16 S2048 D64 bf16; JVP/HVP ms"
# MI355X dense bf16 MFMA peak: 256 CU x 4096 FLOP/clk/CU x 2.4 GHz (no sparsity).
PEAK_BF16_TFLOPS = 2516.6
PEAK_FP32_TFLOPS = 157.3
TRAFFIC_FILE = ROOT / "profiles" / "traffic.json"


def _args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    # The GPU runs its first few tens of milliseconds of work after idle at lower clocks; the default
    # warmup (~0.3 s of steps) reaches the steady state before the timed steps.
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=1000)
    ap.add_argument("--warmup-seconds", type=float, default=0.5,
                    help="warm up for at least this long as well as --warmup steps (clock ramp after idle)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="budget of the CPU-baseline sample")
    ap.add_argument("--no-extras", action="store_true", help="only the config-2 line (for profiling runs)")
    ap.add_argument("--extras", default="c2_fp16,c3,c4,c5,scores",
                    help="comma-separated subset of the other configs to run (c2_fp16, c3, c4, c5, scores)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline (for profiling runs)")
    ap.add_argument("--copy-calibration", action="store_true", help="run a plain copy of known size (PMC scaling)")
    ap.add_argument("--atomic-probe", action="store_true",
                    help="time float32 atomic adds into a config-2 dQ-sized buffer (the fused-backward bound)")
    return ap.parse_args()


def _rand(shape, dtype, dev, seed, std=1.0):
    import torch

    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * std).to(dtype).to(dev)


def _step_fns(q, k, v, do, scale, causal):
    """One fwd + bwd step as the autograd operator runs it: the forward writes O and lse; the dQ kernel forms
    the row term (dO . O, or its exact form on query blocks holding a row flagged peaked in lse) and dQ;
    then the dK/dV kernel reads that row term."""
    import torch

    from theria_amd import _ops

    B, H, S, _ = q.shape
    prob = _ops._problem(q, k, scale, causal)
    delta = torch.empty((B, H, S), dtype=torch.float32, device=q.device)
    dq, dk, dv = (torch.empty_like(q) for _ in range(3))

    def step(ev=None):
        if ev:
            ev[0].record()
        o, lse, _, _ = _ops.fwd(q, k, v, scale, causal)
        if ev:
            ev[1].record()
        _ops.bwd_dq(prob, q, k, v, o, False, do, lse, delta, dq)
        if ev:
            ev[2].record()
        _ops.bwd_dkdv(prob, q, k, v, do, lse, delta, dk, dv)
        if ev:
            ev[3].record()

    return step


def bench_config2(steps: int, warmup: int, warmup_s: float):
    """Timed fwd+bwd steps at config 2; per-kernel HIP-event durations of the three kernels."""
    import torch

    dev = torch.device("cuda:0")
    B, H, S, D = 4, 16, 2048, 64
    dt = torch.bfloat16
    q, k, v, do = (_rand((B, H, S, D), dt, dev, 100 + i) for i in range(4))
    scale = 1.0 / math.sqrt(D)
    step = _step_fns(q, k, v, do, scale, False)

    # W steps, and at least warmup_s seconds: the clocks ramp for the first tens of ms after idle
    t0 = time.perf_counter()
    n = 0
    while n < warmup or time.perf_counter() - t0 < warmup_s:
        step()
        n += 1
        if n % 64 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    warm_s = time.perf_counter() - t0
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps
    # per-kernel durations, measured on the stream the kernels run on (torch's current stream)
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(steps)]
    for e in evs:
        step(e)
    torch.cuda.synchronize()
    fwd_ms = statistics.mean(e[0].elapsed_time(e[1]) for e in evs)
    dq_ms = statistics.mean(e[1].elapsed_time(e[2]) for e in evs)
    dkdv_ms = statistics.mean(e[2].elapsed_time(e[3]) for e in evs)
    unit = B * H * S * S * D
    return dict(
        wall_ms=wall * 1e3, fwd_ms=fwd_ms, dq_ms=dq_ms, dkdv_ms=dkdv_ms, warmup_steps=n, warmup_s=warm_s,
        flop_step=14 * unit, flop_fwd=4 * unit, flop_bwd=10 * unit,
        # algorithmic work of each backward kernel: dq = S, dP, dQ products (6 B H S^2 D);
        # dkdv = S, dP, dV, dK products (8 B H S^2 D); together 14, of which the FA convention counts 10
        flop_dq=6 * unit, flop_dkdv=8 * unit,
        B=B, H=H, S=S, D=D,
    )


def _cpu_threads() -> int:
    """Host threads for the CPU baseline: every core this process may run on (its affinity mask), capped by
    OMP_NUM_THREADS when that is set (a GPU box grants one GPU's share of its cores, whatever
    os.cpu_count() reports for the whole machine)."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    cap = os.environ.get("OMP_NUM_THREADS")
    if cap and cap.isdigit() and int(cap) > 0:
        n = min(n, int(cap))
    return max(1, n)


def cpu_baseline(budget_s: float):
    """The CPU oracle (float32 fwd + bwd, torch on the host cores) on a bounded sample of config-2 heads."""
    import torch

    from oracle import sdpa_oracle as O

    S, D = 2048, 64
    threads = _cpu_threads()
    torch.set_num_threads(threads)
    # the 64 (batch, head) slices of config 2 in turn, over again until the budget is spent
    heads = 0
    t_total = 0.0
    while t_total < budget_s or heads == 0:
        g = torch.Generator().manual_seed(200 + heads % 64)
        q, k, v, do = (torch.randn(1, 1, S, D, generator=g).to(torch.bfloat16).float() for _ in range(4))
        t0 = time.perf_counter()
        O.forward(q, k, v, 1 / 8.0, dtype=torch.float32)
        O.backward(q, k, v, do, 1 / 8.0, dtype=torch.float32)
        t_total += time.perf_counter() - t0
        heads += 1
    flops = 14 * heads * S * S * D
    return {
        "value": round(flops / t_total / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{heads} (batch, head) slices of config 2 (S2048 D64; its 64 slices taken in turn, "
        f"{heads / 64:.1f} passes), fp32 fwd+bwd via the CPU oracle, {t_total:.1f} s; {threads} threads (affinity "
        f"{_affinity()} of os.cpu_count() {os.cpu_count()}, "
        f"OMP_NUM_THREADS={os.environ.get('OMP_NUM_THREADS', 'unset')}); cpu={_cpu_model()}",
    }


def _affinity() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        return -1


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _time(fn, reps: int, warm: int = 3, warm_s: float = 0.25) -> float:
    """Mean ms per call of fn over reps calls, after at least `warm` calls and `warm_s` seconds of warmup."""
    import torch

    t0 = time.perf_counter()
    n = 0
    while n < warm or time.perf_counter() - t0 < warm_s:
        fn()
        n += 1
        if n % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / reps * 1e3


def extras_c2_fp16():
    """Config 2 in float16: the same fwd + dQ + dK/dV step as the headline (which is bfloat16)."""
    import torch

    from theria_amd import _ops

    dev = torch.device("cuda:0")
    B, H, S, D = 4, 16, 2048, 64
    q, k, v, do = (_rand((B, H, S, D), torch.float16, dev, 500 + i) for i in range(4))
    step = _step_fns(q, k, v, do, 1.0 / math.sqrt(D), False)
    ms = _time(step, 30, 5)
    return {"config": "B4 H16 S2048 D64 fp16 fwd+bwd", "ms": round(ms, 4),
            "tflops": round(14 * B * H * S * S * D / (ms * 1e-3) / 1e12, 1)}


def extras_c3():
    """Config 3: B1 H32 S8192 D128 causal bf16 fwd+bwd; FLOPs over the unmasked triangle."""
    import torch

    from theria_amd import _ops

    dev = torch.device("cuda:0")
    B, H, S, D = 1, 32, 8192, 128
    q, k, v = (_rand((B, H, S, D), torch.bfloat16, dev, 300 + i, std=0.5) for i in range(3))
    do = _rand((B, H, S, D), torch.bfloat16, dev, 303)
    scale = 1 / math.sqrt(D)

    run = _step_fns(q, k, v, do, scale, True)
    ms = _time(run, 5, 2)
    useful = 14 * B * H * (S * (S + 1) / 2) * D  # unmasked elements only
    counted = _kernel_tile_counts(q, k, v, do, scale, True)
    n = S // 32
    needed = B * H * n * (n + 1) // 2  # 32 x 32 (query, key) units holding an unmasked element (key <= query)
    total = B * H * n * n
    out = {
        "config": "B1 H32 S8192 D128 causal bf16 fwd+bwd",
        "ms": round(ms, 3),
        "tflops": round(useful / (ms * 1e-3) / 1e12, 1),
        "tile_units": "32 x 32 (query, key) units whose products each kernel ran, counted by the kernels "
                      "(libtheria_sdpa_tiles.so); needed = units holding an unmasked element",
        "tiles_needed": needed,
        "tiles_total": total,
    }
    for name, ex in zip(("fwd", "dq", "dkdv"), counted):
        out[f"tiles_executed_{name}"] = ex
        out[f"tile_skip_efficiency_{name}"] = round(needed / ex, 4) if ex else None
    # unmasked elements over the elements of the executed units
    out["useful_flop_fraction_fwd"] = round(B * H * S * (S + 1) / 2 / (counted[0] * 32 * 32), 4) if counted[0] else None
    return out


def _kernel_tile_counts(q, k, v, do, scale: float, causal: bool):
    """[forward, dQ, dK/dV] executed 32 x 32 tile units of one fwd + bwd step, counted by the kernels themselves in
    the counter-enabled build of the same sources (libtheria_sdpa_tiles.so: THERIA_TILE_COUNT), run through its C
    ABI on the same inputs."""
    import ctypes

    import torch

    from theria_amd import _lib, _ops

    lib = _lib.load(_lib.TILES_LIB_PATH)
    B, H, S, _ = q.shape
    o, dq = torch.empty_like(q), torch.empty_like(q)
    dk, dv = torch.empty_like(k), torch.empty_like(v)
    lse = torch.empty((B, H, S), dtype=torch.float32, device=q.device)
    delta = torch.empty_like(lse)
    prob = _ops._problem(q, k, scale, causal)
    counts = (ctypes.c_uint64 * 3)()

    def ok(rc, what):
        if rc != _lib.OK:
            raise RuntimeError(f"{what}: {lib.theria_last_error().decode(errors='replace')}")

    torch.cuda.synchronize()
    ok(lib.theria_debug_tile_counts(counts, 1), "theria_debug_tile_counts")  # zero them
    st = _ops._stream(q.device)
    tv = _ops._tv
    ok(lib.theria_sdpa_fwd(ctypes.byref(prob), tv(q), tv(k), tv(v), tv(o), 0, lse.data_ptr(), None, None, st),
       "theria_sdpa_fwd (tile counting build)")
    ok(lib.theria_sdpa_bwd_dq(ctypes.byref(prob), tv(q), tv(k), tv(v), tv(o), 0, tv(do), lse.data_ptr(),
                              delta.data_ptr(), tv(dq), st), "theria_sdpa_bwd_dq (tile counting build)")
    ok(lib.theria_sdpa_bwd_dkdv(ctypes.byref(prob), tv(q), tv(k), tv(v), tv(do), lse.data_ptr(), delta.data_ptr(),
                                tv(dk), tv(dv), st), "theria_sdpa_bwd_dkdv (tile counting build)")
    torch.cuda.synchronize()
    ok(lib.theria_debug_tile_counts(counts, 1), "theria_debug_tile_counts")
    return [int(c) for c in counts]


def extras_scores():
    """The partial-fusion score kernels (sdpa_custom backends triton_qk / triton_qk_softmax) at the config-2
    shape: ms and HBM GB/s (Q, K read once, the (B,H,S,S) float32 output written once) against 8 TB/s."""
    import torch

    from theria_amd import _ops

    dev = torch.device("cuda:0")
    B, H, S, D = 4, 16, 2048, 64
    q, k = (_rand((B, H, S, D), torch.bfloat16, dev, 600 + i) for i in range(2))
    out = {"config": "B4 H16 S2048 D64 bf16 in, float32 (B,H,S,S) out", "hbm_peak_gbs": 8000}
    nbytes = 2 * B * H * S * D * 2 + B * H * S * S * 4
    for name, fn in (("qk_scores", lambda: _ops.qk_scores(q, k, out_f32=True)),
                     ("qk_softmax", lambda: _ops.qk_softmax(q, k, 1 / 8.0))):
        ms = _time(fn, 20)
        out[f"{name}_ms"] = round(ms, 4)
        out[f"{name}_gbs"] = round(nbytes / (ms * 1e-3) / 1e9, 1)
    out["bytes_per_call"] = nbytes
    return out


def extras_c4():
    """Config 4: B8 H8 S512 D64; JVP (saved stats) and HVP of 0.5||O - T||^2 (double backward), ms."""
    import torch

    from theria_amd import _ops
    from theria_amd.autograd import GraphedSDPAHVP
    from theria_amd.autograd.hip_sdpa import hip_sdpa, hip_sdpa_hvp

    dev = torch.device("cuda:0")
    B, H, S, D = 8, 8, 512, 64
    out = {}
    for dt, name in ((torch.float32, "fp32"), (torch.bfloat16, "bf16")):
        q, k, v = (_rand((B, H, S, D), dt, dev, 400 + i) for i in range(3))
        tq, tk, tv = (_rand((B, H, S, D), dt, dev, 410 + i, std=0.1) for i in range(3))
        T_ = _rand((B, H, S, D), dt, dev, 420)
        vq, vk, vv = (_rand((B, H, S, D), dt, dev, 430 + i) for i in range(3))
        o, lse, _, _ = _ops.fwd(q, k, v, 1 / 8.0, False)
        # enough calls that the last call's GPU time, not overlapped with host work, does not inflate the mean
        out[f"jvp_ms_{name}"] = round(_time(lambda: _ops.jvp(q, k, v, o, lse, tq, tk, tv, 1 / 8.0, False), 200), 4)
        qg, kg, vg = (t.clone().requires_grad_(True) for t in (q, k, v))

        def hvp():
            # H v = d/dx <grad L, v>: the gradient taken with create_graph, then its vector-Jacobian product with v
            # (grad_outputs), the loss formed in the input dtype as hip_sdpa_hvp forms dO = O - T
            o2 = hip_sdpa(qg, kg, vg)
            loss = 0.5 * ((o2 - T_) ** 2).sum()
            g = torch.autograd.grad(loss, (qg, kg, vg), create_graph=True)
            return torch.autograd.grad(g, (qg, kg, vg), grad_outputs=(vq, vk, vv))

        out[f"hvp_ms_{name}"] = round(_time(hvp, 50), 4)
        # the same autograd HVP captured once in a HIP graph and replayed (no autograd engine on the host)
        graphed = GraphedSDPAHVP(q, k, v, vq, vk, vv, target=T_, scale=1 / 8.0)
        out[f"hvp_graph_ms_{name}"] = round(_time(lambda: graphed(q=q), 200), 4)
        del graphed
        # the same HVP from the kernels directly (forward, double backward, backward of J v; no autograd graph)
        hv = lambda: hip_sdpa_hvp(q, k, v, vq, vk, vv, target=T_, scale=1 / 8.0)  # noqa: E731
        out[f"hvp_kernels_only_ms_{name}"] = round(_time(hv, 100), 4)
        # the double backward forms its own row terms (its delta argument is not read)
        bb = lambda: _ops.bwd_bwd(q, k, v, o, T_, lse, None, vq, vk, vv, 1 / 8.0, False)  # noqa: E731
        out[f"double_backward_kernels_ms_{name}"] = round(_time(bb, 100), 4)
    unit = B * H * S * S * D
    out["jvp_tflops_bf16"] = round(10 * unit / (out["jvp_ms_bf16"] * 1e-3) / 1e12, 1)
    out["config"] = ("B8 H8 S512 D64; JVP with saved stats; HVP of 0.5||O-T||^2 via autograd double backward "
                     "(hvp_ms), the same captured in a HIP graph (hvp_graph_ms) and from the kernels directly "
                     "(hvp_kernels_only_ms)")
    return out


def extras_c5():
    """Config 5: full vs first-order MAML on the 2-layer 4-head classifier, 16 tasks, 5 inner steps."""
    import copy

    import torch

    from theria_amd.maml import meta_loss_on_tasks, meta_loss_on_tasks_batched
    from theria_amd.models import MHAClassifier, MHAConfig
    from theria_amd.tasks import sample_token_count_task

    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    model = MHAClassifier(MHAConfig(), backend="hip").to(dev)
    g = torch.Generator().manual_seed(0)
    tasks = [sample_token_count_task(generator=g, device=dev)[0] for _ in range(16)]
    opt = torch.optim.Adam(model.parameters(), lr=1e-3)

    def meta_step(fo: bool, batched: bool = False):
        opt.zero_grad(set_to_none=True)
        fn = meta_loss_on_tasks_batched if batched else meta_loss_on_tasks
        loss = fn(model, tasks, inner_lr=0.4, inner_steps=5, fo=fo)
        loss.backward()
        opt.step()

    res = {"config": "MHA 2 layers d64 4 heads, token-count task, 16 tasks 5-shot/15-query, 5 inner SGD @0.4, Adam 1e-3"}
    for fo in (False, True):
        ms = _time(lambda: meta_step(fo), 3, 1)
        res[f"meta_steps_per_s_{'fo' if fo else 'full'}"] = round(1e3 / ms, 3)
    # the same meta-step with all 16 tasks adapted in one batched forward/backward per inner step
    for fo in (False, True):
        ms = _time(lambda: meta_step(fo, batched=True), 10, 2)
        res[f"meta_steps_per_s_{'fo' if fo else 'full'}_task_batched"] = round(1e3 / ms, 3)
    # ... and that step captured once in a HIP graph and replayed (Adam with its state on the device)
    from theria_amd.maml import GraphedMetaStep

    for fo in (False, True):
        gm = copy.deepcopy(model)
        gopt = torch.optim.Adam(gm.parameters(), lr=1e-3, capturable=True)
        graphed = GraphedMetaStep(gm, gopt, tasks, inner_lr=0.4, inner_steps=5, fo=fo)
        ms = _time(lambda: graphed.step(), 20, 3)
        res[f"meta_steps_per_s_{'fo' if fo else 'full'}_task_batched_graph"] = round(1e3 / ms, 3)
        del graphed, gopt, gm
    # meta-gradient agreement with the same weights on the pure-PyTorch reference backend
    ref = copy.deepcopy(model)
    ref.set_attention_backend("reference")
    params_h = list(model.parameters())
    params_r = list(ref.parameters())
    gh = torch.autograd.grad(meta_loss_on_tasks(model, tasks, inner_lr=0.4, inner_steps=5), params_h)
    gr = torch.autograd.grad(meta_loss_on_tasks(ref, tasks, inner_lr=0.4, inner_steps=5), params_r)
    fh = torch.cat([x.flatten() for x in gh]).double()
    fr = torch.cat([x.flatten() for x in gr]).double()
    res["metagrad_rel_l2_vs_reference"] = float((fh - fr).norm() / fr.norm())
    res["metagrad_cosine_vs_reference"] = float(torch.nn.functional.cosine_similarity(fh, fr, dim=0))
    gb = torch.autograd.grad(meta_loss_on_tasks_batched(model, tasks, inner_lr=0.4, inner_steps=5), params_h)
    fb = torch.cat([x.flatten() for x in gb]).double()
    res["metagrad_rel_l2_task_batched_vs_reference"] = float((fb - fr).norm() / fr.norm())
    return res


def copy_calibration():
    """A plain device copy of 256 MiB (FETCH_SIZE / WRITE_SIZE calibration for rocprofv3 --pmc)."""
    import torch

    src = torch.ones(64 * 1024 * 1024, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_each_way": src.numel() * 4, "launches": 5}), flush=True)


def atomic_probe():
    """Float32 atomic-add throughput in the pattern a backward forming dQ inside the dK/dV kernel needs: every
    key block adds its partial dQ (config 2: B4 H16 S2048 D64, 33.5 MB in float32) once, so 2048 / 256 = 8 adds
    per element with eight-wave key blocks (16 with four-wave blocks). Runs theria_debug_atomic_probe from the
    counter-enabled build; the same pattern as plain stores for scale. One JSON line."""
    import ctypes

    import torch

    from theria_amd import _lib

    lib = _lib.load(_lib.TILES_LIB_PATH)
    dev = torch.device("cuda:0")
    n = 4 * 16 * 2048 * 64
    buf = torch.zeros(n, dtype=torch.float32, device=dev)
    st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    out = {"probe": "float32 atomic adds, config-2 dQ (B4 H16 S2048 D64)", "buffer_bytes": n * 4}
    for reps in (8, 16):
        for atomic in (1, 0):
            def go():
                rc = lib.theria_debug_atomic_probe(ctypes.c_void_p(buf.data_ptr()), n, reps, atomic, st)
                if rc != _lib.OK:
                    raise RuntimeError(lib.theria_last_error().decode(errors="replace"))
            ms = _time(go, 20)
            key = f"{'atomic' if atomic else 'store'}_x{reps}"
            out[f"{key}_us"] = round(ms * 1e3, 1)
            out[f"{key}_TBps"] = round(n * 4 * reps / (ms * 1e-3) / 1e12, 2)
    print(json.dumps(out), flush=True)


def main() -> int:
    args = _args()
    if args.gpus != 1:
        print(
            f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported (SDPA shards over "
            "batch x heads with no exchange, so the per-GPU figure is the one-GPU run).",
            file=sys.stderr,
        )
        return 2
    import torch

    if not torch.cuda.is_available():
        print("bench.py: no HIP device visible", file=sys.stderr)
        return 1
    from theria_amd import _lib

    _lib.load()
    if args.copy_calibration:
        copy_calibration()
        return 0
    if args.atomic_probe:
        atomic_probe()
        return 0
    r = bench_config2(args.steps, args.warmup, args.warmup_seconds)
    value = r["flop_step"] / (r["wall_ms"] * 1e-3) / 1e12
    achieved = r["flop_dkdv"] / (r["dkdv_ms"] * 1e-3) / 1e12
    traffic = None
    if TRAFFIC_FILE.exists():
        try:
            traffic = json.loads(TRAFFIC_FILE.read_text()).get("dkdv_bytes_per_launch")
        except (OSError, ValueError):
            traffic = None
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_steps_run": r["warmup_steps"],
        "warmup_s": round(r["warmup_s"], 3),
        "ms_per_step": round(r["wall_ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "sdpa_fwd_bwd", "batch": 4, "heads": 16, "seq_len": 2048, "head_dim": 64, "causal": False},
        "mfma_peak_frac": round(value / PEAK_BF16_TFLOPS, 4),
        "roofline": {
            "kernel": "dkdv_pipe_kernel<bf16, non-causal, 8 waves> (theria_sdpa_bwd_dkdv)",
            "bound": "mfma",
            "achieved": round(achieved, 2),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
            "traffic": traffic,
            "flop_per_launch": r["flop_dkdv"],
            "avg_launch_ms": round(r["dkdv_ms"], 4),
        },
        "kernels_ms": {
            "fwd": round(r["fwd_ms"], 4),
            "bwd_dq": round(r["dq_ms"], 4),
            "bwd_dkdv": round(r["dkdv_ms"], 4),
        },
        "fwd_tflops": round(r["flop_fwd"] / (r["fwd_ms"] * 1e-3) / 1e12, 1),
        "bwd_tflops": round(r["flop_bwd"] / ((r["dq_ms"] + r["dkdv_ms"]) * 1e-3) / 1e12, 1),
        "dq_kernel_tflops": round(r["flop_dq"] / (r["dq_ms"] * 1e-3) / 1e12, 1),
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    if not args.no_extras:
        extra = {}
        wanted = {x.strip() for x in args.extras.split(",") if x.strip()}
        for name, fn in (("c2_fp16", extras_c2_fp16), ("c3", extras_c3), ("c4", extras_c4), ("c5", extras_c5),
                         ("scores", extras_scores)):
            if name not in wanted:
                continue
            try:
                extra[name] = fn()
            except Exception as exc:  # an extra must not hide the headline line
                extra[name] = {"error": f"{type(exc).__name__}: {exc}"}
        line["extra"] = extra
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
