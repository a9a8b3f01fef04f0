"""Random parity sweep over every entry point: the GPU library against the float64 oracle (not a pytest module).

Usage, on a GPU host from the repository root:

    python tests/parity_sweep.py N SEED BUDGET_S

draws N cases from random.Random(SEED) (dtype, batch, heads, T, M, head dim, causal), runs case i on inputs
seeded with 1000 + i through the same checks as tests/test_gpu_parity.py (first and second order, every
entry point), stops once BUDGET_S seconds have passed, and prints the failures. The few-key cases committed
in tests/test_gpu_precision.py (FEW_KEY_SWEEP, seed 1000 + i) came from the runs with SEED 7, 8 and 9.
"""

import argparse
import random
import sys
import time
from pathlib import Path

import torch

sys.path.insert(0, str(Path(__file__).resolve().parent))
from test_gpu_parity import _check_all_entry_points, _ids  # noqa: E402

DTYPES = [torch.float32, torch.float16, torch.bfloat16, torch.bfloat16]
HEAD_DIMS = [8, 16, 24, 32, 40, 48, 56, 64, 64, 72, 80, 88, 96, 104, 112, 120, 128, 128]
BATCH_HEADS = [(1, 1), (1, 2), (2, 1), (2, 2), (1, 3)]


def draw(rng: random.Random):
    """One case (dtype, B, H, T, M, D, causal); the draw order fixes which case a seed gives."""
    dt = rng.choice(DTYPES)
    D = rng.choice(HEAD_DIMS)
    T = rng.choice([rng.randint(1, 130), rng.randint(129, 900), rng.randint(129, 900)])
    M = rng.choice([T, rng.randint(1, 200), rng.randint(100, 900)])
    B, H = rng.choice(BATCH_HEADS)
    return (dt, B, H, T, M, D, rng.random() < 0.5)


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("n", type=int)
    ap.add_argument("seed", type=int)
    ap.add_argument("budget", type=float, help="seconds")
    a = ap.parse_args()
    rng = random.Random(a.seed)
    dev = torch.device("cuda:0")
    fails, t0, done = [], time.time(), 0
    for i in range(a.n):
        case = draw(rng)
        print(f"[{i}] {_ids(case)} seed {1000 + i}", flush=True)
        try:
            _check_all_entry_points(case, dev, seed=1000 + i)
        except AssertionError as e:
            fails.append((case, i, " | ".join(str(e).split("\n")[:6])))
            print("   FAIL", fails[-1][2][:400], flush=True)
        done += 1
        if time.time() - t0 > a.budget:
            break
    print(f"done {done} cases, {len(fails)} failures, {time.time() - t0:.0f}s")
    for case, i, msg in fails:
        print("FAIL", _ids(case), f"seed {1000 + i}", msg[:300])


if __name__ == "__main__":
    main()
