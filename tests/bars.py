"""Parity bars of the GPU tests, and a record of how close each test family comes to them.

float32: 1e-5 absolute + 1e-5 relative (the north star's float32 bar).
float16 / bfloat16 outputs: 2e-2 absolute (the north star's 16-bit bar) plus one rounding unit of the output
dtype relative (2^-8 for bfloat16, 2^-11 for float16): an output rounded to nearest is off by half a unit of
the dtype, i.e. up to 2^-9 (bfloat16) or 2^-12 (float16) of its value, which for |x| > 10 alone exceeds 2e-2.
The relative term is twice that rounding, so the computation itself must stay within the absolute bar and one
half-unit. (theria's own GPU tests use rtol = atol = 2e-2, tests/test_triton_sdpa_dq.py:42 in the reference.)

Every comparison made through `close` records err / bar (the largest over the tensor) under its test family (the
test function's name); pytest's terminal summary prints the worst ratio per family (tests/conftest.py), and with
THERIA_MARGIN_LOG set it also writes them there as JSON.
"""

from __future__ import annotations

import os

import torch

ROUND_UNIT = {torch.bfloat16: 2.0**-8, torch.float16: 2.0**-11}
MARGINS: dict[str, tuple[float, str]] = {}


def tol(dtype) -> dict:
    if dtype == torch.float32:
        return dict(rtol=1e-5, atol=1e-5)
    return dict(rtol=ROUND_UNIT[dtype], atol=2e-2)


def family() -> str:
    cur = os.environ.get("PYTEST_CURRENT_TEST", "?")
    name = cur.split("::")[-1].split(" ")[0]
    return name.split("[")[0]


def record(a: torch.Tensor, b: torch.Tensor, rtol: float, atol: float, what: str) -> None:
    """Largest |a - b| / (atol + rtol |b|) of the comparison, kept when it is the family's worst so far."""
    if a.numel() == 0:
        return
    ratio = float(((a - b).abs() / (atol + rtol * b.abs())).max())
    fam = family()
    if fam not in MARGINS or ratio > MARGINS[fam][0]:
        MARGINS[fam] = (ratio, f"{what} ({os.environ.get('PYTEST_CURRENT_TEST', '?').split('::')[-1].split(' ')[0]})")


def close(gpu: torch.Tensor, ref: torch.Tensor, rtol: float, atol: float, what: str) -> None:
    """assert_close of a device result against a CPU float64 reference, with the ratio recorded."""
    a = gpu.detach().double().cpu()
    b = ref.double()
    assert a.shape == b.shape, f"{what}: shape {tuple(a.shape)} vs {tuple(b.shape)}"
    assert torch.isfinite(a).all(), f"{what}: non-finite output"
    record(a, b, rtol, atol, what)
    torch.testing.assert_close(a, b, rtol=rtol, atol=atol, msg=lambda m: f"{what}: {m}")
