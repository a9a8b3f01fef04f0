"""Torch-level wrappers over the C ABI: shape/dtype/device guards, output allocation, stream plumbing.

Each function validates its arguments the way the reference's guards do (AssertionError with a
message, theria/attention/triton_sdpa_backward.py:23-103), allocates fresh outputs on the inputs'
device (the reference's ownership rule, triton_qk.py:321-323) and launches on torch's current stream
of that device. Inputs are never mutated.
"""

from __future__ import annotations

import ctypes
import math

import torch

from . import _lib

ALLOWED_DTYPES = (torch.float16, torch.bfloat16, torch.float32)
_DTYPE_CODE = {torch.float32: _lib.DTYPE_F32, torch.float16: _lib.DTYPE_F16, torch.bfloat16: _lib.DTYPE_BF16}
MAX_HEAD_DIM = 128


def default_scale(head_dim: int) -> float:
    return 1.0 / math.sqrt(head_dim)


def _rowmajor(t: torch.Tensor | None) -> torch.Tensor | None:
    """The kernels need a contiguous last dimension; other strides (incl. broadcast) are fine."""
    if t is None:
        return None
    if t.shape[-1] > 1 and t.stride(-1) != 1:
        return t.contiguous()
    return t


_functorch = None


def _plain(t: torch.Tensor) -> torch.Tensor:
    """Underlying tensor of a torch.func (functorch) wrapper, whose storage the kernels read.

    torch.func.jvp calls SDPAOp.jvp with its saved tensors wrapped for gradient tracking; the values
    are those of the wrapped tensor.
    """
    global _functorch
    if _functorch is None:
        from torch._C import _functorch as ft

        _functorch = (ft.is_functorch_wrapped_tensor, ft.get_unwrapped)
    is_wrapped, unwrap = _functorch
    while is_wrapped(t):
        t = unwrap(t)
    return t


def _tv(t: torch.Tensor | None):
    """theria_tensor_t of a (B,H,rows,D) tensor (ctypes passes it by reference), or NULL."""
    if t is None:
        return None
    t = _plain(t)
    return _lib.TensorView(t.data_ptr(), t.stride(0), t.stride(1), t.stride(2))


def _fp(t: torch.Tensor | None):
    return None if t is None else _plain(t).data_ptr()


def _stream(dev: torch.device):
    """Raw hipStream_t of torch's current stream on `dev`."""
    return torch._C._cuda_getCurrentRawStream(dev.index if dev.index is not None else torch.cuda.current_device())


class _OnDevice:
    """Make `dev` the current device for the duration of a launch (a no-op when it already is)."""

    __slots__ = ("idx", "prev")

    def __init__(self, dev: torch.device):
        self.idx = dev.index if dev.index is not None else torch.cuda.current_device()
        self.prev = None

    def __enter__(self):
        cur = torch.cuda.current_device()
        if cur != self.idx:
            self.prev = cur
            torch.cuda.set_device(self.idx)

    def __exit__(self, *exc):
        if self.prev is not None:
            torch.cuda.set_device(self.prev)
        return False


_HOST = None


def _host():
    """The torch binding of the hot entry points (theria_amd/csrc/host/theria_host.cpp), loaded once after the
    C ABI library. There is no fallback: a missing binding raises, as a missing library does."""
    global _HOST
    if _HOST is None:
        _lib.load()
        try:
            from . import _theria_host as host
        except ImportError as e:
            raise RuntimeError("theria_amd: the torch binding _theria_host is not built. Run `python -m "
                               "theria_amd.build` (needs hipcc and g++) before using the HIP SDPA operators.") from e
        if host.abi_version() != _lib.ABI_VERSION:
            raise RuntimeError(f"theria_amd: _theria_host is linked to ABI {host.abi_version()}, expected "
                               f"{_lib.ABI_VERSION}; rebuild it")
        _HOST = host
    return _HOST


def _problem(q: torch.Tensor, k: torch.Tensor, scale: float, causal: bool) -> _lib.Problem:
    B, H, T, D = q.shape
    return _lib.Problem(_DTYPE_CODE[q.dtype], B, H, T, k.shape[2], D, float(scale), 1 if causal else 0)


def check_inputs(q, k, v, what: str = "theria_amd SDPA", require_v: bool = True) -> None:
    """Device, dtype and shape contract shared by every HIP entry point."""
    for name, t in (("q", q), ("k", k), ("v", v) if require_v else (None, None)):
        if name is None:
            continue
        if t is None:
            raise AssertionError(f"{what}: {name} is required")
        if not t.is_cuda:
            raise AssertionError(f"{what} requires GPU (HIP) tensors; {name} is on {t.device}")
        if t.dtype not in ALLOWED_DTYPES:
            raise AssertionError(f"Unsupported dtype for {name}: {t.dtype}")
        if t.dim() != 4:
            raise AssertionError(f"{what}: {name} must be 4-D (B,H,rows,D), got shape {tuple(t.shape)}")
    B, H, T, D = q.shape
    if k.shape[0] != B or k.shape[1] != H or k.shape[3] != D:
        raise AssertionError("k must have shape (B,H,M,D) with D matching q")
    if k.dtype != q.dtype:
        raise AssertionError(f"{what}: k dtype {k.dtype} != q dtype {q.dtype}")
    if k.device != q.device:
        raise AssertionError(f"{what}: q and k are on different devices")
    if require_v:
        if v.shape[0] != B or v.shape[1] != H or v.shape[2] != k.shape[2]:
            raise AssertionError("v must have shape (B,H,M,Dv) matching k")
        if v.shape[3] != D:
            raise AssertionError("theria_amd SDPA requires Dv == D")
        if v.dtype != q.dtype or v.device != q.device:
            raise AssertionError(f"{what}: v must match q in dtype and device")
    if D > MAX_HEAD_DIM or D < 1:
        raise AssertionError(f"{what} supports 1 <= D <= {MAX_HEAD_DIM}, got D={D}")
    if max(q.shape[2], k.shape[2]) >= 2**31 or B * H >= 2**31:
        raise AssertionError(f"{what}: sizes exceed the 32-bit row index range")


def _like_rows(t: torch.Tensor | None, ref: torch.Tensor, rows: int, name: str) -> torch.Tensor | None:
    """Cast a (B,H,rows,D) operand to the compute dtype and check its shape."""
    if t is None:
        return None
    B, H, _, D = ref.shape
    if tuple(t.shape) != (B, H, rows, D):
        raise AssertionError(f"{name} must have shape {(B, H, rows, D)}, got {tuple(t.shape)}")
    if not t.is_cuda or t.device != ref.device:
        raise AssertionError(f"{name} must be on {ref.device}")
    if t.dtype != ref.dtype:
        t = t.to(ref.dtype)
    return _rowmajor(t)


def fwd(q, k, v, scale: float, causal: bool, out_fp32: bool = False, stats: bool = False, checked: bool = True):
    """O, lse (and the reference's m, l when stats=True). O is float32 when out_fp32. With 16-bit inputs the
    lowest mantissa bit of lse flags the peaked rows (largest probability above 1/4), which the backward
    takes on its exact path. checked=False skips the Python-side input checks (for callers that made them);
    shapes are still checked by the binding and the C ABI."""
    if checked:
        check_inputs(q, k, v)
    return _host().fwd(q, k, v, float(scale), bool(causal), bool(out_fp32), bool(stats))


def lse_from_stats(m, l, peaked_bits: bool = True):
    """lse = m + log(l) (float32) from the reference's saved statistics, with the peaked-row flag of the
    16-bit backward in its lowest mantissa bit: a row is peaked when its largest probability 1 / l exceeds
    1/4, i.e. l < 4. Infinite entries (rows without visible keys) are left as they are."""
    lse = (m.float() + torch.log(l.float())).contiguous()
    if peaked_bits:
        bits = lse.view(torch.int32)
        flagged = (bits & ~1) | (l.float() < 4.0).to(torch.int32)
        lse = torch.where(torch.isfinite(lse), flagged, bits).view(torch.float32)
    return lse


def bwd(q, k, v, o, lse, do, scale: float, causal: bool, need_dq: bool = True, need_dk: bool = True, out=None,
        checked: bool = True):
    """dQ, dK, dV (input dtype) and the row term delta (float32: dO . O for 16-bit inputs, formed exactly on query
    blocks that hold a row flagged peaked in lse; sum_j P dP / sum_j P for float32). out: (dq, dk, dv) tensors to
    write instead of new ones. checked=False skips the Python-side input checks."""
    if checked:
        check_inputs(q, k, v)
    return _host().bwd(q, k, v, o, lse, do, float(scale), bool(causal), bool(need_dq), bool(need_dk),
                       None if out is None else list(out))


# The two backward kernels (theria_sdpa_bwd = bwd_dq then bwd_dkdv), on the current stream of the
# current device. Arguments are already validated and laid out by bwd().
def bwd_dq(prob, q, k, v, o, o_f32, do, lse, delta, dq) -> None:
    """dQ; with o given, the row term delta is computed and written, else it is read."""
    rc = _lib.load().theria_sdpa_bwd_dq(
        ctypes.byref(prob), _tv(q), _tv(k), _tv(v), _tv(o), 1 if o_f32 else 0, _tv(do), _fp(lse), _fp(delta),
        _tv(dq), _stream(q.device),
    )
    _lib.check(rc, "theria_sdpa_bwd_dq")


def bwd_dkdv(prob, q, k, v, do, lse, delta, dk, dv) -> None:
    rc = _lib.load().theria_sdpa_bwd_dkdv(
        ctypes.byref(prob), _tv(q), _tv(k), _tv(v), _tv(do), _fp(lse), _fp(delta), _tv(dk), _tv(dv),
        _stream(q.device),
    )
    _lib.check(rc, "theria_sdpa_bwd_dkdv")


def bwd_from_stats(q, k, v, do, lse, scale: float, causal: bool, need_dq: bool, need_dk: bool, need_dv: bool,
                   normalize: bool = False):
    """Backward from saved statistics only (no O). v may be None when only dV is requested. lse carries the
    peaked-row flags as in bwd (lse_from_stats sets them from the reference's m, l).

    normalize=False: the reference's frozen-stats backward (P = exp(S - lse) as given, row term
    sum_j P_ij dP_ij). normalize=True: the row term of the normalised P, i.e. the exact softmax gradient, for
    the operator's own lse."""
    check_inputs(q, k, v, require_v=v is not None)
    q, k = _rowmajor(q), _rowmajor(k)
    v = _rowmajor(v)
    B, H, T, D = q.shape
    M = k.shape[2]
    do = _like_rows(do, q, T, "dout")
    lse = lse.contiguous()
    dev = q.device
    delta = torch.empty((B, H, T), dtype=torch.float32, device=dev) if v is not None else None
    dq = torch.empty((B, H, T, D), dtype=q.dtype, device=dev) if need_dq else None
    dk = torch.empty((B, H, M, D), dtype=q.dtype, device=dev) if need_dk else None
    dv = torch.empty((B, H, M, D), dtype=q.dtype, device=dev)
    lib = _lib.load()
    prob = _problem(q, k, scale, causal)
    with _OnDevice(dev):
        rc = lib.theria_sdpa_bwd_from_stats(
            ctypes.byref(prob), _tv(q), _tv(k), _tv(v), _tv(do), _fp(lse), _fp(delta), _tv(dq), _tv(dk),
            _tv(dv), 1 if normalize else 0, _stream(dev),
        )
    _lib.check(rc, "theria_sdpa_bwd_from_stats")
    return dq, dk, (dv if need_dv else None)


def jvp(q, k, v, o, lse, tq, tk, tv, scale: float, causal: bool, normalize: bool = True, checked: bool = True):
    """Tangent of O along (tq, tk, tv) with P rebuilt from lse; o=None rebuilds O inside the kernel.

    normalize=True: the JVP of the exact softmax (P divided by its row sum), for the operator's own lse.
    normalize=False: the reference's frozen-stats JVP, P = exp(S - lse) held as given (o is then not read).
    checked=False skips the Python-side input checks."""
    if checked:
        check_inputs(q, k, v)
    return _host().jvp(q, k, v, o, lse, tq, tk, tv, float(scale), bool(causal), bool(normalize))


def bwd_bwd(q, k, v, o, do, lse, delta, gq, gk, gv, scale: float, causal: bool, noalloc: bool = False, out=None,
            checked: bool = True):
    """(G_Q, G_K, G_V, G_dO): VJP of the backward map with cotangents (gq, gk, gv) (None = zero).
    delta (the backward's row term) is not read: the library recomputes the row term; it may be None.

    noalloc: run theria_sdpa_bwd_bwd_noalloc, whose row workspace is the library's static device array
    (5 * B * H * T up to 5 * 2^20), instead of a workspace allocated here. out: (G_Q, G_K, G_V) written to the
    given tensors. checked=False skips the Python-side input checks."""
    if checked:
        check_inputs(q, k, v)
    return _host().bwd_bwd(q, k, v, o, do, lse, gq, gk, gv, float(scale), bool(causal), bool(noalloc),
                           None if out is None else list(out))


def qk_scores(q, k, out_f32: bool = True):
    """Unscaled scores Q K^T (B,H,T,M): float32, or the input dtype when out_f32 is False."""
    check_inputs(q, k, None, require_v=False)
    q, k = _rowmajor(q), _rowmajor(k)
    B, H, T, _ = q.shape
    M = k.shape[2]
    f32 = out_f32 or q.dtype == torch.float32
    dev = q.device
    out = torch.empty((B, H, T, M), dtype=torch.float32 if f32 else q.dtype, device=dev)
    prob = _problem(q, k, 1.0, False)
    with _OnDevice(dev):
        rc = _lib.load().theria_qk_scores(ctypes.byref(prob), _tv(q), _tv(k), out.data_ptr(), 1 if f32 else 0, _stream(dev))
    _lib.check(rc, "theria_qk_scores")
    return out


def qk_softmax(q, k, scale: float):
    """Probabilities softmax(scale Q K^T) over the keys, float32 (B,H,T,M)."""
    check_inputs(q, k, None, require_v=False)
    q, k = _rowmajor(q), _rowmajor(k)
    B, H, T, _ = q.shape
    M = k.shape[2]
    dev = q.device
    out = torch.empty((B, H, T, M), dtype=torch.float32, device=dev)
    prob = _problem(q, k, scale, False)
    with _OnDevice(dev):
        rc = _lib.load().theria_qk_softmax(ctypes.byref(prob), _tv(q), _tv(k), out.data_ptr(), _stream(dev))
    _lib.check(rc, "theria_qk_softmax")
    return out
