"""The C ABI library loads and exports exactly what include/theria_sdpa.h declares (no GPU needed).

Also checks the host-side contract validation of every entry point (it runs before any HIP call, so
no device is touched), and that the Python bindings and the header agree on struct layouts.
"""

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "theria_sdpa.h"


def _declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(theria_[a-z_]+)\s*\(", text)))


@pytest.mark.parametrize("which", ["production", "tile counting"])
def test_library_exports_every_declared_symbol(which):
    """Both builds (libtheria_sdpa.so and the counter-enabled libtheria_sdpa_tiles.so) export exactly the header."""
    from theria_amd import _lib

    path = _lib.LIB_PATH if which == "production" else _lib.TILES_LIB_PATH
    lib = _lib.load(path)
    declared = _declared_functions()
    assert declared, "no declarations parsed from the header"
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in {HEADER.name} but not exported"
    assert set(declared) == set(_lib.SIGNATURES), "ctypes signature table out of sync with the header"
    nm = subprocess.run(["nm", "-D", "--defined-only", str(path)], capture_output=True, text=True, check=True)
    exported = sorted(set(re.findall(r"\sT\s(theria_\w+)", nm.stdout)))
    assert exported == declared, f"exported {exported} != declared {declared}"
    # Nothing else: exported kernel stubs (weak template symbols) would bind to another copy of the
    # library loaded into the same process, which would then launch kernels of a different build.
    others = [ln.split()[-1] for ln in nm.stdout.splitlines() if ln.split() and not ln.split()[-1].startswith("theria_")]
    assert not others, f"symbols beyond the C ABI are exported: {others[:5]} ..."


def test_abi_version_matches():
    from theria_amd import _lib

    assert _lib.load().theria_abi_version() == _lib.ABI_VERSION


def test_struct_layouts_match_header():
    from theria_amd import _lib

    assert ctypes.sizeof(_lib.TensorView) == 32
    assert ctypes.sizeof(_lib.Problem) == 32


def _call_all(prob):
    """Call every compute entry point with the given problem and NULL tensors; return status codes."""
    from theria_amd import _lib

    lib = _lib.load()
    p = ctypes.byref(prob)
    return {
        "fwd": lib.theria_sdpa_fwd(p, None, None, None, None, 0, None, None, None, None),
        "bwd": lib.theria_sdpa_bwd(p, None, None, None, None, 0, None, None, None, None, None, None, None),
        "bwd_dq": lib.theria_sdpa_bwd_dq(p, None, None, None, None, 0, None, None, None, None, None),
        "bwd_dkdv": lib.theria_sdpa_bwd_dkdv(p, None, None, None, None, None, None, None, None, None),
        "bwd_from_stats": lib.theria_sdpa_bwd_from_stats(p, None, None, None, None, None, None, None, None, None, 0, None),
        "jvp": lib.theria_sdpa_jvp(p, None, None, None, None, None, None, None, None, None, 1, None),
        "bwd_bwd": lib.theria_sdpa_bwd_bwd(
            p, None, None, None, None, None, None, None, None, None, None, None, None, None, None, None, None
        ),
        "bwd_bwd_noalloc": lib.theria_sdpa_bwd_bwd_noalloc(
            p, None, None, None, None, None, None, None, None, None, None, None, None, None, None, None
        ),
        "qk_scores": lib.theria_qk_scores(p, None, None, None, 1, None),
        "qk_softmax": lib.theria_qk_softmax(p, None, None, None, None),
    }


@pytest.mark.parametrize(
    "fields,needle",
    [
        ((9, 1, 1, 4, 4, 8, 0.5, 0), "dtype"),
        ((2, 1, 1, 4, 4, 200, 0.5, 0), "head_dim"),
        ((2, 1, 1, 4, 4, 8, -1.0, 0), "scale"),
        ((2, -1, 1, 4, 4, 8, 0.5, 0), "negative"),
        ((2, 1, 1, 4, 4, 8, 0.5, 0), "required"),
    ],
)
def test_contract_violations_are_reported(fields, needle):
    from theria_amd import _lib

    codes = _call_all(_lib.Problem(*fields))
    lib = _lib.load()
    for name, rc in codes.items():
        assert rc == _lib.ERR_CONTRACT, f"{name} returned {rc}"
    assert needle in lib.theria_last_error().decode()


def test_python_check_maps_contract_errors_to_assertion():
    from theria_amd import _lib

    codes = _call_all(_lib.Problem(9, 1, 1, 4, 4, 8, 0.5, 0))
    with pytest.raises(AssertionError):
        _lib.check(codes["fwd"], "theria_sdpa_fwd")


def test_score_kernels_reject_causal():
    from theria_amd import _lib

    lib = _lib.load()
    prob = _lib.Problem(2, 1, 1, 4, 4, 8, 0.5, 1)
    assert lib.theria_qk_scores(ctypes.byref(prob), None, None, None, 1, None) == _lib.ERR_CONTRACT
    assert "causal" in lib.theria_last_error().decode()
    assert lib.theria_qk_softmax(ctypes.byref(prob), None, None, None, None) == _lib.ERR_CONTRACT


def test_torch_binding_loads_and_matches_the_abi():
    """The tensor-level binding of the hot entry points (theria_amd/_theria_host) imports without a GPU and is
    linked to the library of this ABI version."""
    from theria_amd import _lib, _ops

    host = _ops._host()
    assert host.abi_version() == _lib.ABI_VERSION
    for name in ("fwd", "bwd", "jvp", "bwd_bwd"):
        assert callable(getattr(host, name))


def test_production_library_has_no_tile_counters():
    """theria_debug_tile_counts answers only in the counter-enabled build; the production library refuses it before
    any HIP call."""
    from theria_amd import _lib

    counts = (ctypes.c_uint64 * 3)(7, 7, 7)
    assert _lib.load().theria_debug_tile_counts(counts, 0) == _lib.ERR_CONTRACT
    assert list(counts) == [0, 0, 0]
    assert b"without tile counters" in _lib.load().theria_last_error()


def test_production_library_has_no_atomic_probe():
    """theria_debug_atomic_probe runs only in the counter-enabled build; the production library refuses it before any
    HIP call (the buffer pointer is never dereferenced on the host)."""
    from theria_amd import _lib

    fake = ctypes.c_void_p(0x1000)
    assert _lib.load().theria_debug_atomic_probe(fake, 8192, 1, 1, None) == _lib.ERR_CONTRACT
    assert b"without the measurement kernels" in _lib.load().theria_last_error()
    assert _lib.load().theria_debug_atomic_probe(None, 8192, 1, 1, None) == _lib.ERR_CONTRACT
