"""Build libtheria_sdpa.so (the gfx950 HIP kernels + C ABI) and its torch binding in-tree.

Usage: ``python -m theria_amd.build`` (or ``theria_amd.build.build()``). Every ``csrc/*.hip`` file is
compiled for gfx950 in parallel into ``_build/`` at the repository root and linked into
``theria_amd/lib/libtheria_sdpa.so``; a second time with ``THERIA_TILE_COUNT`` into ``libtheria_sdpa_tiles.so``
(kernels that count the tiles they run, for measurements only). ``csrc/host/theria_host.cpp`` (host code only, g++) is compiled beside
them and linked against that library into the Python module ``theria_amd/_theria_host*.so``, the tensor-level
binding of the hot entry points that the autograd operator calls. The library links against the HIP runtime by its soname
(libamdhip64.so.7), so inside a process that already imported torch it binds to the runtime torch
loaded: one HIP runtime per process. Only the C ABI (``theria_*``) is exported: the host stubs of the
kernel templates are weak symbols, and exported they would bind to another copy of this library loaded
into the same process (an older build, say), whose launches would then run these kernels with that
build's parameter structs.
"""

from __future__ import annotations

import concurrent.futures as _cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
LIB_DIR = PKG_DIR / "lib"
LIB_PATH = LIB_DIR / "libtheria_sdpa.so"
# The same sources compiled with THERIA_TILE_COUNT: kernels that count the tiles they run (measurement only).
TILES_LIB_PATH = LIB_DIR / "libtheria_sdpa_tiles.so"
BUILD_DIR = REPO_DIR / "_build"

ARCH = "gfx950"
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-mcode-object-version=5",
    # Packed float32 VALU ops (v_pk_fma_f32 and friends) are kept out of the generated code.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    f"-I{REPO_DIR / 'include'}",
]


# Linker version script: export the C ABI, keep every other symbol local to the library.
EXPORTS = "{\n  global: theria_*;\n  local: *;\n};\n"


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the HIP toolchain is required to build libtheria_sdpa.so")


def _compile(hipcc: str, src: Path, tiles: bool = False) -> Path:
    obj = (BUILD_DIR / "tiles" if tiles else BUILD_DIR) / (src.stem + ".o")
    cmd = [hipcc, *COMMON_FLAGS, *(["-DTHERIA_TILE_COUNT"] if tiles else []), "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{res.stdout}")
    return obj


HOST_SRC = CSRC / "host" / "theria_host.cpp"


def host_module_path() -> Path:
    import sysconfig

    return PKG_DIR / ("_theria_host" + sysconfig.get_config_var("EXT_SUFFIX"))


def _torch_dirs():
    import torch

    root = Path(torch.__file__).resolve().parent
    return root / "include", root / "lib", int(torch._C._GLIBCXX_USE_CXX11_ABI)


def _compile_host() -> Path:
    """The torch binding's object (host C++ only: torch, c10/hip and HIP runtime headers)."""
    import sysconfig

    inc, _, abi = _torch_dirs()
    obj = BUILD_DIR / "theria_host.o"
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-fvisibility=hidden", "-D__HIP_PLATFORM_AMD__",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}", f"-I{inc}", f"-I{inc / 'torch' / 'csrc' / 'api' / 'include'}",
           "-I/opt/rocm/include", f"-I{REPO_DIR / 'include'}", f"-I{sysconfig.get_paths()['include']}",
           "-c", str(HOST_SRC), "-o", str(obj)]
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{res.stdout}")
    return obj


def _link_host(obj: Path) -> Path:
    """Link the binding against libtheria_sdpa.so (found next to it through an $ORIGIN/lib run path)."""
    _, lib, _ = _torch_dirs()
    out = host_module_path()
    tmp = out.with_suffix(".tmp")
    cmd = ["g++", "-shared", "-fPIC", str(obj), "-o", str(tmp), f"-L{lib}", "-lc10", "-lc10_hip", "-ltorch",
           "-ltorch_cpu", "-ltorch_python", f"-L{LIB_DIR}", "-ltheria_sdpa", "-Wl,-rpath,$ORIGIN/lib"]
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{res.stdout}")
    os.replace(tmp, out)
    return out


def build(verbose: bool = True, jobs: int | None = None) -> Path:
    """Compile every kernel source and link the shared library, then the torch binding. Always rebuilds."""
    hipcc = _hipcc()
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = jobs or min(len(sources) + 1, max(1, (os.cpu_count() or 4)))
    if verbose:
        print(f"[theria_amd.build] compiling {len(sources)} sources for {ARCH} and the torch binding with {jobs} jobs",
              flush=True)
    (BUILD_DIR / "tiles").mkdir(exist_ok=True)
    with _cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        host_obj = ex.submit(_compile_host)
        objs = ex.map(lambda s: _compile(hipcc, s), sources)
        tile_objs = ex.map(lambda s: _compile(hipcc, s, tiles=True), sources)
        objs, tile_objs, host_obj = list(objs), list(tile_objs), host_obj.result()
    _link(hipcc, objs, LIB_PATH)
    _link(hipcc, tile_objs, TILES_LIB_PATH)
    host = _link_host(host_obj)
    if verbose:
        print(f"[theria_amd.build] built {LIB_PATH.name}, {TILES_LIB_PATH.name} and {host.name} in {LIB_DIR.parent}",
              flush=True)
    return LIB_PATH


def _link(hipcc: str, objs, out: Path) -> None:
    tmp = out.with_suffix(".so.tmp")
    vmap = BUILD_DIR / "exports.map"
    vmap.write_text(EXPORTS)
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", f"-Wl,--version-script={vmap}", "-o", str(tmp),
           *map(str, objs)]
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{res.stdout}")
    os.replace(tmp, out)


if __name__ == "__main__":
    build()
    sys.exit(0)
