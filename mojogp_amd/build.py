"""Build the gfx950 shared library ``mojogp_amd/lib/libmojogp_amd.so``.

Every ``csrc/*.hip`` translation unit is compiled with hipcc for gfx950 only
(object files go to ``mojogp_amd/lib/obj``), then linked into one C-ABI
library that the ctypes loader in ``mojogp_amd._lib`` opens.

Usage: ``python -m mojogp_amd.build`` (or ``build()`` from Python).
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
OBJ_DIR = LIB_DIR / "obj"
LIB_PATH = LIB_DIR / "libmojogp_amd.so"
ARCH = "gfx950"

# Packed-FP32 VALU forms are disabled for all device code (hipcc's host pass
# warns that it does not know the feature; that warning is harmless).
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    # MFMA sources/results in ordinary VGPRs: no v_accvgpr_read/write copies
    # between the matrix accumulators and the VALU kernel-value math.
    "-mllvm",
    "-amdgpu-mfma-vgpr-form",
    "-Wno-unused-result",
]


# hiprtc compiles the per-tree product kernels (tree_jit.hip) at run time; no
# vendor math library is linked.
LINK_LIBS = ["-L/opt/rocm/lib", "-lhiprtc", "-Wl,-rpath,/opt/rocm/lib"]


def _hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; the gfx950 library cannot be built")
    return path


# Host-side sanitizers for the checking build (device code is compiled exactly
# as in the product library; every -fsanitize applies to the host pass only).
ASAN_DIR = LIB_DIR / "asan"
ASAN_LIB_PATH = ASAN_DIR / "libmojogp_amd.so"
HOST_SANITIZE_FLAGS = [
    "-Xarch_host", "-fsanitize=address",
    "-Xarch_host", "-fsanitize=undefined",
    "-Xarch_host", "-fno-sanitize=function",
    "-Xarch_host", "-fno-omit-frame-pointer",
    "-Xarch_host", "-fno-sanitize-recover=undefined",
]

# Runtimes preloaded into a process that loads the sanitized library: the
# system GCC libasan / libubsan (same ASan v8 interface).  The ROCm clang ASan
# runtime is not used: it also intercepts the HSA memory-pool allocator for
# device-side ASan, which fails without XNACK, so device allocations abort.
_SANITIZER_RUNTIMES = [Path("/usr/lib/x86_64-linux-gnu/libasan.so.6"),
                       Path("/usr/lib/x86_64-linux-gnu/libubsan.so.1")]


def sanitizer_runtimes() -> list[Path] | None:
    """Libraries to preload (in order) for the sanitized build, or None."""
    return _SANITIZER_RUNTIMES if all(p.exists() for p in _SANITIZER_RUNTIMES) else None


def _compile_one(src: Path, obj_dir: Path = OBJ_DIR, extra=()) -> Path:
    obj = obj_dir / (src.stem + ".o")
    cmd = [_hipcc(), *HIP_FLAGS, *extra, "-I", str(CSRC), "-I", str(REPO_DIR / "include"),
           "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stdout}\n{proc.stderr}")
    return obj


def build(verbose: bool = False, jobs: int | None = None, sanitized: bool = False) -> Path:
    """Compile all HIP sources and link the shared library. Returns its path.

    sanitized: the checking build instead, host code under AddressSanitizer
    and UndefinedBehaviorSanitizer (``mojogp_amd/lib/asan``); a process that
    loads it preloads sanitizer_runtimes()."""
    obj_dir = (ASAN_DIR / "obj") if sanitized else OBJ_DIR
    lib_path = ASAN_LIB_PATH if sanitized else LIB_PATH
    extra = HOST_SANITIZE_FLAGS if sanitized else ()
    obj_dir.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = jobs or min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with _cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda src: _compile_one(src, obj_dir, extra), sources))
    tmp = lib_path.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *map(str, objs), *LINK_LIBS]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, lib_path)
    if verbose:
        print(f"built {lib_path} from {len(sources)} sources")
    return lib_path


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
