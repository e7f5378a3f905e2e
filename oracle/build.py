"""Build the C restatement under oracle/cpu_ref into oracle/lib/liboracle_ref.so
(test/baseline infrastructure; gcc + OpenMP).  No reference sources are
compiled: the reference's path is Mojo and cannot be built here."""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

ORACLE_DIR = Path(__file__).resolve().parent
SRC_DIR = ORACLE_DIR / "cpu_ref"
LIB_DIR = ORACLE_DIR / "lib"
LIB_PATH = LIB_DIR / "liboracle_ref.so"

# x86-64-v3 (AVX2 + FMA) so the library runs on the GPU box's host as well.
CFLAGS = ["-O3", "-fPIC", "-shared", "-fopenmp", "-march=x86-64-v3", "-std=c11"]


def build(verbose: bool = False) -> Path:
    cc = shutil.which("gcc") or "cc"
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    srcs = sorted(str(p) for p in SRC_DIR.glob("*.c"))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [cc, *CFLAGS, "-o", str(tmp), *srcs, "-lm"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{proc.stdout}\n{proc.stderr}")
    tmp.replace(LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
