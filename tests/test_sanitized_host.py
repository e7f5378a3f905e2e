"""The library's host layer under AddressSanitizer + UndefinedBehaviorSanitizer.

mojogp_amd/lib/asan/libmojogp_amd.so is the same sources built with every
-fsanitize applied to the host pass only (mojogp_amd.build, sanitized=True;
device code is unchanged).  A child process loads it with the GCC ASan and
UBSan runtimes preloaded and drives the C entry points
(tests/sanitized_host_calls.py); any sanitizer report aborts it.
"""

import os
import subprocess
import sys

import pytest

from mojogp_amd import build as native_build

HERE = os.path.dirname(os.path.abspath(__file__))


def _run(mode: str, timeout: int):
    rts = native_build.sanitizer_runtimes()
    lib = native_build.ASAN_LIB_PATH
    if rts is None or not lib.exists():
        pytest.skip("sanitized library or sanitizer runtimes missing (python -m mojogp_amd.build)")
    env = dict(os.environ)
    pre = ":".join(str(r) for r in rts)
    env["LD_PRELOAD"] = pre + (":" + env["LD_PRELOAD"] if env.get("LD_PRELOAD") else "")
    env["ASAN_OPTIONS"] = "detect_leaks=0:halt_on_error=1:verify_asan_link_order=0"
    env["UBSAN_OPTIONS"] = "halt_on_error=1:print_stacktrace=1"
    env["MOJOGP_AMD_LIB"] = str(lib)
    proc = subprocess.run([sys.executable, os.path.join(HERE, "sanitized_host_calls.py"), mode],
                          env=env, capture_output=True, text=True, timeout=timeout)
    out = proc.stdout + proc.stderr
    print(out[-4000:])
    assert "ERROR: AddressSanitizer" not in out
    assert "runtime error:" not in out
    assert proc.returncode == 0, out[-4000:]
    assert f"sanitized host layer: {mode} OK" in proc.stdout


def test_host_layer_under_sanitizers_cpu():
    _run("cpu", 600)


@pytest.mark.gpu
def test_host_layer_under_sanitizers_gpu():
    _run("gpu", 600)
