"""The C ABI's host code under AddressSanitizer and UndefinedBehaviorSanitizer
(CPU only; no GPU code runs).

Builds libkla_hip.so with the sanitizers on the host pass
(kalman-linear-attention_amd/csrc/build.py --sanitize) into a temporary
directory, then runs tests/test_abi.py and tests/test_abi_extremes.py in a child
interpreter that loads that build (KLA_HIP_LIB) with the ASan runtime preloaded
and any sanitizer report fatal: every argument check, error path and workspace
size computation the ABI tests reach -- extreme shapes included -- is free of
out-of-bounds accesses and undefined behaviour such as signed overflow.
"""

import glob
import os
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(REPO, "kalman-linear-attention_amd", "csrc")


def _asan_runtime():
    found = sorted(glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    return found[-1] if found else None


@pytest.mark.slow
def test_abi_checks_are_clean_under_asan_and_ubsan(tmp_path):
    runtime = _asan_runtime()
    if runtime is None:
        pytest.skip("no clang AddressSanitizer runtime in /opt/rocm/llvm")
    sys.path.insert(0, CSRC)
    try:
        import build as hip_build
    finally:
        sys.path.remove(CSRC)
    lib = hip_build.build(str(tmp_path / "libkla_hip_sanitized.so"), verbose=False, sanitize=True)
    env = dict(os.environ, KLA_HIP_LIB=lib, LD_PRELOAD=runtime,
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=0",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    proc = subprocess.run([sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider",
                           os.path.join(REPO, "tests", "test_abi.py"),
                           os.path.join(REPO, "tests", "test_abi_extremes.py")],
                          cwd=REPO, env=env, capture_output=True, text=True, timeout=600)
    out = proc.stdout + proc.stderr
    assert "runtime error" not in out and "AddressSanitizer" not in out, out[-4000:]
    assert proc.returncode == 0, out[-4000:]
    assert " passed" in out
