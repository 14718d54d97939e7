"""The C ABI from C: tests/abi_client.c is compiled with gcc against
include/kla_hip.h and linked to the built libkla_hip.so, then run on the CPU
(version, workspace size, argument checks, an empty problem). This is the
binding a C or cgo / JNI / N-API caller would write, with no C++ or torch type
in sight."""

import os
import shutil
import subprocess

import pytest

from kla.ops.hip import _lib

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)


@pytest.mark.skipif(shutil.which("gcc") is None, reason="no C compiler")
def test_c_client_uses_the_abi(tmp_path):
    lib = _lib.LIB_PATH
    assert os.path.exists(lib), f"{lib} is not built (run __graft_entry__.build())"
    exe = tmp_path / "abi_client"
    cmd = ["gcc", "-std=c11", "-Wall", "-Werror", "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(REPO, "include"),
           "-I", "/opt/rocm/include", os.path.join(HERE, "abi_client.c"), "-o", str(exe), lib,
           f"-Wl,-rpath,{os.path.dirname(lib)}"]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    out = subprocess.run([str(exe), str(_lib.ABI_VERSION)], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr + out.stdout
    assert "abi client ok" in out.stdout


@pytest.mark.gpu
@pytest.mark.skipif(shutil.which("gcc") is None, reason="no C compiler")
def test_c_client_runs_the_scans_on_the_gpu(tmp_path):
    """tests/abi_gpu_client.c: the Moebius and affine forward scans from plain C
    (hipMalloc / hipMemcpy / a hipStream_t and the C ABI), against a float64
    per-step loop at rtol 1e-5 / atol 1e-6, no look-back wait given up."""
    lib = _lib.LIB_PATH
    exe = tmp_path / "abi_gpu_client"
    cmd = ["gcc", "-std=c11", "-O2", "-Wall", "-Werror", "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(REPO, "include"),
           "-I", "/opt/rocm/include", os.path.join(HERE, "abi_gpu_client.c"), "-o", str(exe), lib,
           "-L/opt/rocm/lib", "-lamdhip64", "-lm", f"-Wl,-rpath,{os.path.dirname(lib)}", "-Wl,-rpath,/opt/rocm/lib"]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    print("[c client] running the scans from C", flush=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    print(out.stdout, flush=True)
    assert out.returncode == 0, out.stderr + out.stdout
    assert "gpu abi client ok" in out.stdout
