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
