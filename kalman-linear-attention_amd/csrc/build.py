"""Build libkla_hip.so (the gfx950 scan kernels + C ABI) in-tree.

    python kalman-linear-attention_amd/csrc/build.py [--out PATH] [--save-temps DIR]

Runs hipcc directly (no CMake, no torch): the library links only the HIP
runtime, so it loads through ctypes next to whatever HIP runtime torch has
already brought into the process (both carry the soname libamdhip64.so.7).
"""

from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
PKG_ROOT = os.path.dirname(HERE)  # kalman-linear-attention_amd/
REPO = os.path.dirname(PKG_ROOT)
INCLUDE = os.path.join(REPO, "include")
DEFAULT_OUT = os.path.join(PKG_ROOT, "kla", "lib", "libkla_hip.so")
SOURCES = ["kla_hip.hip"]
HEADERS = ["causal_conv.hpp", "fused_kla.hpp", "gate_skip.hpp", "lookback_scan.hpp", "model_ops.hpp", "rows_linear.hpp",
           "scan_ops.hpp"]

# -packed-fp32-ops: keep the compiler from forming v_pk_{add,mul,fma}_f32.
HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-fvisibility=hidden",
    "-Wall",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


# Host-sanitised build (AddressSanitizer + UndefinedBehaviorSanitizer on the host
# code only; each -fsanitize= goes to the host pass, the device code is built
# unoptimised and never run): the C ABI's argument checks and size arithmetic
# under the sanitizers, loaded by tests/test_abi_sanitized.py with the ASan
# runtime preloaded.
SANITIZE_FLAGS = [
    "-Xarch_host", "-fsanitize=address",
    "-Xarch_host", "-fsanitize=undefined",
    "-Xarch_host", "-fno-sanitize-recover=undefined",
    "-Xarch_host", "-fno-omit-frame-pointer",
    "-Xarch_host", "-O1",
    "-Xarch_device", "-O0",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (looked at $HIPCC, /opt/rocm/bin/hipcc, PATH)")


def build(out: str = DEFAULT_OUT, save_temps: str | None = None, verbose: bool = True,
          sanitize: bool = False) -> str:
    out = os.path.abspath(out)
    os.makedirs(os.path.dirname(out), exist_ok=True)
    tmp = out + ".tmp"
    flags = [f for f in HIPCC_FLAGS if not (sanitize and f == "-O3")] + (SANITIZE_FLAGS if sanitize else [])
    cmd = [hipcc(), *flags, "-I", INCLUDE, "-I", HERE]
    if save_temps:
        os.makedirs(save_temps, exist_ok=True)
        cmd += ["-save-temps"]
    cmd += [os.path.join(HERE, s) for s in SOURCES] + ["-o", tmp]
    if verbose:
        print("[kla build]", " ".join(cmd), flush=True)
    cwd = save_temps or HERE
    proc = subprocess.run(cmd, cwd=cwd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"hipcc failed with status {proc.returncode}")
    # Host pass warns that it does not know the packed-fp32 target feature: harmless.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    msgs = [ln for ln in (proc.stdout + proc.stderr).splitlines() if noise not in ln and "warning generated" not in ln]
    if verbose and any(m.strip() for m in msgs):
        print("\n".join(msgs), flush=True)
    os.replace(tmp, out)
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--out", default=DEFAULT_OUT)
    ap.add_argument("--save-temps", default=None, help="directory for compiler intermediates (ISA)")
    ap.add_argument("--sanitize", action="store_true", help="host AddressSanitizer + UBSan build (CPU checks only)")
    args = ap.parse_args(argv)
    build(args.out, args.save_temps, sanitize=args.sanitize)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
