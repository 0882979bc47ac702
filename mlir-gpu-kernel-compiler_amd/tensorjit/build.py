"""Build the HIP executor library in-tree (``tensorjit/libtjhip.so``).

    python -c "import tensorjit.build as b; b.build_library()"

The library is host code (hipRTC + HIP module API); the kernels themselves
are generated per program and compiled at run time by hipRTC for the
device's gfx target.
"""
from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
SRC = ROOT / "csrc" / "runtime.cpp"
OUT = PKG / "libtjhip.so"
ARCH = os.environ.get("TENSORJIT_HIP_ARCH", "gfx950")
# packed-fp32 instructions are kept out of every HIP build on these machines
NO_PACKED_FP32 = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found (ROCm is required to build the HIP executor)")
    return exe


def build_library(verbose: bool = False) -> Path:
    tmp = OUT.with_name(OUT.name + f".tmp{os.getpid()}")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-O2", "-std=c++17", "-shared", "-fPIC", "-Wall", *NO_PACKED_FP32,
           str(SRC), "-o", str(tmp), "-lhiprtc"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"building {OUT.name} failed:\n{' '.join(cmd)}\n{r.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT}")
    return OUT


if __name__ == "__main__":
    build_library(verbose=True)
