"""The native runtime's host code under AddressSanitizer + UndefinedBehaviorSanitizer: a C++
driver (tests/native/abi_driver.cpp) built together with csrc/runtime.cpp, with the
sanitizers on the host side only (``-Xarch_host``), exercising every C-ABI path that needs
no GPU.  Any invalid memory access or undefined behaviour aborts the driver."""
import os
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


@pytest.mark.skipif(not Path(HIPCC).exists(), reason="needs hipcc")
def test_c_abi_error_paths_are_clean_under_asan_and_ubsan(tmp_path):
    exe = tmp_path / "abi_driver"
    cmd = [HIPCC, "--offload-arch=gfx950", "-std=c++17", "-O1", "-g",
           "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
           "-Xarch_host", "-fno-sanitize-recover=all",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           str(ROOT / "mlir-gpu-kernel-compiler_amd" / "csrc" / "runtime.cpp"),
           str(ROOT / "tests" / "native" / "abi_driver.cpp"), "-o", str(exe), "-lhiprtc"]
    build = subprocess.run(cmd, capture_output=True, text=True)
    assert build.returncode == 0, build.stderr[-3000:]
    # the HIP runtime's own one-time allocations are not this library's leaks
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:halt_on_error=1", UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    run = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=120)
    assert run.returncode == 0 and "OK (0 failures)" in run.stdout, run.stdout[-3000:] + run.stderr[-3000:]
