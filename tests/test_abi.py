"""The C-ABI library: loads, exports every entry point include/tensorjit_hip.h declares,
and reports errors through tj_hip_last_error (no GPU needed for these paths)."""
import ctypes
import re
from pathlib import Path

import pytest

from tensorjit.runtime import hip as rt

HEADER = Path(__file__).resolve().parents[1] / "include" / "tensorjit_hip.h"


def _declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(tj_hip_\w+)\s*\(", text)))


def test_library_is_built():
    assert rt.library_path().exists(), "run __graft_entry__.build() first"


def test_library_exports_every_declared_symbol():
    lib = rt.load()
    names = _declared()
    assert len(names) >= 12
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(rt.SIGNATURES)


def test_abi_version_matches():
    assert rt.load().tj_hip_abi_version() == rt.ABI_VERSION


def test_compile_error_carries_the_hiprtc_log():
    with pytest.raises(rt.HipError) as e:
        rt.compile_source('extern "C" __global__ void k() { this is not hip; }', "bad.hip", ["--offload-arch=gfx950"])
    assert "hipRTC compile failed" in str(e.value)


def test_compile_produces_a_code_object():
    code = rt.compile_source('extern "C" __global__ void k(float* p) { p[threadIdx.x] = 1.0f; }', "ok.hip",
                             ["--offload-arch=gfx950", "-O3"])
    assert len(code) > 100


def test_program_create_rejects_bad_arguments_before_touching_a_device():
    lib = rt.load()
    h = ctypes.c_void_p()
    assert lib.tj_hip_program_create(0, None, 0, 0, None, None, None, 0, 0, 0, ctypes.byref(h)) != 0
    assert b"empty code object" in lib.tj_hip_last_error()
    assert lib.tj_hip_program_create(0, b"x", 1, 0, None, None, None, 0, -1, 0, ctypes.byref(h)) != 0
    assert lib.tj_hip_program_run(None, None, None, None) != 0
    assert b"null program" in lib.tj_hip_last_error()
