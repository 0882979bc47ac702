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


def _create(launch_args, arena_bytes, n_in=1, n_out=1):
    """tj_hip_program_create on one kernel with the given argument refs (fails before any
    device work when a reference is invalid)."""
    lib = rt.load()
    names = (ctypes.c_char_p * 1)(b"k")
    desc = (rt.LaunchDesc * 1)()
    desc[0].grid[:] = [1, 1, 1]
    desc[0].block[:] = [64, 1, 1]
    desc[0].nargs = len(launch_args)
    refs = (rt.ArgRef * max(len(launch_args), 1))()
    for i, r in enumerate(launch_args):
        refs[i].kind, refs[i].value = r[0], r[1]
        refs[i].bytes = r[2] if len(r) > 2 else 0
    h = ctypes.c_void_p()
    rc = lib.tj_hip_program_create(0, b"not a code object", 17, 1, names, desc, refs, arena_bytes, n_in, n_out,
                                   ctypes.byref(h))
    return rc, lib.tj_hip_last_error().decode()


@pytest.mark.parametrize("ref,arena,why", [
    ((rt.ARENA, 0, 4097), 4096, "outside the 4096-byte arena"),      # runs past the end
    ((rt.ARENA, 4000, 128), 4096, "outside the 4096-byte arena"),
    ((rt.ARENA, 4096, 1), 4096, "outside the 4096-byte arena"),      # starts at the end
    ((rt.ARENA, -64, 64), 4096, "outside"),
    ((rt.ARENA, 0, 0), 4096, "outside"),                             # size must be given
    ((rt.ARENA, 0, 64), 0, "outside the 0-byte arena"),
    ((rt.INPUT, 1), 4096, "input index out of range"),
    ((rt.OUTPUT, -1), 4096, "output index out of range"),
    ((7, 0), 4096, "bad argument kind"),
])
def test_argument_references_are_validated_before_loading(ref, arena, why):
    rc, msg = _create([ref], arena)
    assert rc != 0 and why in msg, msg


def test_valid_references_get_as_far_as_loading_the_code_object():
    # every reference is in range, so creation fails only at the (bogus) code object
    rc, msg = _create([(rt.INPUT, 0), (rt.ARENA, 64, 4032), (rt.OUTPUT, 0)], 4096)
    assert rc != 0 and "hipModuleLoadData" in msg, msg


def test_toolchain_version_needs_no_device():
    major, minor, runtime = rt.toolchain_version()
    assert major >= 6 and minor >= 0 and runtime >= 60000000
