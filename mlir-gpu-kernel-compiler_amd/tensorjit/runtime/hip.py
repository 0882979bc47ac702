"""ctypes binding of the HIP executor library (``libtjhip.so``, C ABI in
``include/tensorjit_hip.h``).

The library is built in-tree by ``tensorjit.build.build_library()``.  Loading
never falls back to anything else: if the library is missing the hip backend
raises ``HipError`` with the build instruction.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path
from typing import Sequence

LIB_NAME = "libtjhip.so"
LIB_PATH = Path(__file__).resolve().parents[1] / LIB_NAME
ABI_VERSION = 3

INPUT, ARENA, OUTPUT = 0, 1, 2
STATIC_ARENA_BYTES = 64 << 20   # TJ_HIP_STATIC_ARENA_BYTES


class HipError(RuntimeError):
    """Raised for every nonzero status of the C ABI (message from tj_hip_last_error)."""


class ArgRef(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int32), ("pad_", ctypes.c_int32), ("value", ctypes.c_int64),
                ("bytes", ctypes.c_int64)]


class LaunchDesc(ctypes.Structure):
    _fields_ = [("grid", ctypes.c_uint32 * 3), ("block", ctypes.c_uint32 * 3),
                ("lds_bytes", ctypes.c_uint32), ("nargs", ctypes.c_uint32)]


class Stats(ctypes.Structure):
    _fields_ = [("calls", ctypes.c_uint64), ("graph_replays", ctypes.c_uint64),
                ("graph_captures", ctypes.c_uint64), ("host_ns", ctypes.c_uint64),
                ("direct_fallbacks", ctypes.c_uint64)]


class DeviceInfo(ctypes.Structure):
    _fields_ = [("cu_count", ctypes.c_int32), ("lds_per_block", ctypes.c_int32), ("warp_size", ctypes.c_int32),
                ("max_threads_per_block", ctypes.c_int32), ("clock_khz", ctypes.c_int32),
                ("mem_clock_khz", ctypes.c_int32), ("mem_bus_width", ctypes.c_int32), ("l2_bytes", ctypes.c_int32),
                ("total_mem", ctypes.c_int64), ("arch", ctypes.c_char * 64)]


# (name, restype, argtypes) for every exported entry point
_VP = ctypes.c_void_p
_PP = ctypes.POINTER(ctypes.c_void_p)
SIGNATURES = {
    "tj_hip_abi_version": (ctypes.c_int, []),
    "tj_hip_last_error": (ctypes.c_char_p, []),
    "tj_hip_device_info": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(DeviceInfo)]),
    "tj_hip_toolchain_version": (ctypes.c_int, [ctypes.POINTER(ctypes.c_int)] * 3),
    "tj_hip_compile": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p), ctypes.c_int,
                                      _PP, ctypes.POINTER(ctypes.c_size_t)]),
    "tj_hip_free": (None, [_VP]),
    "tj_hip_program_create": (ctypes.c_int, [ctypes.c_int, _VP, ctypes.c_size_t, ctypes.c_int,
                                             ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(LaunchDesc),
                                             ctypes.POINTER(ArgRef), ctypes.c_size_t, ctypes.c_int, ctypes.c_int, _PP]),
    "tj_hip_program_run": (ctypes.c_int, [_VP, _PP, _PP, _VP]),
    "tj_hip_program_run_static": (ctypes.c_int, [_VP, _PP, _PP, _VP]),
    "tj_hip_program_capture": (ctypes.c_int, [_VP, _PP, _PP]),
    "tj_hip_program_replay": (ctypes.c_int, [_VP, _PP, _PP, _VP]),
    "tj_hip_program_stats": (ctypes.c_int, [_VP, ctypes.POINTER(Stats)]),
    "tj_hip_program_arena": (ctypes.c_int, [_VP, _PP, ctypes.POINTER(ctypes.c_size_t)]),
    "tj_hip_kernel_time": (ctypes.c_int, [_VP, ctypes.c_int, _PP, _PP, _VP, ctypes.c_int, ctypes.c_int,
                                          ctypes.POINTER(ctypes.c_float)]),
    "tj_hip_program_time_kernels": (ctypes.c_int, [_VP, _PP, _PP, _VP, ctypes.POINTER(ctypes.c_float)]),
    "tj_hip_program_destroy": (ctypes.c_int, [_VP]),
}

_lib = None


def library_path() -> Path:
    return Path(os.environ.get("TENSORJIT_HIP_LIB", LIB_PATH))


def load() -> ctypes.CDLL:
    """Load ``libtjhip.so`` and declare every signature (raises HipError if absent)."""
    global _lib
    if _lib is not None:
        return _lib
    path = library_path()
    if not path.exists():
        raise HipError(f"{path} is missing: build it with `python -c 'import tensorjit.build as b; b.build_library()'` "
                       "(or __graft_entry__.build())")
    lib = ctypes.CDLL(str(path))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.tj_hip_abi_version() != ABI_VERSION:
        raise HipError(f"{path}: ABI version {lib.tj_hip_abi_version()} != {ABI_VERSION}; rebuild it")
    _lib = lib
    return lib


def check(rc: int, what: str = "") -> None:
    if rc != 0:
        msg = load().tj_hip_last_error().decode(errors="replace")
        raise HipError(f"{what}: {msg}" if what else msg)


def device_info(device: int = 0) -> DeviceInfo:
    info = DeviceInfo()
    check(load().tj_hip_device_info(device, ctypes.byref(info)), "tj_hip_device_info")
    return info


def toolchain_version() -> tuple[int, int, int]:
    """(hipRTC major, hipRTC minor, HIP runtime version); needs no GPU."""
    major, minor, runtime = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    check(load().tj_hip_toolchain_version(ctypes.byref(major), ctypes.byref(minor), ctypes.byref(runtime)),
          "tj_hip_toolchain_version")
    return major.value, minor.value, runtime.value


def compile_source(source: str, name: str, opts: Sequence[str]) -> bytes:
    lib = load()
    copts = (ctypes.c_char_p * len(opts))(*[o.encode() for o in opts])
    code = ctypes.c_void_p()
    size = ctypes.c_size_t()
    check(lib.tj_hip_compile(source.encode(), name.encode(), copts, len(opts), ctypes.byref(code), ctypes.byref(size)),
          "hipRTC")
    try:
        return ctypes.string_at(code, size.value)
    finally:
        lib.tj_hip_free(code)


def ptr_table(ptrs: Sequence[int]):
    return (ctypes.c_void_p * max(len(ptrs), 1))(*ptrs)


class NativeHipProgram:
    """Owns one ``tj_hip_program`` handle."""

    def __init__(self, device: int, code: bytes, names: Sequence[str], launches: Sequence[tuple],
                 args: Sequence[Sequence[tuple[int, ...]]], arena_bytes: int, n_in: int, n_out: int):
        lib = load()
        self._lib = lib
        self.n_in, self.n_out = n_in, n_out
        k = len(names)
        cnames = (ctypes.c_char_p * max(k, 1))(*[n.encode() for n in names])
        descs = (LaunchDesc * max(k, 1))()
        flat: list[tuple[int, ...]] = []
        for i, ((grid, block, lds), refs) in enumerate(zip(launches, args)):
            descs[i].grid[:] = list(grid)
            descs[i].block[:] = list(block)
            descs[i].lds_bytes = lds
            descs[i].nargs = len(refs)
            flat.extend(refs)
        crefs = (ArgRef * max(len(flat), 1))()
        for i, ref in enumerate(flat):
            # (INPUT, i) / (OUTPUT, j) / (ARENA, offset, bytes)
            crefs[i].kind, crefs[i].value = ref[0], ref[1]
            crefs[i].bytes = ref[2] if len(ref) > 2 else 0
        self._code = ctypes.create_string_buffer(code, len(code))
        # pointer tables reused by every call (a program is not re-entrant: it has one arena)
        self._in_arr = (ctypes.c_void_p * max(n_in, 1))()
        self._out_arr = (ctypes.c_void_p * max(n_out, 1))()
        handle = ctypes.c_void_p()
        check(lib.tj_hip_program_create(device, self._code, len(code), k, cnames, descs, crefs, arena_bytes, n_in, n_out,
                                        ctypes.byref(handle)), "tj_hip_program_create")
        self.handle = handle

    def _tables(self, ins: Sequence[int], outs: Sequence[int]):
        if len(ins) != self.n_in or len(outs) != self.n_out:
            raise HipError(f"expected {self.n_in} input and {self.n_out} output pointers, got {len(ins)} and {len(outs)}")
        ia, oa = self._in_arr, self._out_arr
        for i, p in enumerate(ins):
            ia[i] = p
        for j, p in enumerate(outs):
            oa[j] = p
        return ia, oa

    def run(self, ins: Sequence[int], outs: Sequence[int], stream: int) -> None:
        check(self._lib.tj_hip_program_run(self.handle, *self._tables(ins, outs), stream), "tj_hip_program_run")

    def _tensor_tables(self, ins, outs):
        """The pointer tables filled straight from tensors (the per-call path)."""
        if len(ins) != self.n_in or len(outs) != self.n_out:
            raise HipError(f"expected {self.n_in} input and {self.n_out} output tensors, got {len(ins)} and {len(outs)}")
        ia, oa = self._in_arr, self._out_arr
        for i, t in enumerate(ins):
            ia[i] = t.data_ptr()
        for j, t in enumerate(outs):
            oa[j] = t.data_ptr()
        return ia, oa

    def run_tensors(self, ins, outs, stream: int) -> None:
        """``run`` on tensors (their data pointers), the executor's per-call path."""
        if self._lib.tj_hip_program_run(self.handle, *self._tensor_tables(ins, outs), stream):
            check(1, "tj_hip_program_run")

    def replay_tensors(self, ins, outs, stream: int) -> None:
        if self._lib.tj_hip_program_replay(self.handle, *self._tensor_tables(ins, outs), stream):
            check(1, "tj_hip_program_replay")

    def run_static(self, ins: Sequence[int], outs: Sequence[int], stream: int) -> None:
        """``run`` with the intermediates in the library's static per-GPU arena (allocates
        nothing; rejects programs whose arena exceeds ``STATIC_ARENA_BYTES``)."""
        check(self._lib.tj_hip_program_run_static(self.handle, *self._tables(ins, outs), stream),
              "tj_hip_program_run_static")

    def capture(self, ins: Sequence[int], outs: Sequence[int]) -> None:
        check(self._lib.tj_hip_program_capture(self.handle, *self._tables(ins, outs)), "tj_hip_program_capture")

    def replay(self, ins: Sequence[int], outs: Sequence[int], stream: int) -> None:
        check(self._lib.tj_hip_program_replay(self.handle, *self._tables(ins, outs), stream),
              "tj_hip_program_replay")

    def kernel_time(self, k: int, ins: Sequence[int], outs: Sequence[int], stream: int, warmup: int = 2,
                    iters: int = 10) -> float:
        ms = ctypes.c_float()
        check(self._lib.tj_hip_kernel_time(self.handle, k, *self._tables(ins, outs), stream, warmup, iters,
                                           ctypes.byref(ms)), "tj_hip_kernel_time")
        return ms.value

    def time_kernels(self, ins: Sequence[int], outs: Sequence[int], stream: int, n: int) -> list[float]:
        """ms of each of the program's ``n`` launches within one call of the whole program."""
        ms = (ctypes.c_float * max(n, 1))()
        check(self._lib.tj_hip_program_time_kernels(self.handle, *self._tables(ins, outs), stream, ms),
              "tj_hip_program_time_kernels")
        return list(ms[:n])

    def stats(self) -> dict:
        s = Stats()
        check(self._lib.tj_hip_program_stats(self.handle, ctypes.byref(s)), "tj_hip_program_stats")
        return {"calls": s.calls, "graph_replays": s.graph_replays, "graph_captures": s.graph_captures,
                "direct_fallbacks": s.direct_fallbacks, "host_us": s.host_ns / 1e3}

    def arena(self) -> tuple[int, int]:
        p, n = ctypes.c_void_p(), ctypes.c_size_t()
        check(self._lib.tj_hip_program_arena(self.handle, ctypes.byref(p), ctypes.byref(n)), "tj_hip_program_arena")
        return p.value or 0, n.value

    def __del__(self):
        h = getattr(self, "handle", None)
        if h:
            try:
                self._lib.tj_hip_program_destroy(h)
            except Exception:
                pass
            self.handle = None
