"""Caller-visible output buffers that are recycled only once dropped.

Same contract as the reference ``BufferPool`` (``tensorjit/runtime/executor.py:19-79``):
an output handed to the caller is reused by a later call only when no Python
reference, view or storage alias of it remains.  On the GPU this keeps the
pointer set of a program stable across calls, which is what lets a captured
hipGraph be replayed without re-capture.
"""
from __future__ import annotations

import sys

import torch


class BufferPool:
    MAX_HELD = 8
    _BASELINE: int | None = None   # refcount of a tensor held only by the scan below

    def __init__(self):
        self._free: dict[tuple, list[torch.Tensor]] = {}
        self._handed_out: dict[tuple, list[torch.Tensor]] = {}

    def take(self, shape, dtype, device) -> torch.Tensor:
        free = self._free.get((tuple(shape), dtype, str(device)))
        if free:
            return free.pop()
        return torch.empty(shape, dtype=dtype, device=device)

    def give(self, t: torch.Tensor) -> None:
        self._free.setdefault((tuple(t.shape), t.dtype, str(t.device)), []).append(t)

    def _scan(self, held: list[torch.Tensor], record: bool = False):
        """Index of the first held tensor that nobody else references (else None).

        The calibration call (``record=True``) goes through the same loop so the
        CPython reference count it records matches the one seen here.
        """
        for i, t in enumerate(held):
            rc = sys.getrefcount(t)
            if record:
                return rc
            if (rc == self._BASELINE and t._use_count() == 1
                    and torch._C._storage_Use_Count(t.untyped_storage()._cdata) == 2):
                return i
        return None

    def take_output(self, shape, dtype, device) -> torch.Tensor:
        if BufferPool._BASELINE is None:
            BufferPool._BASELINE = self._scan([torch.empty(1)], record=True)
        key = (tuple(shape), dtype, str(device))
        held = self._handed_out.setdefault(key, [])
        i = self._scan(held)
        if i is not None:
            held.append(held.pop(i))
            return held[-1]
        t = torch.empty(shape, dtype=dtype, device=device)
        held.append(t)
        if len(held) > self.MAX_HELD:
            held.pop(0)
        return t
