"""Output buffers that a program hands to its caller, recycled only once dropped.

Contract (the reference's ``BufferPool.take_output``,
``tensorjit/runtime/executor.py:19-79``): a buffer returned by one call is
reused by a later call only when the caller holds nothing that can still see
its memory -- no tensor, no view, no storage handle.

Mechanism (this module's own): the pool owns each buffer as a bare
``UntypedStorage`` and never keeps a tensor of it.  Every call gets a *new*
tensor built on a free storage with ``Tensor.set_``.  Any tensor or view the
caller still holds keeps a reference on the storage's C++ object, so a storage
is free exactly when the pool's handle is its only user: use count 1 on the C++
side and no Python reference to the handle beyond the pool's own (a caller may
hold ``out.untyped_storage()``, which is the very same Python object).

On the GPU the point is pointer stability: a program called in a loop whose
results are dropped each time gets the same output addresses every call,
so a captured hipGraph for that pointer set is replayed, not re-captured.
"""
from __future__ import annotations

import sys

import torch

_use_count = torch._C._storage_Use_Count


class _Buffer:
    """One pooled storage and the layout it is handed out with."""

    __slots__ = ("storage", "dtype", "device", "shape", "stride")

    def __init__(self, shape: tuple[int, ...], dtype: torch.dtype, device):
        t = torch.empty(shape, dtype=dtype, device=device)
        self.storage = t.untyped_storage()
        self.dtype, self.device, self.shape, self.stride = dtype, t.device, tuple(shape), t.stride()

    def unused(self) -> bool:
        # sys.getrefcount sees this attribute and its own argument: 2 means nobody
        # outside the pool holds the storage handle
        return _use_count(self.storage._cdata) == 1 and sys.getrefcount(self.storage) == 2

    def tensor(self) -> torch.Tensor:
        return torch.empty(0, dtype=self.dtype, device=self.device).set_(self.storage, 0, self.shape, self.stride)


class BufferPool:
    """Per (shape, dtype, device): the storages handed out so far, oldest first.

    At most ``MAX_HELD`` storages are remembered per key; when a call finds all
    of them still in the caller's hands it allocates a new one and forgets the
    oldest (which is freed whenever the caller drops it)."""

    MAX_HELD = 8

    def __init__(self):
        self._held: dict[tuple, list[_Buffer]] = {}

    def take_output(self, shape, dtype: torch.dtype, device) -> torch.Tensor:
        if type(shape) is not tuple:
            shape = tuple(int(d) for d in shape)
        key = (shape, dtype, device)
        held = self._held.setdefault(key, [])
        for buf in held:
            if buf.unused():
                return buf.tensor()
        buf = _Buffer(shape, dtype, device)
        held.append(buf)
        if len(held) > self.MAX_HELD:
            del held[0]
        return buf.tensor()

    def held(self) -> int:
        """Storages currently remembered (for tests and stats)."""
        return sum(len(v) for v in self._held.values())
