"""Static arena planning for intermediates.

After fusion a program is a straight line of kernels, so each intermediate
lives over an interval ``[defining kernel, last reading kernel]``.  Buffers
are placed in one arena by greedy best fit over the free gaps, in order of
definition (larger first within a kernel); graph outputs stay outside the
arena because the caller owns them.  Same placement rule, alignment and
verification as the reference (``tensorjit/passes/memory_planner.py:28-129``),
so arena sizes and offsets agree with it for the same program.

On the GPU the arena is one ``hipMalloc`` owned by the program.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

from ..ir import Node
from .fusion import Program

ALIGN = 64  # bytes


@dataclass
class Buffer:
    node: Node
    size: int     # bytes, multiple of ALIGN
    first: int    # defining kernel index
    last: int     # last reading kernel index
    offset: int = -1

    @property
    def shape(self):
        return self.node.shape


@dataclass
class MemoryPlan:
    buffers: dict[int, Buffer] = field(default_factory=dict)
    arena_bytes: int = 0
    naive_bytes: int = 0

    @property
    def savings(self) -> float:
        return 1.0 - self.arena_bytes / self.naive_bytes if self.naive_bytes else 0.0

    def offset(self, node: Node) -> int | None:
        b = self.buffers.get(id(node))
        return None if b is None else b.offset

    def __str__(self) -> str:
        rows = [f"arena {self.arena_bytes} B (naive {self.naive_bytes} B, {self.savings:.0%} saved)"]
        for b in sorted(self.buffers.values(), key=lambda b: b.offset):
            rows.append(f"  [{b.offset:8d}, +{b.size:8d})  k{b.first}..k{b.last}  {b.node.name} {b.shape}")
        return "\n".join(rows)


def _round_up(nbytes: int) -> int:
    return -(-nbytes // ALIGN) * ALIGN


def _nbytes(n: Node) -> int:
    return (math.prod(n.shape) if n.shape else 1) * n.dtype.itemsize


def plan_memory(program: Program) -> MemoryPlan:
    returned = {id(program.resolve(o)) for o in program.graph.outputs}

    buffers: dict[int, Buffer] = {}
    for ki, k in enumerate(program.kernels):
        for o in k.outputs:
            if id(o) not in returned:
                buffers[id(o)] = Buffer(o, _round_up(max(_nbytes(o), 1)), first=ki, last=ki)
        for i in k.inputs:
            b = buffers.get(id(program.resolve(i)))
            if b is not None:
                b.last = ki

    arena = 0
    live: list[Buffer] = []
    for b in sorted(buffers.values(), key=lambda b: (b.first, -b.size)):
        live = [x for x in live if x.last >= b.first]
        best_at, best_gap = None, None
        cursor = 0
        for lo, hi in sorted((x.offset, x.offset + x.size) for x in live) + [(arena, arena)]:
            gap = lo - cursor
            if gap >= b.size and (best_gap is None or gap < best_gap):
                best_at, best_gap = cursor, gap
            cursor = max(cursor, hi)
        b.offset = cursor if best_at is None else best_at
        arena = max(arena, b.offset + b.size)
        live.append(b)

    plan = MemoryPlan(buffers, arena_bytes=arena, naive_bytes=sum(b.size for b in buffers.values()))
    _verify(plan)
    return plan


def _verify(plan: MemoryPlan) -> None:
    """No two buffers that are live at the same time may overlap in the arena."""
    bufs = list(plan.buffers.values())
    for i, a in enumerate(bufs):
        for b in bufs[i + 1:]:
            same_time = not (a.last < b.first or b.last < a.first)
            same_bytes = not (a.offset + a.size <= b.offset or b.offset + b.size <= a.offset)
            if same_time and same_bytes:
                raise AssertionError(f"memory plan conflict: {a.node.name} vs {b.node.name}")
