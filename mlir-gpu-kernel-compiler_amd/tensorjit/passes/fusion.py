"""Partition the graph into kernels, then merge per-row chains into row kernels.

The kernel plan is the backend's input, so it must match the reference plan
for the same graph: same greedy join rule over the topological order, same
cycle check, same epilogue/prologue conditions, same row grouping, same
schedule (``tensorjit/passes/fusion.py:78-333``).

Kernel kinds: ``elementwise`` (pointwise DAG over one iteration space),
``copy`` (a materialised transpose/broadcast), ``matmul`` (+ pointwise
epilogue), ``reduce`` (last-axis reduction + pointwise prologue/epilogue) and,
after ``row_fuse``, ``row`` (a chain of per-row stages read once per row).
"""
from __future__ import annotations

from dataclasses import dataclass, field

from ..ir import Graph, Node, OpKind


@dataclass
class Kernel:
    kind: str
    nodes: list[Node] = field(default_factory=list)     # compute nodes, topological
    anchor: Node | None = None                           # the matmul / reduce / movement node
    inputs: list[Node] = field(default_factory=list)    # values read from outside (no consts)
    outputs: list[Node] = field(default_factory=list)   # values that escape the kernel

    @property
    def iter_shape(self):
        if self.kind == "reduce":
            return self.anchor.inputs[0].shape
        if self.kind == "row":
            return tuple(self.rows) + (self.n,)  # type: ignore[attr-defined]
        return (self.anchor or self.nodes[-1]).shape

    def name(self) -> str:
        return f"{self.kind}_{abs(hash(tuple(n.name for n in self.nodes))) % 10**8:08x}"

    def __repr__(self) -> str:
        return f"Kernel<{self.kind} {[n.op for n in self.nodes]} -> {[o.name for o in self.outputs]}>"


@dataclass
class Program:
    graph: Graph
    kernels: list[Kernel]
    aliases: dict[int, tuple[Node, tuple]]   # id(reshape node) -> (source node, shape)

    def nodes_of(self, k: Kernel):
        return k.nodes

    def resolve(self, n: Node) -> Node:
        """Follow reshape aliases to the node that owns the storage."""
        while id(n) in self.aliases:
            n = self.aliases[id(n)][0]
        return n

    def __str__(self) -> str:
        rows = [f"program {self.graph.name}: {len(self.kernels)} kernels"]
        for k in self.kernels:
            rows.append(f"  {k.kind:12s} {[n.op for n in k.nodes]} -> {[o.name for o in k.outputs]}")
        return "\n".join(rows)


def _resolver(aliases: dict):
    def resolve(n: Node) -> Node:
        while id(n) in aliases:
            n = aliases[id(n)][0]
        return n

    return resolve


def _finalize(k: Kernel, g: Graph) -> None:
    """Recompute a kernel's external inputs (first-use order) and escaping outputs."""
    members = {id(n) for n in k.nodes}
    graph_outs = {id(o) for o in g.outputs}
    k.inputs, k.outputs = [], []
    listed: set[int] = set()
    for n in k.nodes:
        for src in n.inputs:
            if id(src) in members or src.op == "const" or id(src) in listed:
                continue
            listed.add(id(src))
            k.inputs.append(src)
        if id(n) in graph_outs or any(id(u) not in members for u in n.users):
            k.outputs.append(n)


def _dedupe(k: Kernel) -> None:
    seen: set[int] = set()
    unique = []
    for n in k.inputs:
        if id(n) not in seen:
            seen.add(id(n))
            unique.append(n)
    k.inputs = unique


def _escaping(k: Kernel) -> list[Node]:
    members = {id(n) for n in k.nodes}
    return [n for n in k.nodes if any(id(u) not in members for u in n.users)]


def _epilogue_ok(pk: Kernel, n: Node) -> bool:
    """An epilogue op may only read scalars or tensors of rank <= the anchor's."""
    rank = len(pk.anchor.shape)
    return all(i.shape == () or len(i.shape) <= rank for i in n.inputs)


def _no_cycle(target: Kernel, n: Node, producer: dict, resolve) -> bool:
    """Would adding ``n`` to ``target`` make ``target`` depend on itself?"""
    members = {id(m) for m in target.nodes}
    todo = [i for i in n.inputs if id(i) not in members]
    visited: set[int] = set()
    while todo:
        x = resolve(todo.pop())
        if id(x) in visited:
            continue
        visited.add(id(x))
        pk = producer.get(id(x))
        if pk is target:
            return False
        if pk is not None:
            todo.extend(pk.inputs or [i for m in pk.nodes for i in m.inputs])
    return True


def _prologue_source(pk: Kernel | None, red: Node, src: Node, graph_outs: set[int]) -> bool:
    """Can elementwise kernel ``pk`` (producer of ``src``) be pulled into reduction ``red``?"""
    if pk is None or pk.kind != "elementwise":
        return False
    for o in _escaping(pk):
        if id(o) in graph_outs or any(u is not red for u in o.users):
            return False
    return all(m.shape == src.shape for m in pk.nodes)


def fuse(g: Graph) -> Program:
    g.toposort()
    producer: dict[int, Kernel] = {}
    aliases: dict[int, tuple[Node, tuple]] = {}
    kernels: list[Kernel] = []
    graph_outs = {id(o) for o in g.outputs}
    resolve = _resolver(aliases)

    for n in g.nodes:
        if n.kind in (OpKind.INPUT, OpKind.CONST):
            continue

        if n.op == "reshape":
            # a reshape of a contiguous materialised value is a view: no kernel
            src = n.inputs[0]
            aliases[id(n)] = (src, n.shape)
            owner = producer.get(id(src))
            if owner is not None and src not in owner.outputs:
                owner.outputs.append(src)
            continue

        if n.kind in (OpKind.MOVEMENT, OpKind.MATMUL):
            k = Kernel("copy" if n.kind == OpKind.MOVEMENT else "matmul", [n], anchor=n)
            kernels.append(k)
            producer[id(n)] = k
            continue

        if n.kind == OpKind.REDUCE:
            k = Kernel("reduce", [n], anchor=n)
            src = n.inputs[0]
            pk = producer.get(id(src))
            if _prologue_source(pk, n, src, graph_outs):
                kernels.remove(pk)
                k.nodes = pk.nodes + [n]
                for m in pk.nodes:
                    producer[id(m)] = k
            kernels.append(k)
            producer[id(n)] = k
            continue

        if n.kind != OpKind.ELEMENTWISE:
            raise AssertionError(n.op)
        # join the kernel of the first operand whose producer accepts n
        target = None
        for src in n.inputs:
            pk = producer.get(id(resolve(src)))
            if pk is None or id(src) in aliases:
                continue      # graph inputs, consts and reshaped values are read, not fused through
            if pk.kind == "elementwise" and pk.iter_shape == n.shape:
                target = pk
            elif pk.kind in ("matmul", "reduce") and pk.anchor.shape == n.shape and _epilogue_ok(pk, n):
                target = pk
            if target is not None:
                break
        if target is not None and _no_cycle(target, n, producer, resolve):
            target.nodes.append(n)
            producer[id(n)] = target
        else:
            k = Kernel("elementwise", [n])
            kernels.append(k)
            producer[id(n)] = k

    for k in kernels:
        _finalize(k, g)
        _dedupe(k)
    return Program(g, _schedule(kernels, producer, resolve), aliases)


def _schedule(kernels: list[Kernel], producer: dict, resolve) -> list[Kernel]:
    """Order kernels by data dependence, sweeping the creation order repeatedly."""
    deps: dict[int, set[int]] = {}
    for k in kernels:
        needs = set()
        for i in k.inputs:
            src = resolve(i)
            if id(src) in producer:
                needs.add(id(producer[id(src)]))
        needs.discard(id(k))
        deps[id(k)] = needs
    order: list[Kernel] = []
    done: set[int] = set()
    pending = list(kernels)
    while pending:
        ready = False
        for k in list(pending):
            if deps[id(k)] <= done:
                order.append(k)
                done.add(id(k))
                pending.remove(k)
                ready = True
        if not ready:  # pragma: no cover
            raise RuntimeError("cyclic kernel dependency after fusion: " + ", ".join(repr(k) for k in pending))
    return order


# ---------------------------------------------------------------------------
# row fusion
# ---------------------------------------------------------------------------


def _row_class(k: Kernel):
    """``(rows, N, cls)`` for a kernel that is a per-row computation, else None."""
    if k.kind == "reduce":
        shape = k.anchor.inputs[0].shape
        return (shape[:-1], shape[-1], "red") if len(shape) >= 1 else None
    if k.kind == "elementwise":
        shape = k.iter_shape
        return (shape[:-1], shape[-1], "vec") if len(shape) >= 1 else None
    return None


def row_fuse(program: Program, max_n: int | None = None) -> Program:
    """Merge chains of per-row kernels with the same ``(rows, N)`` into ``row`` kernels."""
    kernels = program.kernels
    aliases = program.aliases
    resolve = _resolver(aliases)
    producer: dict[int, Kernel] = {id(o): k for k in kernels for o in k.outputs}

    # transitive kernel dependencies (used to refuse joins that would form a cycle)
    upstream: dict[int, set[int]] = {}
    for k in kernels:
        acc: set[int] = set()
        for i in k.inputs:
            p = producer.get(id(resolve(i)))
            if p is not None:
                acc.add(id(p))
                acc |= upstream.get(id(p), set())
        upstream[id(k)] = acc

    groups: list[list[Kernel]] = []
    group_of: dict[int, list[Kernel]] = {}
    for k in kernels:
        info = _row_class(k)
        eligible = info is not None and (max_n is None or info[1] <= max_n)
        joined = False
        if eligible:
            rows, n, cls = info
            for i in k.inputs:
                p = producer.get(id(resolve(i)))
                if p is None or id(p) not in group_of or id(i) in aliases:
                    continue
                grp = group_of[id(p)]
                if grp[0]._row != (rows, n):
                    continue
                if cls == "vec" and k.iter_shape not in (rows + (n,), rows + (1,), rows):
                    continue
                if not _reads_rows_per_row(k, grp, resolve, rows, n):
                    continue
                if not _joinable(k, grp, producer, upstream, resolve):
                    continue
                grp.append(k)
                group_of[id(k)] = grp
                joined = True
                break
        if joined:
            continue
        grp = [k]
        groups.append(grp)
        if eligible:
            k._row = (info[0], info[1])  # type: ignore[attr-defined]
            group_of[id(k)] = grp

    merged: list[Kernel] = []
    for grp in groups:
        if len(grp) == 1:
            merged.append(grp[0])
            continue
        rk = Kernel("row", nodes=[n for k in grp for n in k.nodes])
        rk.stages = grp  # type: ignore[attr-defined]
        rk.rows, rk.n = grp[0]._row  # type: ignore[attr-defined]
        _finalize(rk, program.graph)
        _dedupe(rk)
        merged.append(rk)
    producer2 = {id(o): k for k in merged for o in k.outputs}
    return Program(program.graph, _schedule(merged, producer2, resolve), aliases)


def _reads_rows_per_row(k: Kernel, grp: list[Kernel], resolve, rows: tuple, n: int) -> bool:
    """Every node of ``k`` that runs over whole rows (shape ``rows + (n,)``) reads the
    group's values whole-row or one per row (shape ``rows + (1,)``).  A per-row value of
    shape ``rows`` broadcasts along the *last* axis of ``rows + (n,)`` (numpy rules align
    trailing dims; possible when ``rows[-1] == n``), so it is a column value, which a row
    kernel, holding one value per row, would apply to the wrong elements.  The reference's
    ``row_fuse`` (``tensorjit/passes/fusion.py:290-295``) checks only the kernels' shapes
    and fuses such a pair: ``x - mean(x, axis=0) * g`` over a square ``x`` then subtracts
    each column's mean along its row.  Such a kernel stays out of the group here."""
    outs = {id(o) for g in grp for o in g.outputs}
    ok = {rows + (n,), rows + (1,)} | ({()} if rows == () else set())
    full = rows + (n,)
    for nd in k.nodes:
        if tuple(nd.shape) != full and not (nd is k.anchor and k.kind == "reduce"):
            continue
        for i in nd.inputs:
            if id(resolve(i)) in outs and tuple(i.shape) not in ok:
                return False
    return True


def _joinable(k: Kernel, grp: list[Kernel], producer: dict, upstream: dict, resolve) -> bool:
    """Every kernel-produced input of ``k`` comes from the group or from a kernel
    that does not itself depend on the group."""
    for j in k.inputs:
        pj = producer.get(id(resolve(j)))
        if pj is None or pj in grp:
            continue
        if any(id(m) in upstream[id(pj)] for m in grp):
            return False
    return True
