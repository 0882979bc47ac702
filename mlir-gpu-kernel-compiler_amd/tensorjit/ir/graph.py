"""SSA tensor IR.

A ``Graph`` is a list of ``Node`` objects in topological order.  Every node
produces one tensor with a static ``TensorType`` (shape and dtype), so the
backend can bake every size and stride into the generated kernel text.

Behaviour follows the reference IR (``tensorjit/ir/graph.py:26-278``):
the dtype set, the op table and its arities, numpy broadcasting, matmul with
an optional transposed B operand and broadcast batch dims, last-axis
reductions with ``keepdim`` and the movement ops.
"""
from __future__ import annotations

import enum
import hashlib
import itertools
from dataclasses import dataclass, field
from typing import Any, Optional, Sequence

Shape = tuple[int, ...]


class DType(str, enum.Enum):
    """Storage dtypes; every backend computes in fp32 (ref ``graph.py:26-42``)."""

    f32 = "f32"
    f16 = "f16"
    bf16 = "bf16"
    i32 = "i32"

    @property
    def itemsize(self) -> int:
        return _ITEMSIZE[self.value]

    @property
    def c_type(self) -> str:
        return _C_TYPE[self.value]

    @property
    def mlir(self) -> str:
        return self.value


_ITEMSIZE = {"f32": 4, "f16": 2, "bf16": 2, "i32": 4}
_C_TYPE = {"f32": "float", "f16": "_Float16", "bf16": "unsigned short", "i32": "int"}


@dataclass(frozen=True)
class TensorType:
    shape: Shape
    dtype: DType = DType.f32

    @property
    def rank(self) -> int:
        return len(self.shape)

    @property
    def numel(self) -> int:
        total = 1
        for d in self.shape:
            total *= d
        return total

    def __str__(self) -> str:
        dims = "x".join(str(d) for d in self.shape)
        return f"tensor<{dims}x{self.dtype.value}>"


class OpKind(enum.Enum):
    ELEMENTWISE = "elementwise"
    MATMUL = "matmul"
    REDUCE = "reduce"
    MOVEMENT = "movement"
    CONST = "const"
    INPUT = "input"


def _table() -> dict[str, tuple[OpKind, int]]:
    t: dict[str, tuple[OpKind, int]] = {"input": (OpKind.INPUT, 0), "const": (OpKind.CONST, 0)}
    for name in ("neg", "exp", "log", "sqrt", "rsqrt", "tanh", "relu", "sigmoid", "gelu", "silu", "abs"):
        t[name] = (OpKind.ELEMENTWISE, 1)
    for name in ("add", "sub", "mul", "div", "pow", "maximum", "minimum"):
        t[name] = (OpKind.ELEMENTWISE, 2)
    t["where"] = (OpKind.ELEMENTWISE, 3)
    t["matmul"] = (OpKind.MATMUL, 2)
    for name in ("sum", "max", "mean"):
        t[name] = (OpKind.REDUCE, 1)
    for name in ("reshape", "transpose", "broadcast_to"):
        t[name] = (OpKind.MOVEMENT, 1)
    return t


# op name -> (kind, arity).  Same op set as the reference (``graph.py:76-110``).
OPS: dict[str, tuple[OpKind, int]] = _table()

_counter = itertools.count()


@dataclass(eq=False)
class Node:
    """One SSA value.  Identity (``is``) is what matters; nodes are unhashable by value."""

    op: str
    inputs: list["Node"]
    type: TensorType
    attrs: dict[str, Any] = field(default_factory=dict)
    name: str = ""
    users: list["Node"] = field(default_factory=list, repr=False)
    meta: dict[str, Any] = field(default_factory=dict, repr=False)

    def __post_init__(self):
        if not self.name:
            self.name = f"%{self.op}{next(_counter)}"
        for src in self.inputs:
            src.users.append(self)

    @property
    def kind(self) -> OpKind:
        return OPS[self.op][0]

    @property
    def shape(self) -> Shape:
        return self.type.shape

    @property
    def dtype(self) -> DType:
        return self.type.dtype

    def replace_all_uses_with(self, other: "Node") -> None:
        for user in list(self.users):
            user.inputs = [other if x is self else x for x in user.inputs]
            other.users.append(user)
        self.users = []

    def __repr__(self) -> str:
        args = ", ".join(i.name for i in self.inputs)
        return f"{self.name} = {self.op}({args}) : {self.type}"


def broadcast_shapes(*shapes: Shape) -> Shape:
    """Numpy broadcasting of several shapes (right-aligned, 1 stretches)."""
    rank = max(len(s) for s in shapes)
    result = []
    for axis in range(rank):
        size = 1
        for s in shapes:
            k = axis - (rank - len(s))
            d = s[k] if k >= 0 else 1
            if d == 1:
                continue
            if size not in (1, d):
                raise ValueError(f"incompatible shapes for broadcasting: {shapes}")
            size = d
        result.append(size)
    return tuple(result)


class Graph:
    """Inputs, nodes (topological), outputs."""

    def __init__(self, name: str = "main"):
        self.name = name
        self.inputs: list[Node] = []
        self.nodes: list[Node] = []
        self.outputs: list[Node] = []

    def add_input(self, type: TensorType, name: Optional[str] = None) -> Node:
        node = Node("input", [], type, name=name or f"%arg{len(self.inputs)}")
        self.inputs.append(node)
        self.nodes.append(node)
        return node

    def const(self, value: float, dtype: DType = DType.f32, shape: Shape = ()) -> Node:
        node = Node("const", [], TensorType(shape, dtype), attrs={"value": float(value)})
        self.nodes.append(node)
        return node

    def create(self, op: str, inputs: Sequence[Node], **attrs) -> Node:
        _, arity = OPS[op]
        if arity and len(inputs) != arity:
            raise ValueError(f"{op} expects {arity} inputs, got {len(inputs)}")
        node = Node(op, list(inputs), infer_type(op, list(inputs), attrs), attrs=dict(attrs))
        self.nodes.append(node)
        return node

    def set_outputs(self, outs: Sequence[Node]) -> None:
        self.outputs = list(outs)

    def erase(self, node: Node) -> None:
        if node.users:
            raise AssertionError(f"cannot erase {node.name}: still has users")
        for src in node.inputs:
            src.users = [u for u in src.users if u is not node]
        self.nodes.remove(node)

    def toposort(self) -> None:
        """Depth-first post-order from every node in current order (stable)."""
        placed: set[int] = set()
        order: list[Node] = []
        for root in self.nodes:
            stack = [(root, False)]
            while stack:
                node, expanded = stack.pop()
                if expanded:
                    order.append(node)
                    continue
                if id(node) in placed:
                    continue
                placed.add(id(node))
                stack.append((node, True))
                for src in reversed(node.inputs):
                    if id(src) not in placed:
                        stack.append((src, False))
        self.nodes = order

    def signature(self) -> str:
        """Structural hash (ops, wiring, types, attrs, outputs)."""
        pos = {id(n): i for i, n in enumerate(self.nodes)}
        h = hashlib.sha256()
        for n in self.nodes:
            wiring = [pos[id(i)] for i in n.inputs]
            h.update(f"{n.op}|{wiring}|{n.type}|{sorted(n.attrs.items())}\n".encode())
        h.update(f"out|{[pos[id(o)] for o in self.outputs]}".encode())
        return h.hexdigest()[:16]

    def __str__(self) -> str:
        from .printer import print_graph

        return print_graph(self)


def infer_type(op: str, inputs: list[Node], attrs: dict) -> TensorType:
    kind = OPS[op][0]
    if kind == OpKind.ELEMENTWISE:
        shape = broadcast_shapes(*(i.shape for i in inputs))
        dtypes = {i.dtype for i in inputs if i.op != "const"} or {inputs[0].dtype}
        if len(dtypes) != 1:
            raise TypeError(f"{op}: mixed dtypes {dtypes}")
        return TensorType(shape, dtypes.pop())
    if kind == OpKind.MATMUL:
        a, b = inputs
        trans_b = bool(attrs.get("trans_b"))
        if a.type.rank < 2 or b.type.rank < 2:
            raise ValueError(f"matmul shape mismatch {a.shape} @ {b.shape} (trans_b={trans_b})")
        kb, n = (b.shape[-1], b.shape[-2]) if trans_b else (b.shape[-2], b.shape[-1])
        if a.shape[-1] != kb:
            raise ValueError(f"matmul shape mismatch {a.shape} @ {b.shape} (trans_b={trans_b})")
        batch = broadcast_shapes(a.shape[:-2], b.shape[:-2])
        return TensorType(batch + (a.shape[-2], n), a.dtype)
    if kind == OpKind.REDUCE:
        (x,) = inputs
        axis = attrs.get("axis", -1)
        if axis not in (-1, x.type.rank - 1):
            raise NotImplementedError("reductions are supported over the last axis only")
        tail = (1,) if attrs.get("keepdim", False) else ()
        return TensorType(x.shape[:-1] + tail, x.dtype)
    if kind == OpKind.MOVEMENT:
        (x,) = inputs
        if op == "reshape":
            shape = tuple(attrs["shape"])
            if -1 in shape:
                known = 1
                for d in shape:
                    if d != -1:
                        known *= d
                shape = tuple(x.type.numel // known if d == -1 else d for d in shape)
            if TensorType(shape).numel != x.type.numel:
                raise AssertionError("reshape numel mismatch")
            return TensorType(shape, x.dtype)
        if op == "transpose":
            return TensorType(tuple(x.shape[p] for p in attrs["perm"]), x.dtype)
        if op == "broadcast_to":
            return TensorType(tuple(attrs["shape"]), x.dtype)
    raise NotImplementedError(op)
