"""Python tracing frontend.

``tj.jit`` runs the user's function once per input signature on ``Tensor``
proxies.  Each proxy operation appends one node to the thread's active
``Graph``.  The composites (softmax, layer_norm, rms_norm, linear) expand
into primitives in the same order as the reference tracer
(``tensorjit/frontend/tracer.py:176-206``), because that order decides what
the fusion passes produce.
"""
from __future__ import annotations

import builtins
import threading
from typing import Callable, Sequence

import torch

from ..ir import DType, Graph, Node, TensorType
from ..runtime.dtypes import FROM_TORCH

_state = threading.local()


def _active() -> Graph:
    g = getattr(_state, "graph", None)
    if g is None:
        raise RuntimeError("tensorjit ops must be used inside a traced (@tensorjit.jit) function")
    return g


class Tensor:
    """Symbolic tensor; every operation records a node in the active graph."""

    __array_priority__ = 1000

    def __init__(self, node: Node):
        self.node = node

    @property
    def shape(self) -> tuple[int, ...]:
        return self.node.shape

    @property
    def dtype(self) -> DType:
        return self.node.dtype

    @property
    def ndim(self) -> int:
        return len(self.node.shape)

    def __repr__(self) -> str:
        return f"tj.Tensor({self.node.name}: {self.node.type})"

    def __add__(self, o):
        return _binary("add", self, o)

    def __radd__(self, o):
        return _binary("add", o, self)

    def __sub__(self, o):
        return _binary("sub", self, o)

    def __rsub__(self, o):
        return _binary("sub", o, self)

    def __mul__(self, o):
        return _binary("mul", self, o)

    def __rmul__(self, o):
        return _binary("mul", o, self)

    def __truediv__(self, o):
        return _binary("div", self, o)

    def __rtruediv__(self, o):
        return _binary("div", o, self)

    def __pow__(self, o):
        return _binary("pow", self, o)

    def __neg__(self):
        return _unary("neg", self)

    def __matmul__(self, o):
        return matmul(self, o)

    def exp(self):
        return _unary("exp", self)

    def log(self):
        return _unary("log", self)

    def sqrt(self):
        return _unary("sqrt", self)

    def rsqrt(self):
        return _unary("rsqrt", self)

    def tanh(self):
        return _unary("tanh", self)

    def abs(self):
        return _unary("abs", self)

    def relu(self):
        return _unary("relu", self)

    def sigmoid(self):
        return _unary("sigmoid", self)

    def sum(self, axis=-1, keepdim=False):
        return reduce("sum", self, axis, keepdim)

    def max(self, axis=-1, keepdim=False):
        return reduce("max", self, axis, keepdim)

    def mean(self, axis=-1, keepdim=False):
        return reduce("mean", self, axis, keepdim)

    def reshape(self, *shape):
        return reshape(self, *shape)

    def view(self, *shape):
        return reshape(self, *shape)

    def transpose(self, a: int, b: int):
        return transpose(self, a, b)

    def permute(self, *perm):
        return permute(self, *perm)

    @property
    def T(self):
        if self.ndim != 2:
            raise AssertionError(".T needs a 2-D tensor")
        return permute(self, 1, 0)


def _operand(x, like: Tensor | None) -> Node:
    """Proxy -> its node; a Python scalar -> a fresh scalar const of the proxy's dtype."""
    if isinstance(x, Tensor):
        return x.node
    if isinstance(x, (bool, int, float)):
        return _active().const(float(x), like.dtype if like is not None else DType.f32)
    raise TypeError(f"unsupported operand {type(x)}")


def _binary(op: str, a, b) -> Tensor:
    like = a if isinstance(a, Tensor) else b
    lhs = _operand(a, like)
    rhs = _operand(b, like)
    return Tensor(_active().create(op, [lhs, rhs]))


def _unary(op: str, a: Tensor) -> Tensor:
    return Tensor(_active().create(op, [a.node]))


def exp(x):
    return _unary("exp", x)


def log(x):
    return _unary("log", x)


def sqrt(x):
    return _unary("sqrt", x)


def rsqrt(x):
    return _unary("rsqrt", x)


def tanh(x):
    return _unary("tanh", x)


def abs(x):  # noqa: A001
    return _unary("abs", x)


def relu(x):
    return _unary("relu", x)


def sigmoid(x):
    return _unary("sigmoid", x)


def gelu(x):
    return _unary("gelu", x)


def silu(x):
    return _unary("silu", x)


def maximum(a, b):
    return _binary("maximum", a, b)


def minimum(a, b):
    return _binary("minimum", a, b)


def where(c, a, b):
    like = next(t for t in (c, a, b) if isinstance(t, Tensor))
    ops = [_operand(c, like), _operand(a, like), _operand(b, like)]
    return Tensor(_active().create("where", ops))


def matmul(a: Tensor, b: Tensor) -> Tensor:
    return Tensor(_active().create("matmul", [a.node, b.node]))


def reduce(op: str, x: Tensor, axis: int = -1, keepdim: bool = False) -> Tensor:
    """Last-axis reduction; another axis is first moved last by a transpose."""
    if axis < 0:
        axis += x.ndim
    if axis != x.ndim - 1:
        order = [d for d in range(x.ndim) if d != axis] + [axis]
        x = permute(x, *order)
    return Tensor(_active().create(op, [x.node], axis=-1, keepdim=keepdim))


def sum(x, axis=-1, keepdim=False):  # noqa: A001
    return reduce("sum", x, axis, keepdim)


def max(x, axis=-1, keepdim=False):  # noqa: A001
    return reduce("max", x, axis, keepdim)


def mean(x, axis=-1, keepdim=False):
    return reduce("mean", x, axis, keepdim)


def reshape(x: Tensor, *shape) -> Tensor:
    if len(shape) == 1 and isinstance(shape[0], (tuple, list)):
        shape = tuple(shape[0])
    return Tensor(_active().create("reshape", [x.node], shape=tuple(int(s) for s in shape)))


def permute(x: Tensor, *perm) -> Tensor:
    if len(perm) == 1 and isinstance(perm[0], (tuple, list)):
        perm = tuple(perm[0])
    perm = tuple(p % x.ndim for p in perm)
    if perm == tuple(range(x.ndim)):
        return x
    return Tensor(_active().create("transpose", [x.node], perm=perm))


def transpose(x: Tensor, a: int, b: int) -> Tensor:
    order = list(range(x.ndim))
    i, j = a % x.ndim, b % x.ndim
    order[i], order[j] = order[j], order[i]
    return permute(x, *order)


def broadcast_to(x: Tensor, shape) -> Tensor:
    return Tensor(_active().create("broadcast_to", [x.node], shape=tuple(shape)))


def _tag(root: Tensor, op: str, args: list, **params) -> Tensor:
    """Record which composite produced ``root`` (non-semantic metadata)."""
    root.node.meta["composite"] = {"op": op, "args": [a.node for a in args if a is not None], **params}
    return root


def softmax(x: Tensor, axis: int = -1) -> Tensor:
    if axis not in (-1, x.ndim - 1):
        raise AssertionError("softmax over last axis")
    e = exp(x - reduce("max", x, -1, keepdim=True))
    return _tag(e / reduce("sum", e, -1, keepdim=True), "softmax", [x])


def layer_norm(x: Tensor, weight: Tensor | None = None, bias: Tensor | None = None, eps: float = 1e-5) -> Tensor:
    centered = x - reduce("mean", x, -1, keepdim=True)
    var = reduce("mean", centered * centered, -1, keepdim=True)
    y = centered * rsqrt(var + eps)
    if weight is not None:
        y = y * weight
    if bias is not None:
        y = y + bias
    return _tag(y, "layer_norm", [x, weight, bias], eps=eps, has_weight=weight is not None, has_bias=bias is not None)


def rms_norm(x: Tensor, weight: Tensor | None = None, eps: float = 1e-6) -> Tensor:
    y = x * rsqrt(reduce("mean", x * x, -1, keepdim=True) + eps)
    if weight is not None:
        y = y * weight
    return _tag(y, "rms_norm", [x, weight], eps=eps, has_weight=weight is not None)


def linear(x: Tensor, w: Tensor, b: Tensor | None = None) -> Tensor:
    """``x @ w.T (+ b)`` with ``w`` stored ``[out, in]`` as in ``torch.nn.Linear``."""
    y = matmul(x, w.T)
    if b is not None:
        y = y + b
    return _tag(y, "linear", [x, w, b], has_bias=b is not None)


def trace(fn: Callable, arg_types: Sequence[TensorType], name: str = "main") -> Graph:
    g = Graph(name)
    saved = getattr(_state, "graph", None)
    _state.graph = g
    try:
        params = [Tensor(g.add_input(t)) for t in arg_types]
        result = fn(*params)
        outs = result if isinstance(result, (tuple, list)) else (result,)
        if not builtins.all(isinstance(o, Tensor) for o in outs):
            raise TypeError("jit functions must return tensors (or a tuple of them)")
        g.set_outputs([o.node for o in outs])
    finally:
        _state.graph = saved
    g.toposort()
    return g


def tensor_type_of(t: torch.Tensor) -> TensorType:
    return TensorType(tuple(t.shape), FROM_TORCH[t.dtype])
