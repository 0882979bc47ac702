"""Graph cleanups run to a fixed point before fusion.

Same rewrite set and the same visiting order as the reference
(``tensorjit/passes/cleanup.py:10-170``): DCE, CSE, scalar constant folding
and algebraic identities, implicit broadcasts, reshape chains and
transpose-into-matmul folding.  The order matters because fusion is greedy
over the resulting node order.
"""
from __future__ import annotations

import math

from ..ir import Graph, Node, OpKind


def dce(g: Graph) -> bool:
    """Erase nodes nobody reads (graph inputs and outputs are always kept)."""
    keep = {id(n) for n in g.outputs} | {id(n) for n in g.inputs}
    changed = False
    for node in reversed(list(g.nodes)):
        if id(node) not in keep and not node.users:
            g.erase(node)
            changed = True
    return changed


def _cse_key(n: Node) -> tuple:
    return (n.op, tuple(id(i) for i in n.inputs), n.type, tuple(sorted(n.attrs.items())))


def cse(g: Graph) -> bool:
    """Replace a node by an earlier node with identical op, operands, type and attrs."""
    first: dict[tuple, Node] = {}
    changed = False
    for node in list(g.nodes):
        if node.op == "input":
            continue
        key = _cse_key(node)
        keep = first.get(key)
        if keep is None:
            first[key] = node
            continue
        node.replace_all_uses_with(keep)
        g.outputs = [keep if o is node else o for o in g.outputs]
        g.erase(node)
        changed = True
    return changed


def _gelu(x: float) -> float:
    return 0.5 * x * (1.0 + math.erf(x / math.sqrt(2.0)))


_FOLD_UNARY = {
    "neg": lambda x: -x,
    "exp": math.exp,
    "log": math.log,
    "sqrt": math.sqrt,
    "rsqrt": lambda x: 1.0 / math.sqrt(x),
    "tanh": math.tanh,
    "relu": lambda x: max(x, 0.0),
    "sigmoid": lambda x: 1.0 / (1.0 + math.exp(-x)),
    "abs": abs,
    "gelu": _gelu,
    "silu": lambda x: x / (1.0 + math.exp(-x)),
}
_FOLD_BINARY = {
    "add": lambda a, b: a + b,
    "sub": lambda a, b: a - b,
    "mul": lambda a, b: a * b,
    "div": lambda a, b: a / b,
    "pow": lambda a, b: a**b,
    "maximum": max,
    "minimum": min,
}


def _scalar_const(n: Node, value=None) -> bool:
    return n.op == "const" and n.shape == () and (value is None or n.attrs["value"] == value)


def _substitute(g: Graph, old: Node, new: Node) -> None:
    old.replace_all_uses_with(new)
    g.outputs = [new if o is old else o for o in g.outputs]
    if not old.users and old not in g.outputs:
        g.erase(old)


def _identity_of(g: Graph, n: Node) -> Node | None:
    """x+0, x-0, 0+x, x*1, x/1, 1*x -> x (only when no broadcast is lost); scalar x*0 -> 0."""
    a, b = n.inputs
    if n.op in ("add", "sub") and _scalar_const(b, 0.0) and a.shape == n.shape:
        return a
    if n.op == "add" and _scalar_const(a, 0.0) and b.shape == n.shape:
        return b
    if n.op in ("mul", "div") and _scalar_const(b, 1.0) and a.shape == n.shape:
        return a
    if n.op == "mul" and _scalar_const(a, 1.0) and b.shape == n.shape:
        return b
    if n.op == "mul" and n.shape == () and (_scalar_const(a, 0.0) or _scalar_const(b, 0.0)):
        # only scalars: kernels take scalar constants, not constant tensors
        return g.const(0.0, n.dtype, n.shape)
    return None


def algebraic_simplify(g: Graph) -> bool:
    changed = False
    for n in list(g.nodes):
        fold = _FOLD_UNARY.get(n.op) or _FOLD_BINARY.get(n.op)
        if fold is None:
            continue
        if all(_scalar_const(i) for i in n.inputs):
            try:
                value = fold(*(i.attrs["value"] for i in n.inputs))
            except (ValueError, ZeroDivisionError, OverflowError):
                continue
            _substitute(g, n, g.const(value, n.dtype, n.shape))
            changed = True
            continue
        if n.op in _FOLD_BINARY:
            repl = _identity_of(g, n)
            if repl is not None:
                _substitute(g, n, repl)
                changed = True
                continue
        src = n.inputs[0]
        if (n.op, src.op) in (("neg", "neg"), ("exp", "log")):
            _substitute(g, n, src.inputs[0])
            changed = True
    return changed


def fold_broadcast(g: Graph) -> bool:
    """A broadcast_to read only by elementwise ops is implicit in their indexing."""
    changed = False
    for n in list(g.nodes):
        if n.op == "broadcast_to" and n not in g.outputs and all(u.kind == OpKind.ELEMENTWISE for u in n.users):
            _substitute(g, n, n.inputs[0])
            changed = True
    return changed


def fold_reshape_chains(g: Graph) -> bool:
    """reshape to the same shape -> source; reshape of a single-use reshape -> one reshape."""
    changed = False
    for n in list(g.nodes):
        if n.op != "reshape":
            continue
        src = n.inputs[0]
        if src.shape == n.shape:
            _substitute(g, n, src)
            changed = True
        elif src.op == "reshape" and len(src.users) == 1:
            _substitute(g, n, g.create("reshape", [src.inputs[0]], shape=n.shape))
            changed = True
    return changed


def fold_transpose_into_matmul(g: Graph) -> bool:
    """matmul(a, transpose(b) swapping the last two dims) -> matmul(a, b, trans_b=True).

    This is the ``x @ w.T`` layout of ``nn.Linear``: B is then read K-contiguous
    straight from the weight instead of through a materialised transpose.
    """
    changed = False
    for n in list(g.nodes):
        if n.op != "matmul" or n.attrs.get("trans_b"):
            continue
        t = n.inputs[1]
        r = t.type.rank
        if t.op != "transpose" or tuple(t.attrs["perm"]) != tuple(range(r - 2)) + (r - 1, r - 2):
            continue
        src = t.inputs[0]
        t.users = [u for u in t.users if u is not n]
        n.inputs[1] = src
        src.users.append(n)
        n.attrs["trans_b"] = True
        changed = True
    return changed
