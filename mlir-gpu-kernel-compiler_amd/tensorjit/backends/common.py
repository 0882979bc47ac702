"""Shared codegen helpers: strides of broadcast / transposed reads, linear-index
offset expressions and the fp32 expression table of the HIP backend.

Stride rules are the reference's (``tensorjit/backends/common.py:10-35``):
row-major contiguous strides, stride 0 on broadcast dims, permuted strides
for a transpose consumer.  Offsets are generated differently: dims whose
strides chain contiguously are merged first, so each input costs one
division/modulo per merged dim instead of one per dim.
"""
from __future__ import annotations

import math

from ..ir import Node, OpKind

Shape = tuple[int, ...]


def contiguous_strides(shape: Shape) -> tuple[int, ...]:
    out = []
    step = 1
    for d in reversed(shape):
        out.append(step)
        step *= d
    return tuple(reversed(out))


def broadcast_strides(in_shape: Shape, iter_shape: Shape) -> tuple[int, ...]:
    """Strides that read a contiguous ``in_shape`` tensor at each point of ``iter_shape``."""
    cs = contiguous_strides(in_shape)
    lead = len(iter_shape) - len(in_shape)
    return (0,) * lead + tuple(
        0 if in_shape[d] == 1 and iter_shape[lead + d] != 1 else cs[d] for d in range(len(in_shape)))


def access_strides(inp: Node, consumer: Node, iter_shape: Shape) -> tuple[int, ...]:
    """How ``consumer`` reads ``inp`` while iterating ``iter_shape``."""
    if consumer.op == "transpose":
        cs = contiguous_strides(inp.shape)
        return tuple(cs[p] for p in consumer.attrs["perm"])
    return broadcast_strides(inp.shape, iter_shape)


def index_expr(idx_vars: list[str], strides: tuple[int, ...]) -> str:
    terms = [v if s == 1 else f"{v}*{s}" for v, s in zip(idx_vars, strides) if s != 0]
    return " + ".join(terms) if terms else "0"


def merged_dims(shape: Shape, strides: tuple[int, ...]) -> list[tuple[int, int, int]]:
    """``[(extent, inner_extent, stride)]`` from innermost to outermost after merging
    adjacent dims whose strides chain (or are both zero).  ``inner_extent`` is the
    product of the iteration sizes of every dim inside the group."""
    groups: list[list[int]] = []   # [extent, inner, stride]
    inner = 1
    for size, st in zip(reversed(shape), reversed(strides)):
        if size == 1:
            continue
        if groups:
            g = groups[-1]
            if (st == 0 and g[2] == 0) or (g[2] != 0 and st == g[2] * g[0]):
                g[0] *= size
                inner *= size
                continue
        groups.append([size, inner, st])
        inner *= size
    return [tuple(g) for g in groups]  # type: ignore[misc]


def offset_expr(linear: str, shape: Shape, strides: tuple[int, ...]) -> str:
    """Offset of the element at row-major linear index ``linear`` of ``shape``."""
    groups = merged_dims(shape, strides)
    total = math.prod(shape) if shape else 1
    terms = []
    for extent, inner, st in groups:
        if st == 0:
            continue
        idx = linear if inner == 1 else f"({linear} / {inner}u)"
        if inner * extent < total:
            idx = f"({idx} % {extent}u)"
        terms.append(idx if st == 1 else f"{idx} * {st}u")
    return " + ".join(terms) if terms else "0u"


def inner_stride(shape: Shape, strides: tuple[int, ...]) -> int:
    """Stride of the innermost non-unit iteration dim (0 if every dim is broadcast)."""
    for size, st in zip(reversed(shape), reversed(strides)):
        if size != 1:
            return st
    return 0


# fp32 expressions.  exp / sigmoid / silu / gelu use the native-unit helpers of the
# device prelude (tj_exp, tj_rcp, A&S 7.1.26 tj_erf): each is within a few ulp (erf
# within 1.5e-7 absolute), far inside the 1e-5 relative parity bound, and keeps
# HBM-bound pointwise kernels off the VALU limit.  ``div`` is IEEE division
# (correctly rounded, as in the reference's expression table): int32 storage
# truncates the fp32 quotient, and a*rcp(b) would turn exact quotients such as
# 41/41 into 0.99999994 -> 0; the hardware reciprocal also flushes 1/b to zero
# for |b| > 2^126.
HIP_EXPR = {
    "neg": "(-{0})",
    "exp": "tj_exp({0})",
    "log": "logf({0})",
    "sqrt": "sqrtf({0})",
    "rsqrt": "(1.0f / sqrtf({0}))",
    "tanh": "tanhf({0})",
    "relu": "fmaxf({0}, 0.0f)",
    "sigmoid": "tj_sigmoid({0})",
    "gelu": "tj_gelu({0})",
    "silu": "({0} * tj_sigmoid({0}))",
    "abs": "fabsf({0})",
    "add": "({0} + {1})",
    "sub": "({0} - {1})",
    "mul": "({0} * {1})",
    "div": "({0} / {1})",
    "pow": "powf({0}, {1})",
    "maximum": "fmaxf({0}, {1})",
    "minimum": "fminf({0}, {1})",
    "where": "(({0}) != 0.0f ? ({1}) : ({2}))",
}


def scalar_literal(v: float) -> str:
    if v != v:
        return "__builtin_nanf(\"\")"
    if v in (math.inf, -math.inf):
        return "(-__builtin_inff())" if v < 0 else "__builtin_inff()"
    return f"{v!r}f"


def emit_expr(node: Node, operand: dict[int, str]) -> str:
    """fp32 HIP expression for one elementwise node; scalar consts are inlined."""
    if node.kind != OpKind.ELEMENTWISE:
        raise AssertionError(node.op)
    args = [scalar_literal(i.attrs["value"]) if i.op == "const" and i.shape == () else operand[id(i)]
            for i in node.inputs]
    return HIP_EXPR[node.op].format(*args)
