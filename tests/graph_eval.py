"""Float64 evaluation of a traced tensorjit graph, node by node, with torch.

Test infrastructure: no fusion, no plan, no generated code -- each IR node evaluated by
its definition (numpy broadcasting for elementwise ops, reductions over the last axis
with or without keepdim, matmul with an optional transposed right operand, transpose,
reshape).  It checks the whole pipeline (fusion plan and oracle code generation alike)
against the ops' meaning: the parity tests compare the hip path with an oracle that
shares its plan, so only an evaluation without a plan can show a plan that computes the
wrong thing.  gelu is the erf form, sigmoid / silu / exp the exact functions."""
from __future__ import annotations

import math

import torch

_UNARY = {
    "neg": torch.neg, "exp": torch.exp, "log": torch.log, "sqrt": torch.sqrt, "rsqrt": torch.rsqrt,
    "tanh": torch.tanh, "relu": torch.relu, "sigmoid": torch.sigmoid, "abs": torch.abs,
    "gelu": lambda x: 0.5 * x * (1.0 + torch.erf(x / math.sqrt(2.0))),
    "silu": lambda x: x * torch.sigmoid(x),
}
_BINARY = {
    "add": torch.add, "sub": torch.sub, "mul": torch.mul, "div": torch.div, "pow": torch.pow,
    "maximum": torch.maximum, "minimum": torch.minimum,
}


def evaluate(graph, *inputs: torch.Tensor) -> list[torch.Tensor]:
    """The graph's outputs for ``inputs``, computed in float64."""
    val: dict[int, torch.Tensor] = {}
    for n, x in zip(graph.inputs, inputs):
        val[id(n)] = x.double()
    for n in graph.nodes:
        if id(n) in val:
            continue
        a = [val[id(i)] for i in n.inputs]
        op = n.op
        if op == "const":
            v = torch.tensor(float(n.attrs["value"]), dtype=torch.float64).expand(tuple(n.shape))
        elif op in _UNARY:
            v = _UNARY[op](a[0])
        elif op in _BINARY:
            v = _BINARY[op](a[0], a[1])
        elif op == "where":
            v = torch.where(a[0] != 0, a[1], a[2])
        elif op in ("sum", "mean", "max", "min"):
            assert n.attrs.get("axis", -1) in (-1, len(n.inputs[0].shape) - 1), n.attrs
            keep = bool(n.attrs.get("keepdim", False))
            if op == "sum":
                v = a[0].sum(-1, keepdim=keep)
            elif op == "mean":
                v = a[0].mean(-1, keepdim=keep)
            else:
                v = getattr(a[0], "amax" if op == "max" else "amin")(-1, keepdim=keep)
        elif op == "matmul":
            b = a[1].transpose(-1, -2) if n.attrs.get("trans_b") else a[1]
            v = torch.matmul(a[0], b)
        elif op == "transpose":
            v = a[0].permute(*n.attrs["perm"])
        elif op == "reshape":
            v = a[0].reshape(tuple(n.shape))
        else:
            raise NotImplementedError(op)
        assert tuple(v.shape) == tuple(n.shape), (op, tuple(v.shape), tuple(n.shape))
        val[id(n)] = v
    return [val[id(o)] for o in graph.outputs]
