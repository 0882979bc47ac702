"""``torch.compile`` backend.

    compiled = torch.compile(model, backend=tensorjit.torch_compile_backend)

Dynamo hands over an FX ``GraphModule`` and example inputs.  The supported
subset is translated into tensorjit IR through the tracer's proxy ops and
compiled for the inputs' device; a graph with an unsupported op runs eagerly
instead (``TENSORJIT_STRICT=1`` raises).  Same op coverage, parameter
handling and fallback rule as the reference
(``tensorjit/frontend/torch_backend.py:116-262``).
"""
from __future__ import annotations

import logging
import operator
import os
from typing import Callable

import torch
import torch.fx as fx
import torch.nn.functional as F

from ..compiler import compile_graph, pick_backend
from ..ir import Graph
from . import tracer as T
from .tracer import Tensor, tensor_type_of

log = logging.getLogger("tensorjit")


class Unsupported(Exception):
    pass


def _unsupported(what: str):
    raise Unsupported(what)


def _reduce_dim(x: Tensor, dim, keepdim: bool, op: str):
    if isinstance(dim, (list, tuple)):
        if len(dim) != 1:
            raise Unsupported("multi-dim reductions")
        dim = dim[0]
    if dim is None:
        x = T.reshape(x, -1)
        dim = -1
    return T.reduce(op, x, dim, keepdim)


def _softmax(x, dim=-1, *_, **__):
    if dim not in (-1, x.ndim - 1):
        raise Unsupported("softmax over non-last dim")
    return T.softmax(x)


def _layer_norm(x, normalized_shape, weight=None, bias=None, eps=1e-5, **_):
    if tuple(normalized_shape) != (x.shape[-1],):
        raise Unsupported("layer_norm over multiple dims")
    return T.layer_norm(x, weight, bias, eps)


def _expand(x, *shape):
    if len(shape) == 1 and isinstance(shape[0], (tuple, list)):
        shape = tuple(shape[0])
    return T.broadcast_to(x, tuple(x.shape[i] if s == -1 else s for i, s in enumerate(shape)))


def _scaled(b, alpha):
    return b * alpha if alpha != 1 else b


def _max(x, dim=None, keepdim=False, **_):
    if dim is None:
        return _reduce_dim(x, None, False, "max")
    raise Unsupported("torch.max with dim returns (values, indices)")


def _dropout_fn(x, p=0.5, training=False, inplace=False):
    return _unsupported("dropout(train)") if training else x


def _mean(x, dim=None, keepdim=False, **_):
    return _reduce_dim(x, dim, keepdim, "mean")


def _sum(x, dim=None, keepdim=False, **_):
    return _reduce_dim(x, dim, keepdim, "sum")


def _amax(x, dim=-1, keepdim=False, **_):
    return _reduce_dim(x, dim, keepdim, "max")


FUNCTION_MAP: dict[object, Callable] = {
    operator.add: lambda a, b: a + b,
    operator.sub: lambda a, b: a - b,
    operator.mul: lambda a, b: a * b,
    operator.truediv: lambda a, b: a / b,
    operator.neg: lambda a: -a,
    operator.pow: lambda x, e: x ** e,
    operator.matmul: T.matmul,
    torch.add: lambda a, b, alpha=1: a + _scaled(b, alpha),
    torch.sub: lambda a, b, alpha=1: a - _scaled(b, alpha),
    torch.mul: lambda a, b: a * b,
    torch.div: lambda a, b: a / b,
    torch.neg: lambda a: -a,
    torch.pow: lambda x, e: x ** e,
    torch.matmul: T.matmul,
    torch.mm: T.matmul,
    torch.bmm: T.matmul,
    torch.exp: T.exp,
    torch.log: T.log,
    torch.sqrt: T.sqrt,
    torch.rsqrt: T.rsqrt,
    torch.tanh: T.tanh,
    torch.abs: T.abs,
    torch.sigmoid: T.sigmoid,
    torch.relu: T.relu,
    torch.maximum: T.maximum,
    torch.minimum: T.minimum,
    torch.where: T.where,
    torch.clamp_min: T.maximum,
    # FX records the defaulted ``inplace`` flag of the activations; it has no meaning here
    F.relu: lambda x, inplace=False: T.relu(x),
    F.gelu: lambda x, approximate="none": T.gelu(x) if approximate == "none" else _unsupported("gelu(tanh)"),
    F.silu: lambda x, inplace=False: T.silu(x),
    F.sigmoid: T.sigmoid,
    F.tanh: T.tanh,
    F.softmax: _softmax,
    torch.softmax: _softmax,
    F.layer_norm: _layer_norm,
    F.linear: lambda x, w, b=None: T.linear(x, w, b),
    torch.sum: _sum,
    torch.mean: _mean,
    torch.amax: _amax,
    torch.max: _max,
    F.dropout: _dropout_fn,
    torch.dropout: lambda x, p, train: _unsupported("dropout(train)") if train else x,
    torch.transpose: lambda x, d0, d1: T.transpose(x, d0, d1),
    torch.permute: lambda x, *dims: T.permute(x, *dims),
    torch.reshape: lambda x, *shape: T.reshape(x, *shape),
    torch.t: lambda x: x.T,
}

METHOD_MAP: dict[str, Callable | None] = {
    "add": FUNCTION_MAP[torch.add], "sub": FUNCTION_MAP[torch.sub], "mul": FUNCTION_MAP[torch.mul],
    "div": FUNCTION_MAP[torch.div], "neg": FUNCTION_MAP[torch.neg], "pow": FUNCTION_MAP[torch.pow],
    "matmul": T.matmul, "mm": T.matmul, "bmm": T.matmul,
    "exp": T.exp, "log": T.log, "sqrt": T.sqrt, "rsqrt": T.rsqrt, "tanh": T.tanh, "abs": T.abs,
    "sigmoid": T.sigmoid, "relu": T.relu, "softmax": _softmax,
    "sum": _sum, "mean": _mean, "amax": _amax, "max": _max,
    "transpose": FUNCTION_MAP[torch.transpose], "permute": FUNCTION_MAP[torch.permute],
    "view": FUNCTION_MAP[torch.reshape], "reshape": FUNCTION_MAP[torch.reshape], "expand": _expand,
    "t": lambda x: x.T, "contiguous": lambda x: x, "clone": lambda x: x, "float": lambda x: x,
    "clamp_min": T.maximum, "size": None, "dim": None,
}


def fx_to_graph(gm: fx.GraphModule, example_inputs) -> tuple[Graph, list]:
    """FX graph -> IR.  Returns the graph and, per IR input, where its tensor comes
    from at call time: a placeholder index or ``("attr", qualified_name)``."""
    params = dict(gm.named_parameters())
    params.update(dict(gm.named_buffers()))
    sources: list = []
    g = Graph(name="fx_graph")

    def new_input(t: torch.Tensor, name: str, source) -> Tensor:
        sources.append(source)
        return Tensor(g.add_input(tensor_type_of(t), name=name))

    def translate() -> list:
        env: dict[str, object] = {}
        placeholders = [n for n in gm.graph.nodes if n.op == "placeholder"]
        for i, (n, ex) in enumerate(zip(placeholders, example_inputs)):
            env[n.name] = new_input(ex, f"%{n.name}", i) if isinstance(ex, torch.Tensor) else ex
        result = None
        for n in gm.graph.nodes:
            if n.op == "placeholder":
                continue
            args = fx.node.map_arg(n.args, lambda a: env[a.name])
            kwargs = fx.node.map_arg(n.kwargs, lambda a: env[a.name])
            if n.op == "get_attr":
                p = params.get(n.target)
                if p is None:
                    raise Unsupported(f"get_attr {n.target}")
                env[n.name] = new_input(p, f"%{n.target.replace('.', '_')}", ("attr", n.target))
            elif n.op == "call_function":
                fn = FUNCTION_MAP.get(n.target)
                if fn is None:
                    raise Unsupported("getattr" if n.target is getattr else f"function {n.target}")
                env[n.name] = fn(*args, **kwargs)
            elif n.op == "call_method":
                fn = METHOD_MAP.get(n.target)
                if fn is None:
                    raise Unsupported(f"method {n.target}")
                env[n.name] = fn(*args, **kwargs)
            elif n.op == "call_module":
                env[n.name] = module_call(gm.get_submodule(n.target), n.target, args)
            elif n.op == "output":
                result = args[0]
            else:
                raise Unsupported(n.op)
        outs = result if isinstance(result, (tuple, list)) else (result,)
        if not all(isinstance(o, Tensor) for o in outs):
            raise Unsupported("non-tensor output")
        return [o.node for o in outs]

    def module_call(mod: torch.nn.Module, target: str, args):
        if isinstance(mod, torch.nn.Linear):
            w = new_input(mod.weight, f"%{target}_w", ("attr", f"{target}.weight"))
            b = new_input(mod.bias, f"%{target}_b", ("attr", f"{target}.bias")) if mod.bias is not None else None
            return T.linear(args[0], w, b)
        if isinstance(mod, torch.nn.LayerNorm):
            w = new_input(mod.weight, f"%{target}_w", ("attr", f"{target}.weight")) if mod.weight is not None else None
            b = new_input(mod.bias, f"%{target}_b", ("attr", f"{target}.bias")) if mod.bias is not None else None
            return _layer_norm(args[0], mod.normalized_shape, w, b, mod.eps)
        acts = {torch.nn.GELU: T.gelu, torch.nn.ReLU: T.relu, torch.nn.SiLU: T.silu, torch.nn.Sigmoid: T.sigmoid,
                torch.nn.Tanh: T.tanh}
        if type(mod) in acts:
            return acts[type(mod)](args[0])
        if isinstance(mod, torch.nn.Dropout):
            return args[0]
        raise Unsupported(f"module {type(mod).__name__}")

    saved = getattr(T._state, "graph", None)
    T._state.graph = g
    try:
        g.set_outputs(translate())
    finally:
        T._state.graph = saved
    g.toposort()
    return g, sources


def torch_compile_backend(gm: fx.GraphModule, example_inputs: list):
    """Entry point for ``torch.compile(..., backend=tensorjit.torch_compile_backend)``."""
    strict = os.environ.get("TENSORJIT_STRICT", "0") == "1"
    try:
        graph, sources = fx_to_graph(gm, example_inputs)
        dev = next((e.device for e in example_inputs if isinstance(e, torch.Tensor)), torch.device("cpu"))
        compiled = compile_graph(graph, pick_backend(dev.type), device=str(dev))
    except (Unsupported, NotImplementedError, AssertionError, ValueError) as e:
        if strict:
            raise
        log.warning("tensorjit: falling back to eager for this graph (%s)", e)
        return gm.forward

    params = dict(gm.named_parameters())
    params.update(dict(gm.named_buffers()))
    returns_seq = isinstance(next(n for n in gm.graph.nodes if n.op == "output").args[0], (tuple, list))

    def run(*args):
        ins = [args[s] if isinstance(s, int) else params[s[1]] for s in sources]
        outs = compiled(*ins)
        return list(outs) if returns_seq else outs[0]

    run.tensorjit_compiled = compiled  # type: ignore[attr-defined]
    return run
