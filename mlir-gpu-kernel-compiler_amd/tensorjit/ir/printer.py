"""Textual IR dump in an MLIR-like syntax (same format as the reference's
``tensorjit/ir/printer.py:13-26``)."""
from __future__ import annotations

from .graph import Graph


def _attr(v) -> str:
    return f"{v:.6g}" if isinstance(v, float) else str(v)


def print_graph(g: Graph) -> str:
    params = ", ".join(f"{i.name}: {i.type}" for i in g.inputs)
    results = ", ".join(str(o.type) for o in g.outputs)
    out = [f"func @{g.name}({params}) -> ({results}) {{"]
    for n in g.nodes:
        if n.op == "input":
            continue
        attrs = ""
        if n.attrs:
            attrs = " {" + ", ".join(f"{k} = {_attr(v)}" for k, v in n.attrs.items()) + "}"
        args = ", ".join(i.name for i in n.inputs)
        out.append(f"  {n.name} = {n.op}({args}){attrs} : {n.type}")
    out.append("  return " + ", ".join(o.name for o in g.outputs))
    out.append("}")
    return "\n".join(out)
