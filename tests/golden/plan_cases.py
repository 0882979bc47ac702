"""Workloads whose kernel plans and memory plans are pinned by ``plans.json``, and the
one function that turns a lowered program into that file's JSON form.

Nothing here imports a tensorjit package: the fixture writer calls it with the
reference's modules and the tests with this repository's, on the same functions
(``bench.py``'s workloads, so the pinned programs are the ones the benchmark runs).

A program is described by positions in its optimised graph's node list, so two
graphs agree only if the tracer and the cleanup passes produced the same nodes in the
same order; kernels, row-kernel stages, reshape aliases and arena offsets are then
compared through those positions.
"""
from __future__ import annotations

# (case, bench function, [(shape, dtype)], environment overrides)
CASES = [
    ("c1_mlp_f32", "_fn_mlp", [((512, 768), "f32"), ((768,), "f32"), ((3072, 768), "f32"), ((3072,), "f32"),
                               ((768, 3072), "f32"), ((768,), "f32")], {}),
    ("c2_eltwise_f32", "_fn_c2", [((16384, 4096), "f32"), ((4096,), "f32"), ((4096,), "f32"),
                                  ((16384, 4096), "f32")], {}),
    ("c2_eltwise_bf16", "_fn_c2", [((16384, 4096), "bf16"), ((4096,), "bf16"), ((4096,), "bf16"),
                                   ((16384, 4096), "bf16")], {}),
    ("c2_eltwise_f32_no_row_fusion", "_fn_c2", [((16384, 4096), "f32"), ((4096,), "f32"), ((4096,), "f32"),
                                                ((16384, 4096), "f32")], {"TENSORJIT_NO_ROW_FUSION": "1"}),
    ("c3_layernorm_bf16", "_fn_ln", [((65536, 4096), "bf16"), ((4096,), "bf16")], {}),
    ("c3_rmsnorm_bf16", "_fn_rms", [((65536, 4096), "bf16"), ((4096,), "bf16")], {}),
    ("c3_softmax_f32", "_fn_softmax", [((65536, 2048), "f32")], {}),
    ("c4_gemm_bf16", "_fn_gemm", [((8192, 8192), "bf16"), ((8192, 8192), "bf16"), ((8192,), "bf16")], {}),
    ("c4_gemm_f32", "_fn_gemm", [((4096, 4096), "f32"), ((4096, 4096), "f32"), ((4096,), "f32")], {}),
    ("c4_skinny_bf16", "_fn_gemm", [((16, 8192), "bf16"), ((8192, 8192), "bf16"), ((8192,), "bf16")], {}),
    ("c5_attention_bf16", "_fn_attn", [((4, 32, 2048, 128), "bf16")] * 3, {}),
    ("c5_block_bf16", "_fn_block", [((4, 2048, 4096), "bf16"), ((4096,), "bf16"), ((4096, 4096), "bf16"),
                                    ((4096, 4096), "bf16"), ((4096, 4096), "bf16"), ((4096, 4096), "bf16"),
                                    ((4096,), "bf16"), ((11008, 4096), "bf16"), ((4096, 11008), "bf16")], {}),
    ("overhead_chain_f32", "_fn_chain", [((16, 32), "f32"), ((32, 32), "f32")], {}),
]

# the reference's cuda backend and this repository's hip backend share the row-fusion
# limit (8192), so their plans are the same function of the graph
REFERENCE_BACKEND = "cuda"
BACKEND = "hip"


def _attr(v):
    if isinstance(v, (list, tuple)):
        return [_attr(x) for x in v]
    if isinstance(v, float) and v != v:
        return "nan"
    if isinstance(v, (bool, int, float, str)) or v is None:
        return v
    return repr(v)


def describe(program, plan) -> dict:
    """JSON form of a lowered program and its memory plan."""
    g = program.graph
    pos = {id(n): i for i, n in enumerate(g.nodes)}

    def ids(nodes):
        return [pos[id(n)] for n in nodes]

    nodes = [[n.op, ids(n.inputs), list(n.shape), n.dtype.value,
              sorted([k, _attr(v)] for k, v in n.attrs.items())] for n in g.nodes]
    kernels = []
    for k in program.kernels:
        d = {"kind": k.kind, "nodes": ids(k.nodes), "anchor": None if k.anchor is None else pos[id(k.anchor)],
             "inputs": ids(k.inputs), "outputs": ids(k.outputs)}
        if k.kind == "row":
            d["rows"], d["n"] = list(k.rows), k.n
            d["stages"] = [[s.kind, ids(s.nodes)] for s in k.stages]
        kernels.append(d)
    aliases = sorted([pos[i], pos[id(src)], list(shape)]
                     for i, (src, shape) in program.aliases.items() if i in pos)
    offsets = sorted([pos[id(b.node)], b.offset, b.size] for b in plan.buffers.values())
    return {"graph": {"nodes": nodes, "inputs": ids(g.inputs), "outputs": ids(g.outputs)},
            "kernels": kernels, "aliases": aliases,
            "memory": {"arena_bytes": plan.arena_bytes, "naive_bytes": plan.naive_bytes, "buffers": offsets}}


def trace_case(tj, ir, fn, args):
    types = [ir.TensorType(tuple(shape), getattr(ir.DType, dt)) for shape, dt in args]
    return tj.trace(fn, types)
