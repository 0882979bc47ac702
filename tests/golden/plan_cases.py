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
    # rows past the reference's GPU row-fusion limit (8192) and up to the hip limit:
    # one row kernel each, the odd lengths on scalar lanes; 32769 is one past the limit
    # (the norms then plan as reductions and pointwise kernels)
    ("ln_bf16_512x16384", "_fn_ln", [((512, 16384), "bf16"), ((16384,), "bf16")], {}),
    ("ln_f32_256x32768", "_fn_ln", [((256, 32768), "f32"), ((32768,), "f32")], {}),
    ("ln_f32_1024x12000", "_fn_ln", [((1024, 12000), "f32"), ((12000,), "f32")], {}),
    ("ln_f32_64x32769", "_fn_ln", [((64, 32769), "f32"), ((32769,), "f32")], {}),
    ("rms_bf16_512x16384", "_fn_rms", [((512, 16384), "bf16"), ((16384,), "bf16")], {}),
    ("rms_f32_256x32768", "_fn_rms", [((256, 32768), "f32"), ((32768,), "f32")], {}),
    ("rms_bf16_1024x12001", "_fn_rms", [((1024, 12001), "bf16"), ((12001,), "bf16")], {}),
    ("softmax_f32_512x16384", "_fn_softmax", [((512, 16384), "f32")], {}),
    ("softmax_bf16_256x32768", "_fn_softmax", [((256, 32768), "bf16")], {}),
    ("softmax_f32_1024x12000", "_fn_softmax", [((1024, 12000), "f32")], {}),
    ("softmax_f32_64x32769", "_fn_softmax", [((64, 32769), "f32")], {}),
]

# Every case is lowered by the reference's own passes -- ``fuse(optimize(graph))`` and then
# ``row_fuse(program, max_n=ROW_FUSION_MAX_N)`` -- with the hip backend's row-fusion limit.
# The reference's cuda backend passes 8192 (reference tensorjit/compiler.py:34); below
# 8193 elements per row the two limits give the same plan.
ROW_FUSION_MAX_N = 32768
REFERENCE_BACKEND = "cuda"
BACKEND = "hip"


def _fn_column_centre(x, g):
    """A no-keepdim mean over axis 0 (one value per column) read along the rows of a
    square x: the reference's row fusion applies it per row."""
    import tensorjit as tj

    return x - tj.mean(x, axis=0) * g


# Cases where this repository's plan departs from the reference's on purpose: the
# reference's row_fuse (reference tensorjit/passes/fusion.py:279-295) joins kernels by
# their (rows, N) shapes only, so over a square x the column value above lands in a row
# kernel that holds one value per row; the hip plan keeps that pair as a reduction and a
# pointwise kernel.  (case, function in this module, [(shape, dtype)], reference kernel
# kinds, hip kernel kinds)
DIVERGENT = [
    ("column_centre_f32_64x64", "_fn_column_centre", [((64, 64), "f32"), ((64,), "f32")],
     ["copy", "row"], ["copy", "reduce", "elementwise"]),
]


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
