"""IR, cleanup passes, fusion and row fusion: the kernel plan must match the
reference's for the same graph (its known-answer tests,
tests/test_ir_and_passes.py:13-127 and tests/test_cuda_backend.py:60-63, plus the
plans derived for the benchmark configs)."""
import torch

import tensorjit as tj
import tensorjit.compiler as C
from tensorjit.ir import DType, Graph, TensorType
from tensorjit.passes import fuse, optimize
from tensorjit.passes.cleanup import cse, dce


def _graph(fn, *shapes, dtype=DType.f32):
    return tj.trace(fn, [TensorType(s, dtype) for s in shapes])


def _plan(fn, *shapes, dtype=DType.f32):
    p = C.lower(_graph(fn, *shapes, dtype=dtype), "hip")
    return [(k.kind, [n.op for n in k.nodes]) for k in p.kernels], p


def test_type_inference_and_broadcast():
    g = _graph(lambda a, b: a * b + 1.0, (4, 1, 8), (3, 8))
    assert g.outputs[0].shape == (4, 3, 8)


def test_matmul_batched_broadcast_shape():
    g = _graph(lambda a, b: tj.matmul(a, b), (2, 1, 5, 7), (3, 7, 4))
    assert g.outputs[0].shape == (2, 3, 5, 4)


def test_mixed_dtypes_rejected():
    import pytest

    g = Graph()
    a = g.add_input(TensorType((4,), DType.f32))
    b = g.add_input(TensorType((4,), DType.bf16))
    with pytest.raises(TypeError):
        g.create("add", [a, b])


def test_cse_merges_duplicates():
    g = _graph(lambda x: tj.exp(x) + tj.exp(x), (8,))
    assert sum(n.op == "exp" for n in g.nodes) == 2
    cse(g)
    assert sum(n.op == "exp" for n in g.nodes) == 1


def test_algebraic_simplify_and_dce():
    g = _graph(lambda x: (x * 1.0 + 0.0) * (2.0 * 3.0), (8,))
    optimize(g)
    ops = [n.op for n in g.nodes if n.op not in ("input", "const")]
    assert ops == ["mul"], ops
    assert any(abs(c.attrs["value"] - 6.0) < 1e-12 for c in g.nodes if c.op == "const")


def test_dce_removes_unused():
    g = _graph(lambda x: (x + 1.0, (x * 5.0)), (4,))
    g.set_outputs([g.outputs[0]])
    assert dce(g)
    assert not any(n.op == "mul" for n in g.nodes)


def test_fold_transpose_into_matmul_and_broadcast():
    g = optimize(_graph(lambda x, w: tj.matmul(x, tj.broadcast_to(w.T, (3, 5)) * 1.0), (2, 3), (5, 3)))
    # broadcast_to feeds an elementwise op -> folded; the mul by 1 -> folded; transpose -> trans_b
    mm = next(n for n in g.nodes if n.op == "matmul")
    assert mm.attrs.get("trans_b") and mm.inputs[1].op == "input"


def test_fusion_groups_elementwise_chain_into_one_kernel():
    p = fuse(optimize(_graph(lambda x, y: tj.relu(x * 2.0 + y).exp(), (16, 32), (32,))))
    assert len(p.kernels) == 1 and p.kernels[0].kind == "elementwise"
    assert [n.op for n in p.kernels[0].nodes] == ["mul", "add", "relu", "exp"]


def test_fusion_matmul_epilogue():
    p = fuse(optimize(_graph(lambda x, w, b: tj.gelu(tj.matmul(x, w) + b), (8, 16), (16, 32), (32,))))
    assert [k.kind for k in p.kernels] == ["matmul"]
    assert [n.op for n in p.kernels[0].nodes] == ["matmul", "add", "gelu"]


def test_fusion_reduce_prologue():
    p = fuse(optimize(_graph(lambda x: tj.sum(x * x), (8, 16))))
    assert len(p.kernels) == 1 and p.kernels[0].kind == "reduce"
    assert [n.op for n in p.kernels[0].nodes] == ["mul", "sum"]


def test_fusion_does_not_duplicate_compute():
    p = fuse(optimize(_graph(lambda x: tj.layer_norm(x), (8, 16))))
    assert [n.op for k in p.kernels for n in k.nodes].count("sub") == 1


def test_reshape_is_free():
    p = fuse(optimize(_graph(lambda x: tj.exp(x.reshape(4, 8)), (8, 4))))
    assert len(p.kernels) == 1 and p.aliases


def test_signature_is_stable_and_shape_sensitive():
    g1 = _graph(lambda x: tj.exp(x), (8,))
    g2 = _graph(lambda x: tj.exp(x), (8,))
    g3 = _graph(lambda x: tj.exp(x), (9,))
    assert g1.signature() == g2.signature() != g3.signature()


def test_printer_roundtrip_mentions_ops():
    s = str(_graph(lambda x: tj.softmax(x), (4, 8)))
    assert "max(" in s and "exp(" in s and "sum(" in s and "func @" in s


def test_graph_builder_api():
    g = Graph("manual")
    a = g.add_input(TensorType((2, 3)))
    g.set_outputs([g.create("exp", [a])])
    assert g.outputs[0].shape == (2, 3)
    assert isinstance(torch.empty(1), torch.Tensor)


def test_row_fusion_layernorm_softmax_single_kernel():
    g = optimize(_graph(lambda x, w, b: (tj.layer_norm(x, w, b), tj.softmax(x)), (8, 64), (64,), (64,)))
    p = C.lower(g, "hip")
    assert [k.kind for k in p.kernels] == ["row", "row"]
    assert all(len(k.outputs) == 1 for k in p.kernels)


def test_row_fusion_respects_dependencies_through_matmul():
    def f(x, w):
        mu = tj.mean(x, keepdim=True)
        y = tj.matmul(x - mu, w)
        return tj.softmax(y) + mu

    kinds = [k.kind for k in C.lower(optimize(_graph(f, (8, 32), (32, 32))), "hip").kernels]
    assert "matmul" in kinds and kinds.index("matmul") < len(kinds) - 1


def test_row_fusion_limit_keeps_long_rows_apart():
    """Row fusion keeps rows longer than its limit apart: with the reference's GPU limit
    (8192) a softmax over 10000 stays four kernels; the hip backend's limit is 32768, so
    there it is one row kernel, and a softmax over 40000 is four again."""
    from tensorjit.passes import row_fuse

    g = optimize(_graph(lambda x: tj.softmax(x), (4, 10000)))
    assert [k.kind for k in row_fuse(fuse(g), max_n=8192).kernels] == ["reduce", "elementwise", "reduce", "elementwise"]
    assert C.ROW_FUSION_MAX_N["hip"] == 32768
    assert [k for k, _ in _plan(lambda x: tj.softmax(x), (4, 10000))[0]] == ["row"]
    assert [k for k, _ in _plan(lambda x: tj.softmax(x), (4, 32768))[0]] == ["row"]
    kinds, _ = _plan(lambda x: tj.softmax(x), (4, 40000))
    assert kinds[0][0] == "reduce" and len(kinds) == 4


# --- plans of the benchmark configurations (derived by reading the reference's
# --- tensorjit/passes/fusion.py; the README prints the LayerNorm/MLP lists) -------

MLP = lambda x, g, w1, b1, w2, b2: x + tj.linear(tj.gelu(tj.linear(tj.layer_norm(x, g), w1, b1)), w2, b2)  # noqa: E731


def test_plan_mlp_block_config1():
    kinds, _ = _plan(MLP, (512, 768), (768,), (3072, 768), (3072,), (768, 3072), (768,))
    assert kinds == [
        ("row", ["mean", "sub", "mul", "mean", "add", "rsqrt", "mul", "mul"]),
        ("matmul", ["matmul", "add", "gelu"]),
        ("matmul", ["matmul", "add", "add"]),
    ]


def test_plan_eltwise_chain_config2_is_one_row_kernel_with_two_stages():
    kinds, p = _plan(lambda x, a, b, c: tj.gelu(x * a + b) * tj.sigmoid(c) + x,
                     (16384, 4096), (4096,), (4096,), (16384, 4096))
    assert kinds == [("row", ["sigmoid", "mul", "add", "gelu", "mul", "add"])]
    k = p.kernels[0]
    assert [[n.op for n in st.nodes] for st in k.stages] == [["sigmoid"], ["mul", "add", "gelu", "mul", "add"]]
    assert [i.name for i in k.inputs][0] == "%arg3" and len(k.inputs) == 4 and len(k.outputs) == 1


def test_plan_eltwise_chain_without_row_fusion(monkeypatch):
    monkeypatch.setenv("TENSORJIT_NO_ROW_FUSION", "1")
    kinds, _ = _plan(lambda x, a, b, c: tj.gelu(x * a + b) * tj.sigmoid(c) + x,
                     (64, 32), (32,), (32,), (64, 32))
    assert kinds == [("elementwise", ["sigmoid"]), ("elementwise", ["mul", "add", "gelu", "mul", "add"])]


def test_plan_row_configs3():
    kinds, p = _plan(lambda x, g: tj.layer_norm(x, g), (65536, 4096), (4096,), dtype=DType.bf16)
    assert kinds == [("row", ["mean", "sub", "mul", "mean", "add", "rsqrt", "mul", "mul"])]
    assert len(p.kernels[0].stages) == 4
    kinds, p = _plan(lambda x, g: tj.rms_norm(x, g), (65536, 4096), (4096,), dtype=DType.bf16)
    assert kinds == [("row", ["mul", "mean", "add", "rsqrt", "mul", "mul"])] and len(p.kernels[0].stages) == 2
    kinds, p = _plan(lambda s: tj.softmax(s), (65536, 2048))
    assert kinds == [("row", ["max", "sub", "exp", "sum", "div"])] and len(p.kernels[0].stages) == 4


def test_plan_gemm_config4():
    kinds, p = _plan(lambda x, w, b: tj.gelu(tj.linear(x, w, b)), (8192, 8192), (8192, 8192), (8192,),
                     dtype=DType.bf16)
    assert kinds == [("matmul", ["matmul", "add", "gelu"])]
    assert p.kernels[0].anchor.attrs.get("trans_b") is True


def test_plan_launch_geometry_shape_of_mlp():
    # reference tests/test_cuda_backend.py:60-63: the MLP is [row, matmul, matmul]
    kinds, _ = _plan(MLP, (64, 128), (128,), (256, 128), (256,), (128, 256), (128,))
    assert [k for k, _ in kinds] == ["row", "matmul", "matmul"]


def test_plan_transformer_block_config5():
    import bench

    shapes = [(4, 2048, 4096), (4096,), (4096, 4096), (4096, 4096), (4096, 4096), (4096, 4096), (4096,),
              (11008, 4096), (4096, 11008)]
    kinds, p = _plan(bench._fn_block, *shapes, dtype=DType.bf16)
    assert [k for k, _ in kinds] == ["row", "matmul", "copy", "matmul", "copy", "matmul", "copy", "matmul", "row",
                                     "matmul", "copy", "matmul", "row", "matmul", "matmul", "elementwise"]
    qk = p.kernels[7]
    assert qk.anchor.attrs.get("trans_b") and [n.op for n in qk.nodes] == ["matmul", "mul"]   # k^T folded, scale fused
    assert [n.op for n in p.kernels[8].nodes] == ["max", "sub", "exp", "sum", "div"]
    assert [n.op for n in p.kernels[11].nodes] == ["matmul", "add", "mul"]                  # residual (+ next x*x) fused
    assert [n.op for n in p.kernels[13].nodes] == ["matmul", "gelu"]


def test_row_fusion_keeps_column_broadcasts_out_of_row_kernels():
    """A reduced value without keepdim, shape ``rows``, broadcasts along the last axis
    of ``rows + (N,)`` when ``rows[-1] == N``: it is a column value, and a row kernel
    holding one value per row would apply it to the wrong elements.  The reference's
    shape-only check fuses such pairs; here they stay apart, and the oracle agrees with
    eager torch (float64) where the fused plan was off by O(1)."""
    import oracle

    torch.manual_seed(0)
    cases = [
        # per-column mean subtracted from a square matrix (column normalisation)
        (lambda t, w: t - tj.mean(t, axis=0) * w, [(64, 64), (64,)],
         lambda t, w: t - t.mean(0) * w),
        # a reduction whose prologue reads the row means as a column broadcast
        (lambda t, w: tj.sum(t * tj.mean(t, axis=-1), axis=-1) + w, [(48, 48), (48,)],
         lambda t, w: (t * t.mean(-1)).sum(-1) + w),
    ]
    for fn, shapes, ref_fn in cases:
        kinds, _ = _plan(fn, *shapes)
        assert not any(k == "row" for k, _ in kinds), kinds
        args = [torch.randn(s) for s in shapes]
        out = oracle.run(fn, *args)[0]
        ref = ref_fn(*[a.double() for a in args])
        assert float((out.double() - ref).abs().max()) <= 1e-4 * float(ref.abs().max()), fn
    # with keepdim the same chain is per row and row-fuses
    kinds, _ = _plan(lambda t, w: t - tj.mean(t, axis=-1, keepdim=True) * w, (64, 64), (64,))
    assert [k for k, _ in kinds] == ["row"]
