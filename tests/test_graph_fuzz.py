"""Seeded random programs (tests/graph_fuzz.py) through the hip backend.

CPU: every program lowers, gets the backend rewrites and generates HIP that hipRTC
compiles for gfx950.  GPU: the programs run against the CPU oracle -- float32 within
1e-5 of the output's magnitude; bfloat16 within 5e-2 and float16 within 1e-2, since
every kernel boundary rounds the intermediates to the storage type where the oracle
keeps float32 (torch's own float16 evaluation of these programs is up to 1.6e-3 from
float64)."""

import pytest
import torch

import graph_fuzz
import tensorjit as tj
from parity import LOWP_NORM, attention_plan_reference, compare
from tensorjit.backends import hip_backend as hb
from tensorjit.compiler import lower
from tensorjit.ir import DType, TensorType

CPU_SEEDS = range(16)
GPU_SEEDS = range(80)
# norm-wise bounds (tests/parity.py) per storage type: a program stores its intermediates
# in that type between kernels, each store a rounding of ~1.7e-3 (bf16) or ~2e-4 (fp16)
# RMS relative that later kernels carry forward
NORM = {torch.float32: 1e-5, torch.bfloat16: 1e-2, torch.float16: 2e-3}


@pytest.mark.parametrize("seed", CPU_SEEDS)
def test_random_program_generates_and_compiles(seed, tj_env):
    fn, shapes = graph_fuzz.program(seed)
    for dt in (DType.f32, DType.bf16):
        p = lower(tj.trace(fn, [TensorType(s, dt) for s in shapes]), "hip")
        p = hb.fold_elementwise_into_gemm(hb.fuse_attention(p))
        src, launches = hb.generate(p)
        assert len(launches) >= len(p.kernels)
        hb.compile_source(src, "gfx950")


def test_the_programs_cover_every_kernel_family(tj_env):
    kinds = set()
    for seed in range(64):
        fn, shapes = graph_fuzz.program(seed)
        p = lower(tj.trace(fn, [TensorType(s, DType.f32) for s in shapes]), "hip")
        kinds |= {k.kind for k in p.kernels}
    assert kinds >= {"elementwise", "copy", "row", "reduce", "matmul"}


@pytest.mark.gpu
@pytest.mark.parametrize("seed", GPU_SEEDS)
def test_random_program_matches_the_oracle(seed, monkeypatch):
    import oracle

    monkeypatch.setenv("TENSORJIT_NO_AUTOTUNE", "1")
    fn, shapes = graph_fuzz.program(seed)
    g = torch.Generator().manual_seed(seed)
    ins = [torch.randn(s, generator=g) for s in shapes]
    for dt, tol in ((torch.float32, 1e-5), (torch.bfloat16, 5e-2), (torch.float16, 1e-2)):
        print(f"random program {seed} {dt} {shapes}", flush=True)
        outs = tj.jit(fn)(*[t.to(dt).cuda() for t in ins])
        outs = outs if isinstance(outs, (tuple, list)) else [outs]
        refs = oracle.run(fn, *[t.to(dt).float() for t in ins])
        assert len(outs) == len(refs)
        for i, (o, r) in enumerate(zip(outs, refs)):
            compare(o, r, rtol=tol, scale=tol, norm=NORM[dt], what=f"seed {seed} {dt} output {i}")


ATTN_SEEDS = range(24)
LAYER_SEEDS = range(16)


@pytest.mark.parametrize("seed", ATTN_SEEDS)
def test_random_attention_generates_and_compiles(seed, tj_env, monkeypatch):
    fn, shapes = graph_fuzz.attention_program(seed)
    p = lower(tj.trace(fn, [TensorType(s, DType.bf16) for s in shapes]), "hip")
    q = hb.fuse_attention(p)
    # head dims that are multiples of 32 fuse; 16 keeps the reference plan's three kernels
    fused = shapes[0][-1] % 32 == 0
    assert [k.kind for k in q.kernels] == (["attention"] if fused else [k.kind for k in p.kernels]), (seed, shapes)
    src, _ = hb.generate(q)
    hb.compile_source(src, "gfx950")
    if fused and shapes[0][-1] % 64 == 0 and shapes[2][-1] % 64 == 0:
        # the ping-pong schedule, which the layout rule keeps for large grids
        monkeypatch.setenv("TENSORJIT_HIP_ATTENTION_WAVES", "8")
        src, (l,) = hb.generate(q)
        assert l.block == (512, 1, 1)
        hb.compile_source(src, "gfx950")


@pytest.mark.parametrize("seed", LAYER_SEEDS)
def test_random_layer_gets_the_backend_rewrites(seed, tj_env):
    fn, shapes = graph_fuzz.layer_program(seed)
    p = lower(tj.trace(fn, [TensorType(s, DType.bf16) for s in shapes]), "hip")
    q = hb.sink_epilogue_into_rows(hb.fold_elementwise_into_gemm(hb.fuse_attention(p)))
    # the second residual joins the last GEMM's epilogue
    assert len(q.kernels) == len(p.kernels) - 1 and q.kernels[-1].kind == "matmul"
    src, _ = hb.generate(q)
    hb.compile_source(src, "gfx950")


def _check_vs_oracle(fn, shapes, seed, dts, scales=None):
    import oracle

    g = torch.Generator().manual_seed(seed)
    ins = [torch.randn(s, generator=g) * (scales[i] if scales else 1.0) for i, s in enumerate(shapes)]
    for dt, tol in dts:
        outs = tj.jit(fn)(*[t.to(dt).cuda() for t in ins])
        outs = outs if isinstance(outs, (tuple, list)) else [outs]
        refs = oracle.run(fn, *[t.to(dt).float() for t in ins])
        for i, (o, r) in enumerate(zip(outs, refs)):
            assert torch.isfinite(o).all()
            compare(o, r, rtol=tol, scale=tol, norm=NORM[dt], what=f"seed {seed} {dt} output {i}")


@pytest.mark.gpu
@pytest.mark.parametrize("seed", ATTN_SEEDS)
def test_random_attention_matches_the_oracle(seed, monkeypatch):
    """The fused flash kernel on random shapes, bf16 and fp16, against the fp32 oracle
    of the reference plan (2e-2, the bound of the hand-written attention tests).  Head
    dims that are not multiples of 32 keep the reference plan's three kernels, which store
    the scores and probabilities in the storage type: those are held to the float64
    emulation of that plan's stores (at bf16 a stored logit of a few units moves its
    probability by more than the output's own rounding)."""
    monkeypatch.setenv("TENSORJIT_NO_AUTOTUNE", "1")
    fn, shapes = graph_fuzz.attention_program(seed)
    print(f"random attention {seed} {shapes}", flush=True)
    if shapes[0][-1] % 32 == 0:
        _check_vs_oracle(fn, shapes, seed, [(torch.bfloat16, 2e-2), (torch.float16, 2e-2)])
    else:
        g = torch.Generator().manual_seed(seed)
        ins = [torch.randn(s, generator=g) for s in shapes]
        for dt in (torch.bfloat16, torch.float16):
            args = [t.to(dt) for t in ins]
            f = tj.jit(fn)
            out = f(*[t.cuda() for t in args])
            assert [k.kind for k in f.compiled(*[t.cuda() for t in args]).program.kernels].count("attention") == 0
            compare(out, attention_plan_reference(*args, fn.scores, dt), rtol=2e-2, scale=2e-2, norm=LOWP_NORM,
                    what=f"seed {seed} {dt} unfused vs emulated plan")
    if shapes[0][-1] % 64 == 0 and shapes[2][-1] % 64 == 0:
        # the same cores on the ping-pong schedule (the layout rule keeps it for grids of
        # at least 256 workgroups, which these shapes do not reach)
        monkeypatch.setenv("TENSORJIT_HIP_ATTENTION_WAVES", "8")
        print(f"random attention {seed} {shapes} ping-pong", flush=True)
        _check_vs_oracle(fn, shapes, seed, [(torch.bfloat16, 2e-2)])


@pytest.mark.gpu
@pytest.mark.parametrize("seed", LAYER_SEEDS)
def test_random_layer_matches_the_oracle(seed, monkeypatch):
    """A random residual layer through every backend rewrite, fp32 (1e-5) and bf16
    (5e-2: intermediates stored in bf16), against the oracle of the reference plan."""
    monkeypatch.setenv("TENSORJIT_NO_AUTOTUNE", "1")
    fn, shapes = graph_fuzz.layer_program(seed)
    print(f"random layer {seed} {shapes}", flush=True)
    _check_vs_oracle(fn, shapes, seed, [(torch.float32, 1e-5), (torch.bfloat16, 5e-2)])


BCAST_SEEDS = range(24)


@pytest.mark.parametrize("seed", range(12))
def test_random_broadcast_program_generates_and_compiles(seed, tj_env):
    fn, shapes = graph_fuzz.broadcast_program(seed)
    for dt in (DType.f32, DType.bf16):
        p = lower(tj.trace(fn, [TensorType(s, dt) for s in shapes]), "hip")
        src, _ = hb.generate(hb.sink_epilogue_into_rows(hb.fold_elementwise_into_gemm(hb.fuse_attention(p))))
        hb.compile_source(src, "gfx950")


@pytest.mark.gpu
@pytest.mark.parametrize("seed", BCAST_SEEDS)
def test_random_broadcast_program_matches_the_oracle(seed, monkeypatch):
    """3-D / 4-D programs over size-1 (broadcast) dims with permutes and middle-axis
    reductions, fp32 (1e-5), bf16 (5e-2) and fp16 (1e-2), against the oracle."""
    monkeypatch.setenv("TENSORJIT_NO_AUTOTUNE", "1")
    fn, shapes = graph_fuzz.broadcast_program(seed)
    print(f"random broadcast program {seed} {shapes}", flush=True)
    _check_vs_oracle(fn, shapes, seed, [(torch.float32, 1e-5), (torch.bfloat16, 5e-2), (torch.float16, 1e-2)])


BLOCK_SEEDS = range(12)


@pytest.mark.parametrize("seed", range(6))
def test_random_transformer_stack_generates_and_compiles(seed, tj_env):
    """One or two transformer blocks in one module: in bf16 every block's attention is
    one flash kernel and its MLP residual joins the down-projection's epilogue."""
    fn, shapes, _ = graph_fuzz.block_program(seed)
    p = lower(tj.trace(fn, [TensorType(s, DType.bf16) for s in shapes]), "hip")
    q = hb.sink_epilogue_into_rows(hb.fold_elementwise_into_gemm(hb.fuse_attention(p)))
    kinds = [k.kind for k in q.kernels]
    layers = kinds.count("attention")
    assert layers >= 1 and len(kinds) == 9 * layers and "copy" not in kinds, (seed, kinds)
    src, _ = hb.generate(q)
    hb.compile_source(src, "gfx950")


@pytest.mark.gpu
@pytest.mark.parametrize("seed", BLOCK_SEEDS)
def test_random_transformer_stack_matches_the_oracle(seed, monkeypatch):
    """Random one- and two-block transformer stacks (weights scaled by 1/sqrt(fan-in)):
    fp32 within 1e-5 (attention unfused: the reference plan's kernels), bf16 within 3e-2
    (fused attention, bf16 intermediates; torch's own bf16 evaluation of these programs
    is up to 1e-2 from float64), against the oracle of the reference plan."""
    monkeypatch.setenv("TENSORJIT_NO_AUTOTUNE", "1")
    fn, shapes, scales = graph_fuzz.block_program(seed)
    print(f"random transformer stack {seed} {shapes[0]}", flush=True)
    _check_vs_oracle(fn, shapes, seed, [(torch.float32, 1e-5), (torch.bfloat16, 3e-2)], scales)


RED_SEEDS = range(24)


@pytest.mark.parametrize("seed", range(12))
def test_random_long_reduction_splits_and_compiles(seed, tj_env):
    """Random reductions over few long rows: in fp32 and bf16 the reduction splits its
    rows over workgroups (a combine launch follows it) and the module compiles."""
    fn, shapes = graph_fuzz.reduction_program(seed)
    for dt in (DType.f32, DType.bf16):
        p = lower(tj.trace(fn, [TensorType(s, dt) for s in shapes]), "hip")
        src, launches = hb.generate(p)
        assert [l.meta["family"] for l in launches][-2:] == ["row", "row_combine"], (seed, dt)
        hb.compile_source(src, "gfx950")


@pytest.mark.gpu
@pytest.mark.parametrize("seed", RED_SEEDS)
def test_random_long_reduction_matches_the_oracle(seed, monkeypatch):
    """Split reductions with random prologues, epilogues, row counts and ragged row
    lengths, fp32 (1e-5) and bf16 (5e-2), against the oracle."""
    monkeypatch.setenv("TENSORJIT_NO_AUTOTUNE", "1")
    fn, shapes = graph_fuzz.reduction_program(seed)
    print(f"random long reduction {seed} {shapes}", flush=True)
    _check_vs_oracle(fn, shapes, seed, [(torch.float32, 1e-5), (torch.bfloat16, 5e-2)])


TRANSPOSE_SEEDS = range(32)


def test_random_transposes_take_the_tiled_copy(tj_env):
    """Every random permute (output innermost dim strided in the source, 16-byte rows)
    plans as one copy kernel on the LDS-tiled path, for 2- and 4-byte elements."""
    for seed in TRANSPOSE_SEEDS:
        shape, perm = graph_fuzz.transpose_case(seed)
        for dt in (DType.f32, DType.bf16):
            p = lower(tj.trace(lambda t: tj.permute(t, *perm), [TensorType(shape, dt)]), "hip")
            src, launches = hb.generate(p)
            assert [l.meta.get("tiled") for l in launches] == [64], (seed, shape, perm, dt)
            if seed < 4:
                hb.compile_source(src, "gfx950")


@pytest.mark.gpu
@pytest.mark.parametrize("seed", TRANSPOSE_SEEDS)
def test_random_transposes_are_bit_exact(seed):
    shape, perm = graph_fuzz.transpose_case(seed)
    print(f"random transpose {seed} {shape} {perm}", flush=True)
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=g) * 1000
    for dt in (torch.float32, torch.bfloat16, torch.float16, torch.int32):
        y = x.to(dt).cuda()
        out = tj.jit(lambda t: tj.permute(t, *perm))(y)
        assert torch.equal(out, y.permute(*perm).contiguous()), (seed, dt)


WIDE_SEEDS = range(24)


@pytest.mark.parametrize("seed", range(8))
def test_random_wide_row_program_is_one_row_kernel(seed, tj_env):
    """Random chains of row ops over rows of 4097-32768 elements plan as one row kernel
    (the hip row-fusion limit is 32768) and compile."""
    fn, shapes = graph_fuzz.wide_row_program(seed)
    for dt in (DType.f32, DType.bf16):
        p = lower(tj.trace(fn, [TensorType(s, dt) for s in shapes]), "hip")
        q = hb.sink_epilogue_into_rows(hb.fold_elementwise_into_gemm(hb.fuse_attention(p)))
        assert [k.kind for k in q.kernels] == ["row"], (seed, dt)
        src, _ = hb.generate(q)
        hb.compile_source(src, "gfx950")


@pytest.mark.gpu
@pytest.mark.parametrize("seed", WIDE_SEEDS)
def test_random_wide_row_program_matches_the_oracle(seed, monkeypatch):
    """Wide-row chains (1024-lane and 256-lane layouts, odd lengths on scalar lanes), fp32
    within 1e-5 and bf16 within 5e-2, against the oracle."""
    monkeypatch.setenv("TENSORJIT_NO_AUTOTUNE", "1")
    fn, shapes = graph_fuzz.wide_row_program(seed)
    print(f"random wide-row program {seed} {shapes}", flush=True)
    _check_vs_oracle(fn, shapes, seed, [(torch.float32, 1e-5), (torch.bfloat16, 5e-2)])


COL_SEEDS = range(24)


@pytest.mark.parametrize("seed", range(8))
def test_random_column_reduction_folds_and_compiles(seed, tj_env):
    """Random reductions over a non-last axis: every reduction of the transposed value
    becomes a column reduction and the module compiles, in fp32 and bf16."""
    fn, shapes = graph_fuzz.column_program(seed)
    for dt in (DType.f32, DType.bf16):
        p = lower(tj.trace(fn, [TensorType(s, dt) for s in shapes]), "hip")
        q = hb.fold_transpose_into_reduce(hb.sink_epilogue_into_rows(hb.fold_elementwise_into_gemm(hb.fuse_attention(p))))
        kinds = [k.kind for k in q.kernels]
        assert "copy" not in kinds and kinds.count("colreduce") == [k.kind for k in p.kernels].count("reduce"), (seed, dt)
        src, _ = hb.generate(q)
        hb.compile_source(src, "gfx950")


@pytest.mark.gpu
@pytest.mark.parametrize("seed", COL_SEEDS)
def test_random_column_reduction_matches_the_oracle(seed, monkeypatch):
    """Column reductions with random prologues, axes, keepdim, shared transposes and
    epilogues, fp32 (1e-5) and bf16 (5e-2), against the oracle."""
    monkeypatch.setenv("TENSORJIT_NO_AUTOTUNE", "1")
    fn, shapes = graph_fuzz.column_program(seed)
    print(f"random column reduction {seed} {shapes}", flush=True)
    _check_vs_oracle(fn, shapes, seed, [(torch.float32, 1e-5), (torch.bfloat16, 5e-2)])


def test_rows_of_one_element_read_per_row(tj_env):
    """Random program 144 has rows of one element ([2, 37, 1]): a per-row epilogue reads
    a value of an earlier whole-row stage, which a row is then just one element of.  The
    hip generator and the oracle both emitted a read of a loop-local name there; now the
    hip kernel compiles and the oracle's row-fused plan agrees with its unfused plan."""
    import os

    import oracle

    fn, shapes = graph_fuzz.program(144)
    assert shapes[0][-1] == 1
    p = lower(tj.trace(fn, [TensorType(s, DType.f32) for s in shapes]), "hip")
    assert any(k.kind == "row" for k in p.kernels)
    src, _ = hb.generate(hb.sink_epilogue_into_rows(hb.fold_elementwise_into_gemm(hb.fuse_attention(p))))
    hb.compile_source(src, "gfx950")
    g = torch.Generator().manual_seed(144)
    ins = [torch.randn(s, generator=g) for s in shapes]
    fused = oracle.run(fn, *ins)
    os.environ["TENSORJIT_NO_ROW_FUSION"] = "1"
    try:
        plain = oracle.run(fn, *ins)
    finally:
        del os.environ["TENSORJIT_NO_ROW_FUSION"]
    for a, b in zip(fused, plain):
        torch.testing.assert_close(a, b, rtol=1e-6, atol=1e-6)


@pytest.mark.gpu
def test_rows_of_one_element_read_per_row_on_the_gpu(monkeypatch):
    monkeypatch.setenv("TENSORJIT_NO_AUTOTUNE", "1")
    fn, shapes = graph_fuzz.program(144)
    print(f"random program 144 {shapes}", flush=True)
    _check_vs_oracle(fn, shapes, 144, [(torch.float32, 1e-5), (torch.bfloat16, 5e-2), (torch.float16, 1e-2)])


DIFF_CASES = ([("program", s) for s in range(0, 200, 5)] + [("broadcast", s) for s in range(0, 60, 5)]
              + [("column", s) for s in range(0, 24, 3)] + [("wide_row", s) for s in range(0, 24, 4)]
              + [("program", 144)])


# Programs whose own fp32 evaluation sits far from float64 relative to the output's RMS.
# Broadcast program 35 layer-normalises a softmax of a softmax: its rows are nearly uniform
# (~1/96), so x - mean(x) cancels ~7 of fp32's 24 bits and both plans land 2.2e-5 * rms
# from the float64 graph evaluation at the same element.
ILL_CONDITIONED = {("broadcast", 35): 3e-5}


@pytest.mark.parametrize("gen,seed", DIFF_CASES)
def test_row_fusion_matches_the_unfused_plan(gen, seed, monkeypatch):
    """The oracle with row fusion against the oracle without it, on random programs: the
    parity tests compare the hip path with an oracle that shares its plan, so a plan that
    computes the wrong thing (column values applied per row) or a generator that cannot
    express a fused row (rows of one element) shows only here.  fp32, within 1e-5."""
    import oracle

    r = {"program": graph_fuzz.program, "broadcast": graph_fuzz.broadcast_program,
         "column": graph_fuzz.column_program, "wide_row": graph_fuzz.wide_row_program}[gen](seed)
    fn, shapes = r[0], r[1]
    g = torch.Generator().manual_seed(seed)
    ins = [torch.randn(s, generator=g) for s in shapes]
    fused = oracle.run(fn, *ins)
    monkeypatch.setenv("TENSORJIT_NO_ROW_FUSION", "1")
    plain = oracle.run(fn, *ins)
    tol = ILL_CONDITIONED.get((gen, seed), 1e-5)
    for i, (a, b) in enumerate(zip(fused, plain)):
        compare(a, b, rtol=1e-5, scale=tol, norm=1e-5, what=f"{gen} {seed} output {i}")


EVAL_CASES = ([("program", s) for s in range(0, 300, 10)] + [("broadcast", s) for s in range(0, 100, 10)]
              + [("attention", s) for s in range(0, 30, 5)] + [("column", s) for s in range(0, 30, 5)]
              + [("wide_row", s) for s in range(0, 16, 4)] + [("block", 0), ("reduction", 0)])


@pytest.mark.parametrize("gen,seed", EVAL_CASES)
def test_oracle_matches_the_float64_graph_evaluation(gen, seed):
    """The oracle (the reference plan as C) against the traced graph evaluated node by
    node in float64 (tests/graph_eval.py: no fusion, no plan): a plan or oracle that
    computes something other than the ops' meaning fails here, whatever the hip path
    does.  Within 2e-5 of the output's magnitude (fp32 accumulation; the largest seen
    over 510 programs was 9.4e-6)."""
    import graph_eval
    import oracle

    r = {"program": graph_fuzz.program, "broadcast": graph_fuzz.broadcast_program,
         "attention": graph_fuzz.attention_program, "column": graph_fuzz.column_program,
         "wide_row": graph_fuzz.wide_row_program, "block": graph_fuzz.block_program,
         "reduction": graph_fuzz.reduction_program}[gen](seed)
    fn, shapes = r[0], r[1]
    scales = r[2] if len(r) > 2 else None
    g = torch.Generator().manual_seed(seed)
    ins = [torch.randn(s, generator=g) * (scales[i] if scales else 1.0) for i, s in enumerate(shapes)]
    ref = graph_eval.evaluate(tj.trace(fn, [TensorType(s, DType.f32) for s in shapes]), *ins)
    out = oracle.run(fn, *ins)
    for i, (o, rf) in enumerate(zip(out, ref)):
        compare(o, rf, rtol=2e-5, scale=2e-5, norm=2e-5, what=f"{gen} {seed} output {i}")


def test_graph_evaluation_catches_a_column_value_applied_per_row(tj_env):
    """The float64 evaluation tells the two readings of a no-keepdim column mean apart:
    over a square x, the column reading (the ops' meaning) and the per-row reading (what
    a row kernel would compute) differ by O(1)."""
    import graph_eval

    x, w = torch.randn(64, 64, dtype=torch.float64), torch.randn(64, dtype=torch.float64)
    (ref,) = graph_eval.evaluate(tj.trace(lambda t, v: t - tj.mean(t, axis=0) * v,
                                          [TensorType((64, 64), DType.f32), TensorType((64,), DType.f32)]), x, w)
    torch.testing.assert_close(ref, x - x.mean(0) * w)
    assert float((ref - (x - (x.mean(0) * w)[:, None])).abs().max()) > 0.1
