"""The hip backend's rewrites of the planned program, CPU side: fused attention
(matmul -> softmax -> matmul) and elementwise kernels moved into a GEMM's epilogue --
which planned programs are rewritten, what the rewritten program looks like, and that
the generated flash-attention kernel compiles for gfx950 with hipRTC."""
import re

import pytest

import tensorjit as tj
import tensorjit.compiler as C
from tensorjit.backends import hip_backend as hb
from tensorjit.backends.hip_attention import fuse_attention
from tensorjit.ir import DType, TensorType
from tensorjit.passes.memory_planner import plan_memory


def attn(q, k, v, scale=0.125):
    s = tj.matmul(q, tj.transpose(k, -1, -2))
    return tj.matmul(tj.softmax(s * scale if scale != 1.0 else s), v)


def lowered(fn, shapes, dtype=DType.bf16):
    return C.lower(tj.trace(fn, [TensorType(s, dtype) for s in shapes]), "hip")


QKV = [(2, 4, 128, 64), (2, 4, 128, 64), (2, 4, 128, 64)]


def test_plain_attention_chain_becomes_one_kernel():
    p = lowered(attn, QKV)
    assert [k.kind for k in p.kernels] == ["matmul", "row", "matmul"]
    f = fuse_attention(p)
    assert [k.kind for k in f.kernels] == ["attention"]
    k = f.kernels[0]
    assert [i.shape for i in k.inputs] == [(2, 4, 128, 64)] * 3
    assert k.outputs[0].shape == (2, 4, 128, 64) and k.attn["scale"] == 0.125
    # the scores and probabilities get no arena space any more
    assert plan_memory(p).arena_bytes >= 2 * 4 * 128 * 128 * 2
    assert plan_memory(f).arena_bytes == 0


def test_attention_layout_rule():
    """Ping-pong (8 waves) only where it measured faster: head dims of at least 128 and a
    grid of at least one ping-pong workgroup per CU; 4 waves otherwise."""
    from tensorjit.backends.hip_attention import attention_layout

    assert attention_layout(128, 2048, 128, 128) == (8, 1)       # config 5: 1024 workgroups
    assert attention_layout(16, 4096, 128, 128) == (8, 1)        # exactly 256
    assert attention_layout(16, 2048, 128, 128) == (4, 1)        # 128 workgroups
    assert attention_layout(128, 2048, 64, 64) == (4, 1)         # head dim 64
    assert attention_layout(512, 256, 128, 128) == (4, 1)        # short query sequences
    assert attention_layout(128, 2048, 96, 96) == (4, 1)


def test_key_splits_for_grids_short_of_the_cus():
    """Key-range splits only for 4-wave grids short of one workgroup per CU, with an
    equal share of at least 2 key blocks each: the smallest count that fills the CUs."""
    from tensorjit.backends.hip_attention import attention_splits

    assert attention_splits(32, 16, False) == 8          # 2 blocks each, 256 workgroups
    assert attention_splits(32, 64, False) == 8
    assert attention_splits(1, 64, False) == 32          # the largest count that divides
    assert attention_splits(9, 5, False) == 1            # 5 blocks: no equal >= 2-block split
    assert attention_splits(256, 64, False) == 1         # the grid already fills the CUs
    assert attention_splits(8, 64, True) == 1            # not for the ping-pong schedule


@pytest.mark.parametrize("shapes", [[(2, 2, 1000, 128)] * 3, [(1, 1, 4096, 128)] * 3,
                                    [(1, 3, 200, 64), (1, 3, 2000, 64), (1, 3, 2000, 128)]])
def test_split_attention_compiles_with_its_combine_launch(shapes, tj_env):
    f = fuse_attention(lowered(attn, shapes))
    src, launches = hb.generate(f)
    main, comb = launches
    ns = main.meta["splits"]
    assert ns > 1 and comb.meta["splits"] == ns and main.meta["ws_arg"] and comb.meta["ws_arg"]
    B = main.meta["batch"]
    Sq, Dv = shapes[0][-2], shapes[2][-1]
    # partial rows plus a (reference, sum) pair per row and split
    assert main.meta["workspace"] == ns * B * Sq * (Dv + 2) * 4
    assert comb.grid[0] * 256 >= B * Sq * Dv // 8
    hb.compile_source(src, "gfx950")


def test_two_attention_cores_in_one_program_compile(tj_env):
    """Two fused attention kernels share one module: their lane-pair helpers live in the
    prelude, so the source holds each device function once and hipRTC compiles it."""
    fn = lambda q, k, v: attn(attn(q, k, v), k, v)  # noqa: E731
    f = fuse_attention(lowered(fn, QKV))
    assert [k.kind for k in f.kernels] == ["attention", "attention"]
    src, launches = hb.generate(f)
    assert len(launches) == 2 and src.count("float tj_pair_max(") == 1
    hb.compile_source(src, "gfx950")


def test_unscaled_and_differently_sized_value_heads():
    f = fuse_attention(lowered(lambda q, k, v: attn(q, k, v, 1.0), [(3, 50, 32), (3, 70, 32), (3, 70, 96)]))
    assert [k.kind for k in f.kernels] == ["attention"] and f.kernels[0].attn["scale"] == 1.0


@pytest.mark.parametrize("form,scale", [
    (lambda s: s / 8.0, 0.125),                 # q @ kᵀ / sqrt(d)
    (lambda s: s / 3.0, 1.0 / 3.0),
    (lambda s: 0.25 * s, 0.25),                 # constant on the left of the multiply
])
def test_scale_written_as_division_or_left_multiply(form, scale):
    fn = lambda q, k, v: tj.matmul(tj.softmax(form(tj.matmul(q, tj.transpose(k, -1, -2)))), v)  # noqa: E731
    f = fuse_attention(lowered(fn, QKV))
    assert [k.kind for k in f.kernels] == ["attention"] and f.kernels[0].attn["scale"] == scale


@pytest.mark.parametrize("form", [lambda s: 8.0 / s, lambda s: s / 0.0], ids=["constant_over_scores", "by_zero"])
def test_divisions_that_are_not_a_scale_stay_unfused(form):
    fn = lambda q, k, v: tj.matmul(tj.softmax(form(tj.matmul(q, tj.transpose(k, -1, -2)))), v)  # noqa: E731
    f = fuse_attention(lowered(fn, QKV))
    assert all(k.kind != "attention" for k in f.kernels)


@pytest.mark.parametrize("case", ["fp32", "probs_returned", "scores_reused", "head_dim_8", "head_dim_16",
                                  "extra_epilogue"])
def test_chains_that_must_stay_unfused(case):
    if case == "fp32":
        p = lowered(attn, QKV, DType.f32)
    elif case == "probs_returned":
        def fn(q, k, v):
            pr = tj.softmax(tj.matmul(q, tj.transpose(k, -1, -2)) * 0.1)
            return tj.matmul(pr, v), pr
        p = lowered(fn, QKV)
    elif case == "scores_reused":
        def fn(q, k, v):
            s = tj.matmul(q, tj.transpose(k, -1, -2)) * 0.1
            return tj.matmul(tj.softmax(s), v) + tj.sum(s, axis=-1, keepdim=True)
        p = lowered(fn, QKV)
    elif case == "head_dim_8":
        p = lowered(attn, [(2, 16, 8)] * 3)
    elif case == "head_dim_16":
        # 64 keys x 16 dims is 128 16-byte chunks, fewer than the 256 lanes that copy a block
        p = lowered(attn, [(2, 64, 16), (2, 700, 16), (2, 700, 64)])
    else:
        p = lowered(lambda q, k, v: tj.relu(attn(q, k, v)), QKV)
    f = fuse_attention(p)
    assert all(k.kind != "attention" for k in f.kernels)


def test_env_switch_keeps_the_reference_plan(monkeypatch):
    monkeypatch.setenv("TENSORJIT_HIP_ATTENTION", "0")
    p = lowered(attn, QKV)
    assert fuse_attention(p) is p


def test_config5_block_fuses_its_attention():
    import bench

    shapes = [(4, 2048, 4096), (4096,), (4096, 4096), (4096, 4096), (4096, 4096), (4096, 4096), (4096,),
              (11008, 4096), (4096, 11008)]
    p = lowered(bench._fn_block, shapes)
    assert len(p.kernels) == 16
    f = fuse_attention(p)
    # the attention chain and the four head transposes around it are one kernel
    assert len(f.kernels) == 10 and [k.kind for k in f.kernels].count("attention") == 1
    (att,) = [k for k in f.kernels if k.kind == "attention"]
    assert att.attn["layouts"] == ["bshd"] * 3 and att.attn["out_layout"] == "bshd"
    assert [i.shape for i in att.inputs] == [(4, 2048, 32, 128)] * 3 and att.outputs[0].shape == (4, 2048, 32, 128)
    assert all(k.kind != "copy" for k in f.kernels)
    # the 1 GiB score and probability buffers are gone from the arena (2.25 GiB -> 428 MiB)
    assert plan_memory(f).arena_bytes < plan_memory(p).arena_bytes - 1.5 * 2**30


def test_config5_second_residual_joins_the_down_projection():
    """The reference plan keeps config 5's last add as an elementwise kernel behind the
    down-projection; the backend rewrite moves it into that GEMM's epilogue (9 kernels),
    and the 64 MiB down-projection result is no longer a planned buffer."""
    import bench
    from tensorjit.backends.hip_backend import fold_elementwise_into_gemm

    shapes = [(4, 2048, 4096), (4096,), (4096, 4096), (4096, 4096), (4096, 4096), (4096, 4096), (4096,),
              (11008, 4096), (4096, 11008)]
    f = fuse_attention(lowered(bench._fn_block, shapes))
    assert f.kernels[-1].kind == "elementwise" and f.kernels[-2].kind == "matmul"
    down = f.kernels[-2].outputs[0]
    q = fold_elementwise_into_gemm(f)
    assert len(q.kernels) == 9 and q.kernels[-1].kind == "matmul"
    assert [n.op for n in q.kernels[-1].nodes] == ["matmul", "add"]
    assert q.kernels[-1].outputs == f.kernels[-1].outputs
    assert plan_memory(f).offset(down) is not None and plan_memory(q).offset(down) is None


def test_config5_square_of_the_residual_moves_into_the_rmsnorm_row():
    """The plan computes the second RMSNorm's x1 * x1 in the out-projection's epilogue
    and stores it for the row kernel; the rewrite computes it in the row kernel's
    reduction stage, so the GEMM stores x1 only and the row kernel reads x1 and g."""
    import bench
    from tensorjit.backends.hip_backend import fold_elementwise_into_gemm, sink_epilogue_into_rows

    shapes = [(4, 2048, 4096), (4096,), (4096, 4096), (4096, 4096), (4096, 4096), (4096, 4096), (4096,),
              (11008, 4096), (4096, 11008)]
    f = fold_elementwise_into_gemm(fuse_attention(lowered(bench._fn_block, shapes)))
    q = sink_epilogue_into_rows(f)
    out_proj = [k for k in f.kernels if k.kind == "matmul" and len(k.outputs) == 2]
    assert len(out_proj) == 1 and [n.op for n in out_proj[0].nodes] == ["matmul", "add", "mul"]
    i = f.kernels.index(out_proj[0])
    assert [n.op for n in q.kernels[i].nodes] == ["matmul", "add"] and len(q.kernels[i].outputs) == 1
    row = q.kernels[i + 1]
    assert row.kind == "row" and [n.op for n in row.nodes][:2] == ["mul", "mean"]
    assert [x.shape for x in row.inputs] == [(4, 2048, 4096), (4096,)]
    assert [n.op for n in row.stages[0].nodes][:2] == ["mul", "mean"]
    assert len(q.kernels) == len(f.kernels) == 9


def test_epilogue_values_read_elsewhere_stay_in_the_gemm():
    """x1 * x1 also returned (or read by a pointwise kernel) keeps its place."""
    from tensorjit.backends.hip_backend import sink_epilogue_into_rows

    def fn(x, w, g):
        h = x + tj.linear(x, w)
        sq = h * h
        return tj.rms_norm(h, g), sq

    p = lowered(fn, [(256, 512), (512, 512), (512,)])
    q = sink_epilogue_into_rows(p)
    assert [[n.op for n in k.nodes] for k in q.kernels] == [[n.op for n in k.nodes] for k in p.kernels]


def test_gemm_results_with_other_users_are_not_folded():
    """A GEMM result that is also a graph output (or read by another kernel) keeps its
    own store: the elementwise kernel stays."""
    from tensorjit.backends.hip_backend import fold_elementwise_into_gemm

    def fn(x, a, b):
        h = x + tj.linear(x, a)
        y = tj.linear(tj.relu(h), b)
        return h + y, y

    p = lowered(fn, [(256, 512), (512, 512), (512, 512)])
    assert [k.kind for k in fold_elementwise_into_gemm(p).kernels] == [k.kind for k in p.kernels]


@pytest.mark.parametrize("dtype", [DType.bf16, DType.f16])
@pytest.mark.parametrize("shapes", [QKV, [(1, 100, 32), (1, 75, 32), (1, 75, 64)], [(2, 2, 256, 128)] * 3,
                                    [(1, 2, 600, 64), (1, 2, 1000, 64), (1, 2, 1000, 128)],
                                    [(1, 2, 512, 64), (1, 2, 900, 64), (1, 2, 900, 64)],
                                    [(1, 2, 512, 64), (1, 2, 128, 64), (1, 2, 128, 64)],
                                    [(1, 2, 512, 64), (1, 2, 40, 64), (1, 2, 40, 64)]])
@pytest.mark.parametrize("forced", [None, "8"], ids=["rule", "pingpong"])
def test_flash_kernel_compiles_for_gfx950(shapes, dtype, forced, tj_env, monkeypatch):
    if forced:
        monkeypatch.setenv("TENSORJIT_HIP_ATTENTION_WAVES", forced)
    f = fuse_attention(lowered(attn, shapes, dtype))
    src, launches = hb.generate(f)
    l = launches[0]
    # a combine launch exactly when the keys are split
    assert len(launches) == (2 if l.meta["splits"] > 1 else 1)
    from tensorjit.backends.hip_attention import attention_layout

    waves, tiles = attention_layout(l.meta["batch"], shapes[0][-2], shapes[0][-1], shapes[2][-1])
    # the forced ping-pong schedule needs head dims that are multiples of 64
    assert waves == (8 if forced and shapes[0][-1] % 64 == 0 and shapes[2][-1] % 64 == 0 else 4)
    assert "attention" in l.name and l.block == (64 * waves, 1, 1)
    assert l.grid == (-(-shapes[0][-2] // (32 * waves * tiles)) * l.meta["batch"] * l.meta["splits"], 1, 1)
    if waves == 8:
        # the last key block computes no scores for a block after it
        kb = -(-shapes[1][-2] // 64)
        tag = f"// block {kb - 1}" if l.meta["schedule"] == "pingpong-dma" else f"const unsigned int jj = {kb - 1}u;"
        last = src.split(tag)[1].split("if (gq == 0u)")[0]
        score_mfma = re.compile(r"\((kf|kt\d+), qf\[")
        assert not score_mfma.search(last) and score_mfma.search(src)
    code = hb.compile_source(src, "gfx950")
    assert len(code) > 1000


def mha(x, wq, wk, wv, heads=2):
    B, S, Dm = x.shape
    d = Dm // heads
    q = tj.linear(x, wq).reshape(B, S, heads, d).transpose(1, 2)
    k = tj.linear(x, wk).reshape(B, S, heads, d).transpose(1, 2)
    v = tj.linear(x, wv).reshape(B, S, heads, d).transpose(1, 2)
    o = tj.matmul(tj.softmax(tj.matmul(q, k.transpose(-1, -2)) * (1.0 / d ** 0.5)), v)
    return o.transpose(1, 2).reshape(B, S, Dm)


def test_head_transposes_are_folded_into_strided_attention(tj_env):
    p = lowered(mha, [(2, 200, 128), (128, 128), (128, 128), (128, 128)])
    assert [k.kind for k in p.kernels].count("copy") == 4
    f = fuse_attention(p)
    assert [k.kind for k in f.kernels] == ["matmul", "matmul", "matmul", "attention"]
    src, launches = hb.generate(f)
    assert "(bh / 2u) * 25600u + (bh % 2u) * 64u" in src       # [B, S, H, D] addressing
    hb.compile_source(src, "gfx950")


def test_transpose_with_another_user_is_not_folded():
    def fn(x, wq, wk, wv):
        B, S, Dm = x.shape
        q = tj.linear(x, wq).reshape(B, S, 2, 64).transpose(1, 2)
        k = tj.linear(x, wk).reshape(B, S, 2, 64).transpose(1, 2)
        v = tj.linear(x, wv).reshape(B, S, 2, 64).transpose(1, 2)
        o = tj.matmul(tj.softmax(tj.matmul(q, k.transpose(-1, -2)) * 0.125), v)
        return o, q * 2.0
    f = fuse_attention(lowered(fn, [(2, 200, 128), (128, 128), (128, 128), (128, 128)]))
    (att,) = [k for k in f.kernels if k.kind == "attention"]
    assert att.attn["layouts"] == ["bhsd", "bshd", "bshd"] and att.attn["out_layout"] == "bhsd"
