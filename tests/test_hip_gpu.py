"""hip backend on a real MI355X: parity with the CPU oracle (the restated reference
`c` backend) and with eager PyTorch on the same seeded inputs.

Tolerances (north star; tests/parity.py): fp32 |a-b| <= 1e-5*rms(b) + 1e-5*|b| per element
and ||a-b|| <= 1e-5*||b|| over the tensor and over every row; bf16/fp16 storage within 2e-2
of the fp32 oracle per element (atol 2e-2*rms) and within 5e-3 in norm, whole and per row;
integer / max / copy results bit-exact.  Case list follows the reference's tests/test_backends.py and
tests/test_cuda_backend.py.
"""
import math
import os

import pytest
import torch
import torch.nn.functional as F

import oracle
import tensorjit as tj
from parity import attention_plan_reference, close_f32, close_lowp

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _skip_without_gpu():
    if not (torch.cuda.is_available() and torch.version.hip):
        pytest.skip("needs a ROCm GPU")


@pytest.fixture(autouse=True)
def _env(monkeypatch, tmp_path_factory):
    _skip_without_gpu()
    monkeypatch.setenv("TENSORJIT_NO_AUTOTUNE", "1")
    monkeypatch.setenv("TENSORJIT_CACHE_DIR", str(tmp_path_factory.getbasetemp() / "tjcache"))
    yield


def check_vs_oracle(fn, *args, rtol=1e-5, scale=1e-5, norm=None, lowp_norm=5e-3):
    f = tj.jit(fn)
    outs = f(*args)
    outs = outs if isinstance(outs, tuple) else (outs,)
    refs = oracle.run(fn, *[a.float().cpu() for a in args])
    for i, (o, r) in enumerate(zip(outs, refs)):
        assert o.is_cuda and o.shape == r.shape
        if o.dtype == torch.float32:
            close_f32(o, r, rtol, scale, norm=norm, what=f"output {i}")
        else:
            close_lowp(o, r, norm=lowp_norm, what=f"output {i}")
    return f, outs


# ------------------------------------------------------------------ pointwise


@pytest.mark.parametrize("shape", [(17,), (8, 33), (2, 3, 5), (64, 4096)])
def test_elementwise_chain(shape):
    torch.manual_seed(0)
    x, y = torch.randn(*shape, device=DEV), torch.randn(shape[-1], device=DEV)
    fn = lambda a, b: tj.exp(tj.relu(a * 2.0 + b)) / (1.0 + tj.sigmoid(a)) - tj.tanh(b)  # noqa: E731
    f, (out,) = check_vs_oracle(fn, x, y)
    ref = torch.exp(torch.relu(x * 2 + y)) / (1 + torch.sigmoid(x)) - torch.tanh(y)
    torch.testing.assert_close(out, ref, atol=1e-4, rtol=1e-4)
    assert f.compiled(x, y).backend == "hip"


@pytest.mark.parametrize("op", ["gelu", "silu", "log", "sqrt", "rsqrt", "abs", "sigmoid", "exp", "tanh", "relu"])
def test_unary_ops(op):
    torch.manual_seed(0)
    x = torch.rand(4096, device=DEV) + 0.5
    check_vs_oracle(getattr(tj, op), x, rtol=2e-6, scale=2e-6)


def test_where_maximum_pow():
    torch.manual_seed(0)
    x, y = torch.randn(40, device=DEV), torch.randn(40, device=DEV)
    x[::7] = 0.0
    check_vs_oracle(lambda a, b: tj.where(a, tj.maximum(a, b), tj.minimum(a, b)) + tj.abs(a) ** 2.0, x, y)


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16, torch.float16])
def test_config2_chain_small(dt):
    torch.manual_seed(0)
    x, a, b = torch.randn(64, 4096, device=DEV), torch.randn(4096, device=DEV), torch.randn(4096, device=DEV)
    c = torch.rand(64, 4096, device=DEV) * 8 - 4
    args = [t.to(dt) for t in (x, a, b, c)]
    check_vs_oracle(lambda x, a, b, c: tj.gelu(x * a + b) * tj.sigmoid(c) + x, *args)


def test_transpose_reshape_and_copies_are_bit_exact():
    torch.manual_seed(0)
    x = torch.randn(3, 4, 5, device=DEV)
    f = tj.jit(lambda t: tj.exp(tj.permute(t, 2, 0, 1)).reshape(5, 12) + 1.0)
    torch.testing.assert_close(f(x), torch.exp(x.permute(2, 0, 1)).reshape(5, 12) + 1)
    for dt in (torch.float32, torch.bfloat16, torch.int32):
        y = (torch.randn(4, 64, 8, 32, device=DEV) * 100).to(dt)
        g = tj.jit(lambda t: tj.transpose(t, 1, 2))
        assert torch.equal(g(y), y.transpose(1, 2).contiguous())
        h = tj.jit(lambda t: tj.permute(t, 3, 0, 2, 1))
        assert torch.equal(h(y), y.permute(3, 0, 2, 1).contiguous())


@pytest.mark.parametrize("shape,perm", [((128, 64), (1, 0)), ((104, 48), (1, 0)), ((3, 40, 72), (2, 0, 1)),
                                        ((5, 8, 16, 24), (3, 1, 0, 2)), ((2, 3, 96, 80), (0, 1, 3, 2)),
                                        ((6, 5, 16, 8), (1, 3, 0, 2)), ((1000, 520), (1, 0))])
@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16, torch.float16, torch.int32])
def test_tiled_transposes_are_bit_exact(shape, perm, dt):
    """Transposes whose output's innermost dim is strided in the source go through the
    LDS-tiled copy (ragged edge tiles included), bit for bit against torch."""
    g = torch.Generator(device=DEV).manual_seed(7)
    y = (torch.randn(shape, device=DEV, generator=g) * 1000).to(dt)
    f = tj.jit(lambda t: tj.permute(t, *perm))
    out = f(y)
    assert f.compiled(y).launches[0].meta.get("tiled") == 64
    assert torch.equal(out, y.permute(*perm).contiguous())


@pytest.mark.parametrize("shape", [(16384, 4095), (1000, 1001), (3, 5, 7, 9)])
@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16, torch.float16, torch.int32])
def test_odd_rows_of_contiguous_operands_vectorise_bit_exact(shape, dt):
    """Same-shape pointwise kernels over odd row lengths run 16-byte vectors across rows:
    bit for bit against torch (x * 2 + y is exact in every dtype: the product by 2 is
    exact, one rounding for the sum)."""
    g = torch.Generator(device=DEV).manual_seed(11)
    x = (torch.randn(shape, device=DEV, generator=g) * 100).to(dt)
    y = (torch.randn(shape, device=DEV, generator=g) * 100).to(dt)
    f = tj.jit(lambda a, b: a * 2.0 + b)
    out = f(x, y)
    numel = math.prod(shape)
    assert f.compiled(x, y).launches[0].meta["vec"] == (16 // x.element_size() if numel % (16 // x.element_size()) == 0 else 1)
    assert torch.equal(out, x * 2 + y)


def test_int32_arithmetic_and_max_are_exact_below_2_24():
    """int32 storage: pointwise ops evaluate in fp32, as the reference's expressions do, and
    convert on store, so integer results below 2^24 in magnitude are exact -- a pointwise chain
    with Python scalars, a maximum, and a row max (reduction from -inf) against torch's integer
    arithmetic, bit for bit."""
    g = torch.Generator(device=DEV).manual_seed(0)
    x = torch.randint(-2 ** 20, 2 ** 20, (64, 1000), device=DEV, dtype=torch.int32, generator=g)
    y = torch.randint(-2 ** 20, 2 ** 20, (64, 1000), device=DEV, dtype=torch.int32, generator=g)
    f = tj.jit(lambda a, b: tj.maximum(a * 3 - b + 7, b))
    out = f(x, y)
    assert out.dtype == torch.int32 and torch.equal(out, torch.maximum(x * 3 - y + 7, y))
    m = tj.jit(lambda a: tj.max(a))
    assert torch.equal(m(x), x.amax(-1))


def test_int32_matmul_and_sums_are_exact_below_2_24():
    """int32 GEMMs (plain, transposed weight, batched, with an integer epilogue) and row sums run
    in fp32, as the reference's float evaluation does; with every partial sum below 2^24 the
    stored results equal integer arithmetic bit for bit."""
    g = torch.Generator(device=DEV).manual_seed(0)
    a = torch.randint(-8, 9, (130, 200), device=DEV, dtype=torch.int32, generator=g)
    b = torch.randint(-8, 9, (200, 70), device=DEV, dtype=torch.int32, generator=g)
    w = torch.randint(-8, 9, (90, 200), device=DEV, dtype=torch.int32, generator=g)
    c = torch.randint(-100, 100, (90,), device=DEV, dtype=torch.int32, generator=g)
    ref = lambda x, y: (x.cpu().long() @ y.cpu().long()).int()  # noqa: E731
    assert torch.equal(tj.jit(lambda x, y: tj.matmul(x, y))(a, b).cpu(), ref(a, b))
    assert torch.equal(tj.jit(lambda x, y, z: tj.linear(x, y, z) * 3)(a, w, c).cpu(), (ref(a, w.t()) + c.cpu()) * 3)
    ab = torch.randint(-8, 9, (3, 40, 64), device=DEV, dtype=torch.int32, generator=g)
    bb = torch.randint(-8, 9, (3, 64, 24), device=DEV, dtype=torch.int32, generator=g)
    got = tj.jit(lambda x, y: tj.matmul(x, y))(ab, bb).cpu()
    assert torch.equal(got, torch.stack([ref(ab[i], bb[i]) for i in range(3)]))
    rows = torch.randint(-1000, 1000, (64, 5000), device=DEV, dtype=torch.int32, generator=g)
    assert torch.equal(tj.jit(lambda x: tj.sum(x))(rows).cpu(), rows.cpu().long().sum(-1).int())


def test_int32_division_is_exact():
    """int32 a / b evaluates as a correctly rounded fp32 quotient truncated on store (the
    reference's expression is a plain ``/``).  For |a| < 2^24 the rounded quotient never
    crosses an integer, so the result equals integer division truncated toward zero --
    including exact multiples such as 41 / 41, which a reciprocal-multiply would store as 0."""
    q = torch.arange(-199, 200, device=DEV, dtype=torch.int32)
    d = torch.arange(1, 3000, device=DEV, dtype=torch.int32)
    a = (q[:, None] * d[None, :]).contiguous()
    b = d[None, :].expand_as(a).contiguous()
    f = tj.jit(lambda u, v: u / v)
    out = f(a, b)
    assert out.dtype == torch.int32
    assert torch.equal(out, q[:, None].expand_as(a))
    assert int(f(torch.tensor([41], device=DEV, dtype=torch.int32),
                 torch.tensor([41], device=DEV, dtype=torch.int32))[0]) == 1
    g = torch.Generator(device=DEV).manual_seed(1)
    a = torch.randint(-2 ** 23, 2 ** 23, (256, 1024), device=DEV, dtype=torch.int32, generator=g)
    b = torch.randint(1, 2 ** 12, (256, 1024), device=DEV, dtype=torch.int32, generator=g)
    b = torch.where(torch.rand(b.shape, device=DEV, generator=g) < 0.5, -b, b)
    assert torch.equal(f(a, b), torch.div(a, b, rounding_mode="trunc"))


def test_fp32_division_keeps_tiny_quotients():
    """fp32 ``/`` is IEEE division: quotients by divisors near the top of the range come out
    as the correctly rounded (subnormal) values torch computes, not 0."""
    x = torch.linspace(-4, 4, 1000, device=DEV)
    y = torch.full((1000,), 3.0e38, device=DEV)
    out = tj.jit(lambda u, v: u / v)(x, y)
    assert torch.equal(out, x / y) and bool((out[x != 0] != 0).all())


# ------------------------------------------------------------------ reductions / rows


@pytest.mark.parametrize("n", [1, 17, 100, 1000, 100000])
def test_reductions(n):
    torch.manual_seed(0)
    red = lambda t: (tj.sum(t), tj.max(t), tj.mean(t, keepdim=True))  # noqa: E731
    f = tj.jit(red)
    if n <= 1000:
        x = torch.randn(6, n, device=DEV)
        s, m, mu = f(x)
        refs = oracle.run(red, x.cpu())
        close_f32(s, refs[0], scale=1e-5 * math.sqrt(n))
        assert torch.equal(m.cpu(), x.amax(-1).cpu())          # max is bit-exact
        close_f32(mu, refs[2], scale=1e-5 * math.sqrt(n))
    # small integers: every partial sum is an integer below 2^24, so the sum is exact in
    # any order and a dropped or doubled element changes it; mean = sum / n correctly rounded
    xi = torch.randint(-3, 4, (6, n), device=DEV).float()
    s, m, mu = f(xi)
    exact = xi.cpu().double().sum(-1)
    assert torch.equal(s.cpu().double(), exact)
    assert torch.equal(m.cpu(), xi.amax(-1).cpu())
    assert torch.equal(mu.cpu().reshape(-1), exact.float() / float(n))


SPLIT_CASES = {
    # full reduction of one long row: 1024 workgroups, one 8-chunk segment each
    "sum_1row": (lambda x: tj.sum(x), [(1 << 23,)], torch.float32),
    # two workgroups' worth of segments per workgroup (the segment loop runs twice)
    "sum_loop": (lambda x: tj.sum(x, axis=-1), [(1, 1 << 24)], torch.float32),
    # mean of a two-input prologue, a ragged last chunk (300000 = 292.97 chunks)
    "mse": (lambda x, y: tj.mean((x - y) * (x - y), axis=-1), [(3, 300000), (3, 300000)], torch.float32),
    # bf16 rows, epilogue after the mean
    "rms": (lambda x: tj.sqrt(tj.mean(x * x, axis=-1) + 1e-5), [(8, 262144)], torch.bfloat16),
    # max with a keepdim output and an epilogue
    "max": (lambda x: tj.max(x, axis=-1, keepdim=True) * 2.0, [(4, 262144)], torch.float32),
    # an odd row length: scalar lanes (one element per lane)
    "odd": (lambda x: tj.sum(tj.abs(x), axis=-1), [(2, 300001)], torch.float32),
    # an epilogue reading a per-row input in the combine launch
    "epi_input": (lambda x, b: tj.sum(x, axis=-1) * b, [(3, 300000), (3,)], torch.float32),
    # two outputs of the epilogue (keepdim), both stored by the combine launch
    "two_outputs": (lambda x, b: (tj.mean(x * x, axis=-1, keepdim=True) + tj.abs(b),
                                  tj.sqrt(tj.mean(x * x, axis=-1, keepdim=True) + tj.abs(b))), [(3, 300000), (3, 1)],
                    torch.float32),
    # a prologue value stored as a second output beside the row sum
    "vec_out": (lambda x: (tj.exp(tj.tanh(x)), tj.sum(tj.exp(tj.tanh(x)), axis=-1)), [(2, 262144)], torch.float32),
}


@pytest.mark.parametrize("case", sorted(SPLIT_CASES))
def test_split_row_reductions_vs_oracle(case):
    """Reductions over few long rows, split over workgroups with a combine launch: against
    the oracle, and on small integers (every partial sum exact) bit for bit against the
    exact sum, so a dropped or doubled chunk or segment shows."""
    fn, shapes, dt = SPLIT_CASES[case]
    torch.manual_seed(0)
    print(f"split reduction {case} {shapes} {dt}", flush=True)
    args = [torch.randn(s, device=DEV).to(dt) for s in shapes]
    f = tj.jit(fn)
    launches = f.compiled(*args).launches
    assert [l.meta["family"] for l in launches[-2:]] == ["row", "row_combine"], case
    n = shapes[0][-1]
    outs = f(*args)
    outs = outs if isinstance(outs, tuple) else (outs,)
    refs = oracle.run(fn, *[a.float().cpu() for a in args])
    for o, r in zip(outs, refs):
        assert o.shape == r.shape
        if o.dtype == torch.float32:
            close_f32(o, r, scale=1e-5 * math.sqrt(n / 1024))
        else:
            close_lowp(o, r)
    if case == "max":
        assert torch.equal(outs[0], args[0].amax(-1, keepdim=True) * 2.0)
    if case in ("sum_1row", "sum_loop", "odd"):
        xi = torch.randint(-3, 4, shapes[0], device=DEV).float()
        exact = xi.abs().double().sum(-1) if case == "odd" else xi.double().sum(-1)
        assert torch.equal(f(xi).double(), exact)


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_norms_over_rows_past_the_row_fusion_limit(dt):
    """LayerNorm / RMSNorm / softmax over 3 rows of 300000: the plan gives their reductions
    and pointwise steps kernels of their own (rows past 32768 are not row-fused), and
    each reduction splits its rows over workgroups."""
    torch.manual_seed(0)
    x = (torch.randn(3, 300000, device=DEV) * 2).to(dt)
    g = (1 + 0.1 * torch.randn(300000, device=DEV)).to(dt)
    print(f"long-row norms {dt}", flush=True)
    f, _ = check_vs_oracle(lambda t, w: (tj.layer_norm(t, w), tj.rms_norm(t, w), tj.softmax(t)), x, g, scale=2e-5)
    fams = [l.meta["family"] for l in f.compiled(x, g).launches]
    assert fams.count("row_combine") >= 4, fams


def test_forced_split_of_short_ragged_rows(monkeypatch):
    """The split forced onto short rows (37 rows of 5000: five one-chunk segments per row,
    the last part-used) agrees with one workgroup per row: sums on small integers bit for
    bit, the max bit for bit, the mean to rounding."""
    torch.manual_seed(0)
    x = torch.randint(-3, 4, (37, 5000), device=DEV).float()
    fn = lambda t: (tj.sum(t, axis=-1), tj.max(t * 0.5 + 1.0, axis=-1), tj.mean(t * t, axis=-1))  # noqa: E731
    monkeypatch.setenv("TENSORJIT_HIP_ROW_SPLIT", "1")
    fs = tj.jit(fn)
    assert sum(l.meta["family"] == "row_combine" for l in fs.compiled(x).launches) == 3
    split = fs(x)
    monkeypatch.setenv("TENSORJIT_HIP_ROW_SPLIT", "0")
    fo = tj.jit(lambda t: (tj.sum(t, axis=-1), tj.max(t * 0.5 + 1.0, axis=-1), tj.mean(t * t, axis=-1)))
    assert not any(l.meta["family"] == "row_combine" for l in fo.compiled(x).launches)
    one = fo(x)
    assert torch.equal(split[0], one[0]) and torch.equal(split[1], one[1])
    torch.testing.assert_close(split[2], one[2], rtol=1e-6, atol=0)
    assert torch.equal(split[0].double(), x.double().sum(-1))


COL_CASES = {
    # sum over the leading axis: 64 slices of 64 rows, a combine launch
    "sum_axis0": (lambda x: tj.sum(x, axis=0), [(4096, 4096)], torch.float32),
    # mean-pooling over a sequence in bf16, an epilogue reading a per-output input
    "mean_pool": (lambda x, g: tj.tanh(tj.mean(x, axis=1) * 0.5) + g, [(8, 1024, 1024), (8, 1024)], torch.bfloat16),
    # an elementwise prologue folded in, max with keepdim
    "max_prologue": (lambda x: tj.max(x * 2.0 + 1.0, axis=0, keepdim=True), [(2048, 2048)], torch.float32),
    # one slice of the reduced axis: no combine launch
    "one_slice": (lambda x: tj.sum(x, axis=1), [(2048, 8, 256)], torch.float32),
    # a middle axis of a 4-D tensor, ragged against the 64-lane column blocks
    "middle_4d": (lambda x: tj.sum(x, axis=1), [(5, 37, 7, 24)], torch.float32),
    # odd inner dim: one element per lane
    "odd_inner": (lambda x: tj.mean(x, axis=0), [(999, 301)], torch.float32),
    "fp16": (lambda x: tj.sum(x * x, axis=0), [(3000, 520)], torch.float16),
}


@pytest.mark.parametrize("case", sorted(COL_CASES))
def test_column_reductions_vs_oracle(case):
    """Reductions over a non-last axis as one column reduction (the transpose kernel
    folded away): against the oracle, sums of small integers bit for bit against the
    exact sum, and the max bit for bit against the reference plan's kernels."""
    fn, shapes, dt = COL_CASES[case]
    torch.manual_seed(0)
    print(f"column reduction {case} {shapes} {dt}", flush=True)
    args = [torch.randn(s, device=DEV).to(dt) for s in shapes]
    f = tj.jit(fn)
    assert f.compiled(*args).launches[0].meta["family"] == "colreduce"
    n = shapes[0][1] if case in ("mean_pool", "one_slice", "middle_4d") else shapes[0][0]
    out = f(*args)
    ref = oracle.run(fn, *[a.float().cpu() for a in args])[0]
    assert out.shape == ref.shape
    if dt == torch.float32:
        close_f32(out, ref, scale=1e-5 * math.sqrt(n / 64))
    else:
        close_lowp(out, ref)
    if case == "max_prologue":
        assert torch.equal(out, (args[0] * 2.0 + 1.0).amax(0, keepdim=True).t())
    if case in ("sum_axis0", "one_slice", "middle_4d"):
        xi = torch.randint(-3, 4, shapes[0], device=DEV).float()
        axis = 0 if case == "sum_axis0" else 1
        assert torch.equal(f(xi).double(), xi.double().sum(axis))


@pytest.mark.parametrize("shape,dt,splits", [((16384, 4096), torch.float32, 16), ((32768, 4096), torch.float32, 32),
                                             ((16384, 4096), torch.bfloat16, 128)])
def test_column_reductions_at_benchmark_sizes(shape, dt, splits):
    """The split count follows the streamed bytes (one workgroup per CU at 256 MiB, two at
    512 MiB, four at 128 MiB): each layout against the oracle, and small-integer sums bit
    for bit against the exact sum."""
    torch.manual_seed(0)
    print(f"column reduction {shape} {dt}", flush=True)
    fn = lambda x: tj.sum(x, axis=0)  # noqa: E731
    x = torch.randn(shape, device=DEV).to(dt)
    f = tj.jit(fn)
    out = f(x)
    launches = f.compiled(x).launches
    assert launches[0].meta["family"] == "colreduce" and launches[0].meta["splits"] == splits, launches[0].meta
    (ref,) = oracle.run(fn, x.float().cpu())
    if dt == torch.float32:
        close_f32(out, ref, scale=1e-5 * math.sqrt(shape[0] / 64))
    else:
        close_lowp(out, ref)
    if dt == torch.float32:
        xi = torch.randint(-3, 4, shape, device=DEV).float()
        assert torch.equal(f(xi).double(), xi.double().sum(0))


def test_column_reduction_matches_the_reference_plan(monkeypatch):
    """The same max and mean with the fold switched off (transpose kernel + row
    reduction): the max bit for bit, the mean to rounding."""
    torch.manual_seed(0)
    x = torch.randn(3000, 1000, device=DEV)
    fn = lambda t: (tj.max(t, axis=0), tj.mean(t, axis=0))  # noqa: E731
    f = tj.jit(fn)
    fams = [l.meta["family"] for l in f.compiled(x).launches]
    assert fams.count("colreduce") == 2
    col = f(x)
    monkeypatch.setenv("TENSORJIT_HIP_COLREDUCE", "0")
    g = tj.jit(lambda t: (tj.max(t, axis=0), tj.mean(t, axis=0)))
    assert "colreduce" not in [l.meta["family"] for l in g.compiled(x).launches]
    ref = g(x)
    assert torch.equal(col[0], ref[0])
    torch.testing.assert_close(col[1], ref[1], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("n,dt", [(64, torch.float32), (4096, torch.float32), (4096, torch.bfloat16)])
def test_column_values_over_square_rows_match_eager(n, dt):
    """``x - mean(x, axis=0) * g`` and a row sum of ``x * mean(x, axis=-1)`` over square
    ``x``: the per-column value broadcasts along the last axis, so row fusion must not
    apply it per row.  Checked against eager torch in float64 (not only the oracle, which
    shares the plan)."""
    torch.manual_seed(0)
    x = torch.randn(n, n, device=DEV).to(dt)
    g = torch.randn(n, device=DEV).to(dt)
    xd, gd = x.double(), g.double()
    print(f"column values over square rows {n} {dt}", flush=True)
    out = tj.jit(lambda t, w: t - tj.mean(t, axis=0) * w)(x, g)
    ref = xd - xd.mean(0) * gd
    out2 = tj.jit(lambda t, w: tj.sum(t * tj.mean(t, axis=-1), axis=-1) + w)(x, g)
    ref2 = (xd * xd.mean(-1)).sum(-1) + gd
    for o, r in ((out, ref), (out2, ref2)):
        if dt == torch.float32:
            close_f32(o, r, scale=1e-5 * math.sqrt(n / 64))
        else:
            close_lowp(o, r)


def test_reduce_non_last_axis_via_transpose():
    torch.manual_seed(0)
    x = torch.randn(4, 5, 6, device=DEV)
    check_vs_oracle(lambda t: tj.sum(t, axis=1), x)


@pytest.mark.parametrize("shape", [(9, 70), (16, 768), (8, 4096), (4, 8192)])
def test_softmax_layernorm_rmsnorm(shape):
    torch.manual_seed(0)
    n = shape[-1]
    x = torch.randn(*shape, device=DEV)
    g, b = torch.randn(n, device=DEV), torch.randn(n, device=DEV)
    fn = lambda t, w, c: (tj.softmax(t), tj.layer_norm(t, w, c), tj.rms_norm(t, w))  # noqa: E731
    f, (sm, ln, rms) = check_vs_oracle(fn, x, g, b, scale=2e-5)
    torch.testing.assert_close(sm, torch.softmax(x, -1), atol=1e-4, rtol=1e-4)
    torch.testing.assert_close(ln, F.layer_norm(x, (n,), g, b), atol=1e-3, rtol=1e-3)


@pytest.mark.parametrize("rows,n,dt", [
    (1030, 768, torch.float32),      # one wave per row, 4 rows per workgroup, ragged last workgroup
    (1025, 2048, torch.bfloat16),    # 4 KiB rows: the largest wave-per-row case, ragged
    (1000, 520, torch.float16),      # too few rows for 4 per workgroup; 65 chunks: a part-used lane
    (300, 1200, torch.float32),      # one chunk per lane, 300 of 320 lanes used
    (257, 4096, torch.bfloat16),     # 8 KiB rows: 512 lanes x 1 chunk
    (64, 4096, torch.float32),       # 16 KiB rows, five reductions: 256 lanes x 4 chunks (the max: 1024 x 1)
    (16, 12288, torch.float32),      # longer rows: several chunks per lane (512 x 6)
    (37, 4097, torch.float32),       # odd length: scalar lanes, 832 lanes x 5 elements
    (8, 16384, torch.float32),       # 512 lanes x 8 chunks (the max: 256 x 16)
    (6, 32767, torch.float32),       # 1024 scalar lanes x 32 elements, the last lane part-used
    (3, 32768, torch.float32),       # 1024 lanes x 8 chunks
    (4, 32768, torch.bfloat16),      # 256 lanes x 16 chunks of 8
    (5, 20000, torch.float16),       # 256 lanes x 10 chunks, a ragged last chunk
])
def test_row_layouts_vs_oracle(rows, n, dt):
    """Every row layout (wave per row with a ragged last workgroup, one chunk per lane with idle
    lanes, several chunks per lane) for LayerNorm / RMSNorm / softmax against the oracle, and
    the row max, which a DPP all-reduce must give bit for bit."""
    from tensorjit.backends.hip_kernels import row_shape

    torch.manual_seed(0)
    x = (torch.randn(rows, n, device=DEV) * 2).to(dt)
    g = (1 + 0.1 * torch.randn(n, device=DEV)).to(dt)
    vec = 16 // x.element_size() if n % (16 // x.element_size()) == 0 else 1
    f, _ = check_vs_oracle(lambda t, w: (tj.layer_norm(t, w), tj.rms_norm(t, w), tj.softmax(t)), x, g)
    cp = f.compiled(x, g)
    # the gain is broadcast over rows
    shape = row_shape(n, vec, False, reductions=sum(st.kind == "reduce" for st in cp.program.kernels[0].stages))
    launch = cp.launches[0]
    assert launch.meta["threads"] == shape.lanes and launch.meta["chunks"] == shape.chunks
    m = tj.jit(lambda t: tj.max(t))
    assert torch.equal(m(x), x.amax(-1))
    assert m.compiled(x).launches[0].meta["threads"] == row_shape(n, vec, True).lanes      # one stage


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_row_kernels_low_precision_storage(dt):
    torch.manual_seed(0)
    x = torch.randn(32, 4096, device=DEV).to(dt)
    g = (1 + 0.1 * torch.randn(4096, device=DEV)).to(dt)
    check_vs_oracle(lambda t, w: (tj.layer_norm(t, w), tj.rms_norm(t, w), tj.softmax(t)), x, g)


# ------------------------------------------------------------------ matmul


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (7, 13, 5), (64, 64, 64), (33, 128, 65), (256, 512, 384)])
def test_matmul_with_epilogue_fp32(m, k, n):
    torch.manual_seed(0)
    a, b, bias = torch.randn(m, k, device=DEV), torch.randn(k, n, device=DEV), torch.randn(n, device=DEV)
    f, (out,) = check_vs_oracle(lambda x, y, z: tj.gelu(tj.matmul(x, y) + z), a, b, bias, rtol=1e-5, scale=1e-5)
    torch.testing.assert_close(out, F.gelu(a @ b + bias), atol=1e-3, rtol=1e-3)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,k,n", [(64, 128, 256), (33, 72, 65), (256, 1024, 512), (16, 4096, 512)])
def test_matmul_low_precision_vs_fp32(dt, m, k, n):
    torch.manual_seed(0)
    x = torch.randn(m, k, device=DEV).to(dt)
    w = (0.02 * torch.randn(n, k, device=DEV)).to(dt)
    bias = torch.randn(n, device=DEV).to(dt)
    f = tj.jit(lambda x, w, b: tj.gelu(tj.linear(x, w, b)))
    out = f(x, w, bias)
    ref = F.gelu(F.linear(x.float(), w.float(), bias.float()))
    close_lowp(out, ref, tol=2e-2)
    (orc,) = oracle.run(lambda x, w, b: tj.gelu(tj.linear(x, w, b)), x.float().cpu(), w.float().cpu(), bias.float().cpu())
    close_lowp(out, orc, tol=2e-2)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,k,n", [(1, 4096, 512), (5, 1000, 300), (16, 8192, 1024), (20, 2048, 96), (32, 512, 64)])
def test_skinny_decode_matmul(dt, m, k, n):
    torch.manual_seed(0)
    x = torch.randn(m, k, device=DEV).to(dt)
    w = (0.02 * torch.randn(n, k, device=DEV)).to(dt)
    bias = torch.randn(n, device=DEV).to(dt)
    fn = lambda x, w, b: tj.gelu(tj.linear(x, w, b))  # noqa: E731
    out = tj.jit(fn)(x, w, bias)
    (orc,) = oracle.run(fn, x.float().cpu(), w.float().cpu(), bias.float().cpu())
    close_lowp(out, orc, tol=2e-2)
    # exact on small integers: catches a misplaced lane or k-slice
    xi = torch.randint(-2, 3, (m, k), device=DEV).to(dt)
    wi = torch.randint(-2, 3, (n, k), device=DEV).to(dt)
    yi = tj.jit(lambda x, w: tj.linear(x, w))(xi, wi)
    # the exact integer sum, rounded once to the storage dtype (RNE, as the kernel stores)
    assert torch.equal(yi.cpu(), (xi.double() @ wi.double().t()).to(dt).cpu())


@pytest.mark.parametrize("m", [16, 7, 1])
def test_skinny_candidates_with_a_through_lds_are_exact(m):
    """Every decode-GEMM candidate at K = 4096, where the waves' K slices are whole
    256-deep chunks and A goes through LDS (1 to 8 chunks per wave, rows past M zero
    from the copy's range check), exact on small-integer data against the exact sum
    rounded once to bf16."""
    from tensorjit.backends import hip_backend as hb
    from tensorjit.runtime.autotune import HIP_CANDIDATES

    torch.manual_seed(0)
    a = torch.randint(-2, 3, (m, 4096), device=DEV).bfloat16()
    b = torch.randint(-2, 3, (320, 4096), device=DEV).bfloat16()
    fn = lambda x, y: tj.linear(x, y)  # noqa: E731
    ref = (a.double() @ b.double().t()).bfloat16()
    mm = C_lower(fn, a, b).kernels[0].anchor
    tried = 0
    for cfg in HIP_CANDIDATES:
        if cfg.SPLIT_K == 1 or not hb.config_ok(cfg, hb.compute_dtype(mm), mm):
            continue
        print(f"skinny {m}x320x4096 {cfg}", flush=True)
        out = _run_with_config(fn, [a, b], cfg)
        assert torch.equal(out, ref), (m, cfg)
        tried += 1
    assert tried >= 8


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16, torch.float32])
def test_mfma_layout_is_exact_on_integer_data(dt):
    """Small integers are exact in every dtype and in fp32 accumulation, so any
    misplaced fragment or accumulator element shows up as an exact mismatch."""
    torch.manual_seed(0)
    for (m, k, n, tb) in [(64, 64, 64, True), (128, 96, 160, False), (96, 64, 32, True)]:
        a = torch.randint(-3, 4, (m, k), device=DEV).to(dt)
        b = torch.randint(-3, 4, (n, k) if tb else (k, n), device=DEV).to(dt)
        f = tj.jit((lambda x, y: tj.linear(x, y)) if tb else (lambda x, y: tj.matmul(x, y)))
        out = f(a, b)
        ref = (a.double() @ (b.double().t() if tb else b.double())).to(dt)
        assert torch.equal(out.cpu(), ref.cpu()), (m, k, n, tb, dt)


def test_batched_matmul_broadcast_and_linear():
    torch.manual_seed(0)
    a, b = torch.randn(2, 3, 8, 16, device=DEV), torch.randn(3, 16, 8, device=DEV)
    check_vs_oracle(lambda x, y: tj.relu(tj.matmul(x, y)), a, b)
    x, w, bb = torch.randn(10, 32, device=DEV), torch.randn(48, 32, device=DEV), torch.randn(48, device=DEV)
    check_vs_oracle(tj.linear, x, w, bb)


def test_attention_shaped_batched_matmuls_bf16():
    torch.manual_seed(0)
    q = torch.randn(2, 4, 128, 64, device=DEV).bfloat16()
    k = torch.randn(2, 4, 128, 64, device=DEV).bfloat16()
    v = torch.randn(2, 4, 128, 64, device=DEV).bfloat16()
    f = tj.jit(lambda q, k, v: tj.matmul(tj.softmax(tj.matmul(q, tj.transpose(k, -1, -2)) * 0.125), v))
    out = f(q, k, v)
    p = torch.softmax((q.float() @ k.float().transpose(-1, -2).contiguous()) * 0.125, -1)
    ref = p @ v.float()
    close_lowp(out, ref, tol=3e-2)


ATTN = lambda q, k, v: tj.matmul(tj.softmax(tj.matmul(q, tj.transpose(k, -1, -2)) * 0.125), v)  # noqa: E731


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shapes", [[(2, 4, 128, 64)] * 3, [(1, 100, 32), (1, 75, 32), (1, 75, 64)],
                                    [(1, 2, 300, 128), (1, 2, 1000, 128), (1, 2, 1000, 128)],
                                    [(1, 2, 600, 64), (1, 2, 1000, 64), (1, 2, 1000, 128)],
                                    [(2, 8, 300, 64), (2, 8, 200, 64), (2, 8, 200, 64)],
                                    [(1, 2, 512, 64), (1, 2, 900, 64), (1, 2, 900, 64)],
                                    [(1, 2, 512, 64), (1, 2, 128, 64), (1, 2, 128, 64)],
                                    [(1, 2, 512, 64), (1, 2, 40, 64), (1, 2, 40, 64)]],
                         ids=["even", "ragged_dv64", "multi_block_ragged", "eight_waves_ragged", "xcd_grouped_heads",
                              "eight_waves_odd_blocks", "eight_waves_two_blocks", "eight_waves_one_ragged_block"])
def test_fused_attention_vs_oracle_and_unfused_plan(shapes, dt, monkeypatch):
    """The flash kernel against the fp32 oracle (which runs the reference plan:
    materialised scores, softmax row kernel, PV product) and against this backend's
    own unfused three-kernel plan.  The "eight_waves" cases force the ping-pong schedule,
    which the layout rule otherwise keeps for grids of at least 256 workgroups."""
    if shapes[0][-2] >= 512 and shapes[0][-1] % 64 == 0 and shapes[2][-1] % 64 == 0:
        monkeypatch.setenv("TENSORJIT_HIP_ATTENTION_WAVES", "8")
    torch.manual_seed(0)
    q, k, v = [torch.randn(sh, device=DEV).to(dt) for sh in shapes]
    print(f"attention {shapes} {dt}", flush=True)
    f = tj.jit(ATTN)
    out = f(q, k, v)
    cp = f.compiled(q, k, v)
    assert cp.num_kernels == 1 and "attention" in cp.launches[0].name
    (ref,) = oracle.run(ATTN, *[t.float().cpu() for t in (q, k, v)])
    close_lowp(out, ref, tol=2e-2, what="fused vs fp32 oracle")
    monkeypatch.setenv("TENSORJIT_HIP_ATTENTION", "0")
    f3 = tj.jit(ATTN)
    out3 = f3(q, k, v)
    assert f3.compiled(q, k, v).num_kernels == 3
    # the unfused plan stores its scores and probabilities in the storage type (the fused
    # kernel keeps both in fp32): it is held to the float64 emulation of those stores
    close_lowp(out3, attention_plan_reference(q, k, v, lambda t: t * 0.125, dt), what="unfused vs emulated plan")


def _mha(x, wq, wk, wv, heads):
    B, S, Dm = x.shape
    d = Dm // heads
    q = tj.linear(x, wq).reshape(B, S, heads, d).transpose(1, 2)
    k = tj.linear(x, wk).reshape(B, S, heads, d).transpose(1, 2)
    v = tj.linear(x, wv).reshape(B, S, heads, d).transpose(1, 2)
    o = tj.matmul(tj.softmax(tj.matmul(q, k.transpose(-1, -2)) * (1.0 / d ** 0.5)), v)
    return o.transpose(1, 2).reshape(B, S, Dm)


@pytest.mark.parametrize("B,S,Dm,heads,waves", [(2, 200, 128, 2, "4"), (1, 600, 256, 4, "8"), (1, 600, 512, 4, "8")],
                         ids=["4_waves", "pingpong", "pingpong_dma_16x16x32"])
def test_fused_attention_reads_and_writes_head_interleaved_layout(B, S, Dm, heads, waves, monkeypatch):
    """Multi-head attention with the head transposes folded into the flash kernel's
    strided loads and stores (no copy kernels), against the fp32 oracle."""
    monkeypatch.setenv("TENSORJIT_HIP_ATTENTION_WAVES", waves)
    torch.manual_seed(0)
    x = torch.randn(B, S, Dm, device=DEV).bfloat16()
    ws = [(torch.randn(Dm, Dm, device=DEV) / Dm ** 0.5).bfloat16() for _ in range(3)]
    fn = lambda x, a, b, c: _mha(x, a, b, c, heads)  # noqa: E731
    f = tj.jit(fn)
    out = f(x, *ws)
    cp = f.compiled(x, *ws)
    assert [l.meta["family"] for l in cp.launches].count("attention") == 1 and cp.num_kernels == 4
    (ref,) = oracle.run(fn, *[t.float().cpu() for t in (x, *ws)])
    # norm bound 1e-2: q and k are stored in bf16 by their projection kernels, and a logit
    # rounded by up to 2^-8 relative moves its probability by that times |s|
    close_lowp(out, ref, tol=2e-2, norm=1e-2)


def test_fused_attention_scale_written_as_division():
    """``q @ kᵀ / sqrt(d)`` with a head dim whose square root is not a power of two (the
    kernel multiplies by the rounded reciprocal; the oracle divides), against the fp32 oracle."""
    torch.manual_seed(2)
    q, k, v = [torch.randn(1, 3, 200, 96, device=DEV).bfloat16() for _ in range(3)]
    fn = lambda q, k, v: tj.matmul(tj.softmax(tj.matmul(q, tj.transpose(k, -1, -2)) / 96 ** 0.5), v)  # noqa: E731
    print("attention / sqrt(96)", flush=True)
    f = tj.jit(fn)
    out = f(q, k, v)
    assert f.compiled(q, k, v).num_kernels == 1
    (ref,) = oracle.run(fn, *[t.float().cpu() for t in (q, k, v)])
    close_lowp(out, ref, tol=2e-2)


@pytest.mark.parametrize("shapes", [[(1, 2, 300, 64)] * 3, [(1, 2, 600, 128), (1, 2, 1000, 128), (1, 2, 1000, 128)]],
                         ids=["four_waves", "pingpong_ragged"])
def test_fused_attention_negative_scale(shapes, monkeypatch):
    """A negative score scale: the block extreme is the raw minimum (masked keys +inf),
    the running maximum is still taken over scaled scores."""
    monkeypatch.setenv("TENSORJIT_HIP_ATTENTION_WAVES", "8" if shapes[0][-2] >= 512 else "4")
    torch.manual_seed(3)
    q, k, v = [torch.randn(sh, device=DEV).bfloat16() for sh in shapes]
    fn = lambda q, k, v: tj.matmul(tj.softmax(tj.matmul(q, tj.transpose(k, -1, -2)) * -0.2), v)  # noqa: E731
    print(f"attention negative scale {shapes}", flush=True)
    f = tj.jit(fn)
    out = f(q, k, v)
    assert f.compiled(q, k, v).num_kernels == 1
    (ref,) = oracle.run(fn, *[t.float().cpu() for t in (q, k, v)])
    close_lowp(out, ref, tol=2e-2)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("Sk", [40, 64, 100, 128, 192, 256, 300, 448, 520, 1000])
def test_dma_flash_kernel_equals_the_register_staged_one(Sk, dt, monkeypatch):
    """Head dim 128 on the ping-pong schedule, 1-16 key blocks, ragged and not: the kernel
    whose K and V blocks go into LDS by DMA (4 swizzled stages, a peeled tail of up to 7
    blocks) gives the register-staged kernel's output bit for bit (the same arithmetic in
    the same order; keys past the end read zeros instead of the last key, and their
    probabilities are 0 either way), and is within the flash bound of the fp32 oracle.
    Both on 32x32x16 MFMAs (the DMA kernel's 16x16x32 form is checked below)."""
    monkeypatch.setenv("TENSORJIT_HIP_ATTENTION_WAVES", "8")
    monkeypatch.setenv("TENSORJIT_HIP_ATTENTION_MI16", "0")
    torch.manual_seed(Sk)
    shapes = [(1, 2, 512, 128), (1, 2, Sk, 128), (1, 2, Sk, 128)]
    q, k, v = [torch.randn(sh, device=DEV).to(dt) for sh in shapes]
    print(f"DMA attention Sk={Sk} {dt}", flush=True)
    f = tj.jit(ATTN)
    out = f(q, k, v)
    assert f.compiled(q, k, v).launches[0].meta["schedule"] == "pingpong-dma"
    monkeypatch.setenv("TENSORJIT_HIP_ATTENTION_DMA", "0")
    f0 = tj.jit(ATTN)
    out0 = f0(q, k, v)
    assert f0.compiled(q, k, v).launches[0].meta["schedule"] == "pingpong"
    assert torch.equal(out, out0)
    (ref,) = oracle.run(ATTN, *[t.float().cpu() for t in (q, k, v)])
    close_lowp(out, ref, tol=2e-2)


@pytest.mark.parametrize("balance", ["1", "0"])
@pytest.mark.parametrize("scale", [0.088, -0.2])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("Sq,Sk", [(512, 40), (512, 64), (512, 100), (512, 192), (512, 300), (512, 520), (512, 1000),
                                   (512, 2048), (600, 333), (1000, 2000)])
def test_dma_flash_kernel_on_16x16x32_mfmas(Sq, Sk, dt, scale, balance, monkeypatch):
    """The DMA kernel's default 16x16x32 form (two 16-query tiles per wave, a query's keys
    on four lanes, combined over lanes l ^ 16 and l ^ 32 when the reference moves), 1-32
    key blocks, ragged and not, query counts short of the 256-row tile, positive and
    negative scale, row sums from the 16-bit probabilities in the PV phase (default) or in
    fp32 in the softmax phase: within the flash bound of the
    fp32 oracle, and close to the 32x32x16 form: one 16-bit rounding step of the output
    plus 2^-9 of its RMS (the two forms sum in other orders, and since a lane's keys
    differ between them, the lazy rescale may move the running reference at other
    blocks, so the probabilities round differently)."""
    monkeypatch.setenv("TENSORJIT_HIP_ATTENTION_WAVES", "8")
    monkeypatch.setenv("TENSORJIT_HIP_ATTENTION_BALANCE", balance)
    torch.manual_seed(1000 + Sk)
    shapes = [(1, 2, Sq, 128), (1, 2, Sk, 128), (1, 2, Sk, 128)]
    q, k, v = [torch.randn(sh, device=DEV).to(dt) for sh in shapes]
    fn = lambda q, k, v: tj.matmul(tj.softmax(tj.matmul(q, tj.transpose(k, -1, -2)) * scale), v)  # noqa: E731
    print(f"DMA attention 16x16x32 Sq={Sq} Sk={Sk} {dt} scale={scale} balance={balance}", flush=True)
    monkeypatch.setenv("TENSORJIT_HIP_ATTENTION_MI16", "1")
    f = tj.jit(fn)
    out = f(q, k, v)
    meta = f.compiled(q, k, v).launches[0].meta
    assert meta["schedule"] == "pingpong-dma" and meta["mfma"] == "16x16x32", meta
    assert meta["row_sums"] == ("16-bit" if balance == "1" else "fp32"), meta
    monkeypatch.setenv("TENSORJIT_HIP_ATTENTION_MI16", "0")
    f32 = tj.jit(fn)
    out32 = f32(q, k, v)
    assert f32.compiled(q, k, v).launches[0].meta["mfma"] == "32x32x16"
    (ref,) = oracle.run(fn, *[t.float().cpu() for t in (q, k, v)])
    close_lowp(out, ref, tol=2e-2)
    step = 2.0 ** -7 if dt == torch.bfloat16 else 2.0 ** -10
    o32 = out32.float()
    d = (out.float() - o32).abs()
    bound = step * o32.abs() + 2.0 ** -9 * float(o32.pow(2).mean().sqrt())
    assert bool((d <= bound).all()), float((d - bound).max())


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shapes,scale,splits", [
    ([(2, 2, 1000, 128)] * 3, 0.088, None),                                   # ragged last block, 8 splits
    ([(1, 1, 4096, 128)] * 3, 0.088, None),                                   # one head, 32 splits
    ([(1, 3, 200, 64), (1, 3, 2000, 64), (1, 3, 2000, 128)], 0.125, None),    # Dv != D, ragged
    ([(1, 2, 300, 64), (1, 2, 1280, 64), (1, 2, 1280, 64)], -0.2, "4"),        # negative scale, forced
    ([(2, 2, 1, 128), (2, 2, 2048, 128), (2, 2, 2048, 128)], 0.088, "2"),      # one query row
], ids=["ragged_8", "one_head_32", "dv128_ragged", "negative_scale_4", "single_query_2"])
def test_key_split_attention_vs_oracle(shapes, scale, splits, dt, monkeypatch):
    """Key-range splits for grids short of the CUs: partial rows with their running
    references and sums in the workspace, a second launch combining them, against the
    fp32 oracle of the reference plan."""
    if splits:
        monkeypatch.setenv("TENSORJIT_HIP_ATTENTION_SPLITS", splits)
    torch.manual_seed(5)
    q, k, v = [torch.randn(sh, device=DEV).to(dt) for sh in shapes]
    fn = lambda q, k, v: tj.matmul(tj.softmax(tj.matmul(q, tj.transpose(k, -1, -2)) * scale), v)  # noqa: E731
    print(f"split attention {shapes} {scale} {splits} {dt}", flush=True)
    f = tj.jit(fn)
    out = f(q, k, v)
    cp = f.compiled(q, k, v)
    fam = [l.meta["family"] for l in cp.launches]
    assert fam == ["attention", "attention_combine"] and cp.launches[0].meta["splits"] > 1, fam
    if splits:
        assert cp.launches[0].meta["splits"] == int(splits)
    (ref,) = oracle.run(fn, *[t.float().cpu() for t in (q, k, v)])
    close_lowp(out, ref, tol=2e-2)


def test_key_split_attention_with_head_interleaved_layout():
    """Splits with the head transposes folded into the kernel ([B,S,H,D] reads, the
    combine writes [B,S,H,Dv] rows), against the fp32 oracle."""
    torch.manual_seed(6)
    B, S, Dm, heads = 1, 1024, 256, 2
    x = torch.randn(B, S, Dm, device=DEV).bfloat16()
    ws = [(torch.randn(Dm, Dm, device=DEV) / Dm ** 0.5).bfloat16() for _ in range(3)]
    fn = lambda x, a, b, c: _mha(x, a, b, c, heads)  # noqa: E731
    f = tj.jit(fn)
    out = f(x, *ws)
    cp = f.compiled(x, *ws)
    fam = [l.meta["family"] for l in cp.launches]
    assert "attention_combine" in fam and "copy" not in fam, fam
    (ref,) = oracle.run(fn, *[t.float().cpu() for t in (x, *ws)])
    close_lowp(out, ref, tol=2e-2)


def test_two_fused_attention_layers_in_one_program():
    """Two attention cores in one program (the second reads the first's output as its
    queries): two flash kernels in one module, against the fp32 oracle."""
    torch.manual_seed(4)
    q, k, v = [torch.randn(2, 3, 300, 64, device=DEV).bfloat16() for _ in range(3)]

    def att(q, k, v):
        return tj.matmul(tj.softmax(tj.matmul(q, tj.transpose(k, -1, -2)) * 0.125), v)

    fn = lambda q, k, v: att(att(q, k, v), k, v)  # noqa: E731
    print("two attention layers", flush=True)
    f = tj.jit(fn)
    out = f(q, k, v)
    assert [l.meta["family"] for l in f.compiled(q, k, v).launches] == ["attention", "attention"]
    (ref,) = oracle.run(fn, *[t.float().cpu() for t in (q, k, v)])
    close_lowp(out, ref, tol=2e-2)


def test_fused_attention_large_logits_and_unit_scale():
    """Scores of magnitude ~100 (online max subtraction must keep exp2 in range) and
    no scale multiply in the chain."""
    torch.manual_seed(1)
    q = (3 * torch.randn(2, 256, 64, device=DEV)).bfloat16()
    k = (3 * torch.randn(2, 640, 64, device=DEV)).bfloat16()
    v = torch.randn(2, 640, 96, device=DEV).bfloat16()
    fn = lambda q, k, v: tj.matmul(tj.softmax(tj.matmul(q, tj.transpose(k, -1, -2))), v)  # noqa: E731
    f = tj.jit(fn)
    out = f(q, k, v)
    assert f.compiled(q, k, v).num_kernels == 1
    ref = torch.softmax(q.float() @ k.float().transpose(-1, -2).contiguous(), -1) @ v.float()
    assert torch.isfinite(out.float()).all()
    close_lowp(out, ref, tol=3e-2)


# ------------------------------------------------------------------ programs / executor

MLP = lambda x, g, w1, b1, w2, b2: x + tj.linear(tj.gelu(tj.linear(tj.layer_norm(x, g), w1, b1)), w2, b2)  # noqa: E731


@pytest.mark.parametrize("use_graph", [False, True])
def test_mlp_matches_eager_with_and_without_graph(use_graph, monkeypatch):
    monkeypatch.setenv("TENSORJIT_HIP_GRAPH", "1" if use_graph else "0")
    torch.manual_seed(0)
    x, g = torch.randn(64, 128, device=DEV), torch.ones(128, device=DEV)
    w1, b1 = torch.randn(256, 128, device=DEV), torch.randn(256, device=DEV)
    w2, b2 = torch.randn(128, 256, device=DEV), torch.randn(128, device=DEV)
    f = tj.jit(MLP)
    out = f(x, g, w1, b1, w2, b2)
    ref = x + F.linear(F.gelu(F.linear(F.layer_norm(x, (128,), g), w1, b1)), w2, b2)
    torch.testing.assert_close(out, ref, atol=2e-3, rtol=2e-3)
    out2 = f(x + 1, g, w1, b1, w2, b2)
    ref2 = (x + 1) + F.linear(F.gelu(F.linear(F.layer_norm(x + 1, (128,), g), w1, b1)), w2, b2)
    torch.testing.assert_close(out2, ref2, atol=2e-3, rtol=2e-3)
    cp = f.compiled(x, g, w1, b1, w2, b2)
    assert cp.stats["graph_replays"] == (2 if use_graph else 0)
    assert cp.num_kernels == 3 and "__global__" in cp.source


def test_native_program_counts_calls_and_owns_the_planned_arena(monkeypatch):
    """The reference's native-runtime test (tests/test_runtime_and_planner.py:61-77) for the
    hip executor: three kernels, eager-equal output, one native call per program call, and an
    arena of exactly the planned intermediates (plus split-K workspaces) in one allocation."""
    from tensorjit.backends import hip_backend as hb

    monkeypatch.setenv("TENSORJIT_HIP_GRAPH", "0")
    torch.manual_seed(0)
    x, g = torch.randn(64, 128, device=DEV), torch.ones(128, device=DEV)
    w1, b1 = torch.randn(256, 128, device=DEV), torch.randn(256, device=DEV)
    w2, b2 = torch.randn(128, 256, device=DEV), torch.randn(128, device=DEV)
    f = tj.jit(MLP)
    out = f(x, g, w1, b1, w2, b2)
    cp = f.compiled(x, g, w1, b1, w2, b2)
    ref = x + F.linear(F.gelu(F.linear(F.layer_norm(x, (128,), g), w1, b1)), w2, b2)
    torch.testing.assert_close(out, ref, atol=2e-3, rtol=2e-3)
    st = cp.native_stats()
    assert cp.num_kernels == 3 and st["calls"] == 1 and st["graph_replays"] == 0 and st["host_us"] > 0
    ptr, nbytes = cp.native.arena()
    assert ptr != 0 and nbytes == cp.arena_bytes == hb.workspace_layout(cp.launches, cp.plan.arena_bytes)[1]
    assert cp.plan.arena_bytes == 64 * 128 * 4 + 64 * 256 * 4     # LayerNorm and gelu outputs


def test_graph_replay_is_the_default_from_twelve_launches(monkeypatch):
    """Without TENSORJIT_HIP_GRAPH a program replays a hipGraph when it has at least
    GRAPH_MIN_LAUNCHES launches per call (measured crossover of launch cost vs graph cost)
    and launches directly below that; the variable forces either way."""
    from tensorjit.backends.hip_backend import GRAPH_MIN_LAUNCHES

    monkeypatch.delenv("TENSORJIT_HIP_GRAPH", raising=False)
    x, w = torch.randn(16, 32, device=DEV), torch.randn(32, 32, device=DEV)

    def chain(n):
        def fn(a, b):
            for _ in range(n):
                a = tj.softmax(tj.matmul(a, b) + 0.5)
            return a
        return fn

    ref8 = x
    for _ in range(8):
        ref8 = torch.softmax(ref8 @ w + 0.5, -1)
    long_, short = tj.jit(chain(8)), tj.jit(chain(2))
    for _ in range(3):
        torch.testing.assert_close(long_(x, w), ref8, atol=1e-5, rtol=1e-5)
        short(x, w)
    cl, cs = long_.compiled(x, w), short.compiled(x, w)
    assert len(cl.launches) == 16 >= GRAPH_MIN_LAUNCHES > len(cs.launches) == 4
    assert cl.use_graph and cl.stats["graph_replays"] == 3
    assert not cs.use_graph and cs.stats["graph_replays"] == 0
    monkeypatch.setenv("TENSORJIT_HIP_GRAPH", "0")
    assert not tj.jit(chain(8)).compiled(x, w).use_graph
    monkeypatch.setenv("TENSORJIT_HIP_GRAPH", "1")
    assert tj.jit(chain(2)).compiled(x, w).use_graph


def test_graph_replays_match_eager_every_time(monkeypatch):
    monkeypatch.setenv("TENSORJIT_HIP_GRAPH", "1")
    torch.manual_seed(0)
    x = torch.randn(128, 768, device=DEV)
    args = [torch.ones(768, device=DEV), torch.randn(3072, 768, device=DEV) * 0.02, torch.randn(3072, device=DEV) * 0.02,
            torch.randn(768, 3072, device=DEV) * 0.02, torch.randn(768, device=DEV) * 0.02]
    f = tj.jit(MLP)
    first = f(x, *args).clone()
    for i in range(5):
        y = f(x, *args)
        torch.cuda.synchronize()
        assert torch.equal(y, first), i
        _ = (x * 2).sum().item()          # eager work between replays
    cp = f.compiled(x, *args)
    assert cp.native_stats()["graph_captures"] <= 3 and cp.stats["graph_replays"] == 6


def test_graph_captures_stay_bounded_when_the_caller_keeps_its_outputs(monkeypatch):
    """A 16-launch program replays hipGraphs by default; a caller that keeps every output
    presents a new pointer set on each call.  After 4 captures in a row the runtime
    launches such calls directly (no capture, no instantiation) and captures a pointer
    set only when it recurs, so graph mode comes back once the caller drops its outputs
    and the pool hands the same buffer out again.  Every output is bit-identical."""
    monkeypatch.delenv("TENSORJIT_HIP_GRAPH", raising=False)
    torch.manual_seed(0)
    x, w = torch.randn(16, 32, device=DEV), torch.randn(32, 32, device=DEV)

    def fn(a, b):
        for _ in range(8):
            a = tj.softmax(tj.matmul(a, b) + 0.5)
        return a

    f = tj.jit(fn)
    cp = f.compiled(x, w)
    assert cp.use_graph and len(cp.launches) == 16
    kept = [f(x, w) for _ in range(12)]
    torch.cuda.synchronize()
    st = cp.stats
    assert st["graph_captures"] == 4 and st["graph_replays"] == 4 and st["direct_fallbacks"] == 8, st
    first = kept[0].clone()
    assert all(torch.equal(k, first) for k in kept)
    del kept
    for _ in range(6):
        out = f(x, w)
        torch.cuda.synchronize()
        assert torch.equal(out, first)
        del out
    st2 = cp.stats
    assert st2["graph_replays"] - st["graph_replays"] >= 4 and st2["graph_captures"] - st["graph_captures"] <= 2, st2


def test_graph_replays_of_split_column_and_wide_row_kernels(monkeypatch):
    """A program of 13 launches (column sums, maxima and means, split row sums and means,
    a 16384-wide LayerNorm) replays as a hipGraph by default (12 launches and more): every
    replay, with eager work in between, matches the first call bit for bit and the eager
    results to rounding."""
    monkeypatch.delenv("TENSORJIT_HIP_GRAPH", raising=False)
    torch.manual_seed(0)
    x, y = torch.randn(4096, 2048, device=DEV), torch.randn(4, 1 << 20, device=DEV)
    z, g = torch.randn(32, 16384, device=DEV), 1 + 0.1 * torch.randn(16384, device=DEV)

    def fn(a, b, c, w):
        return (tj.sum(a, axis=0), tj.max(a, axis=0), tj.mean(a * a, axis=0), tj.sum(b, axis=-1),
                tj.mean(tj.abs(b), axis=-1), tj.max(b, axis=-1), tj.layer_norm(c, w))

    f = tj.jit(fn)
    cp = f.compiled(x, y, z, g)
    assert len(cp.launches) == 13 and cp.use_graph
    first = [t.clone() for t in f(x, y, z, g)]
    ref = (x.sum(0), x.amax(0), (x * x).mean(0), y.sum(-1), y.abs().mean(-1), y.amax(-1),
           F.layer_norm(z, (16384,), g))
    for r, o in zip(ref, first):
        torch.testing.assert_close(o, r, rtol=1e-4, atol=1e-4)
    for i in range(4):
        outs = f(x, y, z, g)
        torch.cuda.synchronize()
        assert all(torch.equal(o, p) for o, p in zip(outs, first)), i
        _ = (x * 2).sum().item()          # eager work between replays
    assert cp.stats["graph_replays"] >= 4


def test_transformer_block_small():
    torch.manual_seed(0)
    T_, D, H = 12, 32, 64
    t = [torch.randn(s, device=DEV) for s in [(T_, D), (D,), (H, D), (H,), (D, H), (D,), (D, D), (D, D)]]

    def block(x, ln_g, w1, b1, w2, b2, wq, wk):
        h = tj.layer_norm(x, ln_g)
        q, k = tj.linear(h, wq), tj.linear(h, wk)
        scores = tj.softmax(tj.matmul(q, k.T) * (1.0 / 8.0))
        return x + tj.linear(tj.gelu(tj.linear(h, w1, b1)), w2, b2), scores

    f, (out, sc) = check_vs_oracle(block, *t, rtol=1e-4, scale=1e-4)
    assert f.compiled(*t).num_kernels < 20


def test_specialisation_cache_hits_and_recompiles():
    f = tj.jit(lambda a: tj.exp(a) + 1.0)
    x = torch.randn(8, device=DEV)
    f(x)
    f(x)
    assert f.stats.compiles == 1 and f.stats.hits == 1
    f(torch.randn(9, device=DEV))
    assert f.stats.compiles == 2


def test_output_buffers_reused_only_when_dropped(monkeypatch):
    monkeypatch.setenv("TENSORJIT_HIP_GRAPH", "0")
    f = tj.jit(lambda a: tj.exp(a))
    x = torch.randn(256, 512, device=DEV)
    a = f(x)
    view = a[:3]
    b = f(x + 1)
    assert a.data_ptr() != b.data_ptr()
    del view
    c = f(x + 2)
    assert c.data_ptr() not in (a.data_ptr(), b.data_ptr())
    pa = a.data_ptr()
    del a
    d = f(x + 3)
    assert d.data_ptr() == pa
    torch.testing.assert_close(b, torch.exp(x + 1))
    torch.testing.assert_close(c, torch.exp(x + 2))
    torch.testing.assert_close(d, torch.exp(x + 3))


def test_reshape_and_const_outputs_and_bad_inputs():
    x = torch.randn(3, 4, 5, device=DEV)
    f = tj.jit(lambda t: (tj.exp(t).reshape(5, 12), tj.sum(t * 0.0 + 2.0)))
    a, b = f(x)
    torch.testing.assert_close(a, torch.exp(x).reshape(5, 12))
    torch.testing.assert_close(b, torch.full((3, 4), 10.0, device=DEV))
    g = tj.jit(lambda t: tj.exp(t))
    g(torch.randn(8, device=DEV))
    with pytest.raises(TypeError):
        g.compiled(torch.randn(8, device=DEV))(torch.randn(8, device=DEV), torch.randn(8, device=DEV))


def test_misaligned_input_view_is_handled():
    x = torch.randn(1025, device=DEV)[1:]          # contiguous but 4-byte offset
    f = tj.jit(lambda t: tj.exp(t) * 2.0)
    torch.testing.assert_close(f(x), torch.exp(x) * 2)


def test_zero_size_inputs_are_refused_without_a_launch():
    """An empty tensor never reaches a kernel: tj.jit raises NotImplementedError while
    compiling, and torch.compile (not strict) falls back to eager for that graph."""
    torch._dynamo.reset()
    f = tj.jit(lambda a: tj.exp(a) + 1.0)
    with pytest.raises(NotImplementedError, match="zero-size"):
        f(torch.empty(0, 4, device=DEV))

    def g(a):
        return torch.exp(a) + 1.0

    c = torch.compile(g, backend=tj.torch_compile_backend, dynamic=False)
    x = torch.empty(0, 4, device=DEV)
    out = c(x)
    assert out.shape == (0, 4) and out.device == x.device
    torch._dynamo.reset()


def test_torch_compile_backend_matches_eager(monkeypatch):
    monkeypatch.setenv("TENSORJIT_STRICT", "1")
    torch.manual_seed(0)
    torch._dynamo.reset()

    class Block(torch.nn.Module):
        def __init__(self, d=32, h=64):
            super().__init__()
            self.ln = torch.nn.LayerNorm(d)
            self.fc1 = torch.nn.Linear(d, h)
            self.fc2 = torch.nn.Linear(h, d)
            self.drop = torch.nn.Dropout(0.0)

        def forward(self, x):
            h = self.drop(F.gelu(self.fc1(self.ln(x))))
            y = x + self.fc2(h)
            return torch.softmax(y, dim=-1) * 2 + y.mean(dim=-1, keepdim=True)

    m = Block().to(DEV).eval()
    x = torch.randn(16, 32, device=DEV)
    c = torch.compile(m, backend=tj.torch_compile_backend)
    with torch.no_grad():
        torch.testing.assert_close(c(x), m(x), atol=1e-4, rtol=1e-4)


def test_torch_compile_op_coverage_strict(monkeypatch):
    """FX graphs built from the mapped torch functions / tensor methods compile to hip
    kernels under TENSORJIT_STRICT=1 (no eager fallback) and match eager."""
    monkeypatch.setenv("TENSORJIT_STRICT", "1")
    torch.manual_seed(0)
    torch._dynamo.reset()

    def fn(x, y, w):
        a = torch.tanh(x) + torch.sigmoid(y) * torch.relu(x - 0.5)
        b = torch.rsqrt(torch.abs(y) + 1.0) ** 2.0 - torch.exp(-x.abs())
        c = (torch.maximum(a, b) * 0.75 + torch.minimum(a, b) * 0.25).clamp_min(-0.25)
        d = (c @ w).t().contiguous()
        e = torch.softmax(d.transpose(0, 1) * 0.5, dim=-1) + d.t().amax(dim=-1, keepdim=True)
        return e.sum(dim=-1) + e.mean(dim=-1) * F.silu(e).sum(dim=-1), torch.log(torch.sqrt(a * a + 1.0))

    x, y, w = torch.randn(48, 40, device=DEV), torch.randn(48, 40, device=DEV), torch.randn(40, 24, device=DEV)
    c = torch.compile(fn, backend=tj.torch_compile_backend)
    got, ref = c(x, y, w), fn(x, y, w)
    for g_, r_ in zip(got, ref):
        torch.testing.assert_close(g_, r_, atol=2e-4, rtol=2e-4)


def test_torch_compile_reaches_column_split_and_wide_row_kernels(monkeypatch):
    """Under torch.compile (TENSORJIT_STRICT=1, no eager fallback): a batch mean over dim 0
    (a column reduction), an MSE loss over a whole [2048, 1024] tensor (one long row, split
    over workgroups) and a LayerNorm over rows of 16384 (one row kernel) match eager."""
    from tensorjit.backends import hip_backend as hb

    monkeypatch.setenv("TENSORJIT_STRICT", "1")
    torch.manual_seed(0)
    torch._dynamo.reset()
    fams = []
    orig = hb.HipProgram.__init__

    def spy(self, *a, **kw):
        orig(self, *a, **kw)
        fams.extend(l.meta["family"] for l in self.launches)

    monkeypatch.setattr(hb.HipProgram, "__init__", spy)

    def fn(x, y, z, g):
        return x.mean(dim=0), ((x - y) ** 2.0).mean(), F.layer_norm(z, (z.shape[-1],), g)

    x, y = torch.randn(2048, 1024, device=DEV), torch.randn(2048, 1024, device=DEV)
    z, g = torch.randn(64, 16384, device=DEV), 1 + 0.1 * torch.randn(16384, device=DEV)
    c = torch.compile(fn, backend=tj.torch_compile_backend)
    got, ref = c(x, y, z, g), fn(x, y, z, g)
    for g_, r_ in zip(got, ref):
        torch.testing.assert_close(g_, r_, atol=2e-4, rtol=2e-4)
    assert {"colreduce", "row_combine", "row"} <= set(fams), fams


def test_torch_compile_attention_module_runs_the_flash_kernel(monkeypatch):
    """An attention nn.Module in bf16 under torch.compile lands on the fused kernel."""
    monkeypatch.setenv("TENSORJIT_STRICT", "1")
    torch.manual_seed(0)
    torch._dynamo.reset()
    import tensorjit.frontend.torch_backend as tb

    compiled_programs = []
    orig = tb.compile_graph

    def spy(*a, **kw):
        prog = orig(*a, **kw)
        compiled_programs.append(prog)
        return prog

    monkeypatch.setattr(tb, "compile_graph", spy)

    class Attn(torch.nn.Module):
        def forward(self, q, k, v):
            return torch.softmax(q @ k.transpose(-1, -2) * 0.125, dim=-1) @ v

    q, k, v = [torch.randn(2, 4, 256, 64, device=DEV).bfloat16() for _ in range(3)]
    out = torch.compile(Attn(), backend=tj.torch_compile_backend)(q, k, v)
    qf, kf, vf = q.float(), k.float(), v.float()
    ref = torch.softmax(qf @ kf.transpose(-1, -2).contiguous() * 0.125, dim=-1) @ vf
    close_lowp(out, ref, tol=2e-2)
    assert any(any("attention" in l.name for l in p.launches) for p in compiled_programs)


# ------------------------------------------------------------------ benchmark configs at full size


def test_config2_full_size_fp32_vs_oracle():
    torch.manual_seed(0)
    x = torch.randn(16384, 4096, device=DEV)
    a, b = torch.randn(4096, device=DEV), torch.randn(4096, device=DEV)
    c = torch.rand(16384, 4096, device=DEV) * 8 - 4
    check_vs_oracle(lambda x, a, b, c: tj.gelu(x * a + b) * tj.sigmoid(c) + x, x, a, b, c)


def test_config2_full_size_bf16_vs_oracle():
    """Config 2 in bf16 at its full shape (the bench's `c2_eltwise_bf16` line): one pointwise
    kernel, fp32 arithmetic on bf16 loads, one bf16 rounding at the store, against the fp32
    oracle of the same (upcast) inputs."""
    torch.manual_seed(0)
    x = torch.randn(16384, 4096, device=DEV).bfloat16()
    a, b = torch.randn(4096, device=DEV).bfloat16(), torch.randn(4096, device=DEV).bfloat16()
    c = (torch.rand(16384, 4096, device=DEV) * 8 - 4).bfloat16()
    f, _ = check_vs_oracle(lambda x, a, b, c: tj.gelu(x * a + b) * tj.sigmoid(c) + x, x, a, b, c)
    assert f.compiled(x, a, b, c).num_kernels == 1


def test_config3_full_size_rows_vs_oracle():
    torch.manual_seed(0)
    x = torch.randn(65536, 4096, device=DEV).bfloat16()
    g = (1 + 0.1 * torch.randn(4096, device=DEV)).bfloat16()
    check_vs_oracle(lambda x, g: tj.layer_norm(x, g), x, g)
    check_vs_oracle(lambda x, g: tj.rms_norm(x, g), x, g)
    s = torch.randn(65536, 2048, device=DEV) * 3
    f, (sm,) = check_vs_oracle(lambda s: tj.softmax(s), s, scale=1e-6)
    # size-independent properties: rows sum to 1, argmax preserved
    torch.testing.assert_close(sm.sum(-1), torch.ones(65536, device=DEV), atol=1e-5, rtol=0)
    assert torch.equal(sm.argmax(-1), s.argmax(-1))


def test_config4_gemm_full_size_bf16_rows_vs_oracle():
    torch.manual_seed(0)
    x = torch.randn(8192, 8192, device=DEV).bfloat16()
    w = (0.02 * torch.randn(8192, 8192, device=DEV)).bfloat16()
    bias = (0.02 * torch.randn(8192, device=DEV)).bfloat16()
    f = tj.jit(lambda x, w, b: tj.gelu(tj.linear(x, w, b)))
    out = f(x, w, bias)
    # the oracle on a 64-row sample (rows are independent: same kernel, different tile)
    rows = torch.arange(0, 8192, 128, device=DEV)
    (orc,) = oracle.run(lambda x, w, b: tj.gelu(tj.linear(x, w, b)), x[rows].float().cpu(), w.float().cpu(),
                        bias.float().cpu())
    close_lowp(out[rows], orc, tol=2e-2)
    # and against the library GEMM on the whole output
    ref = F.gelu(F.linear(x.float(), w.float(), bias.float()))
    close_lowp(out, ref, tol=2e-2)


def test_config4_skinny_decode_full_size_vs_oracle():
    """Config 4's decode shape, 16 x 8192 x 8192 bf16 + bias + gelu, through ``tj.jit`` on its
    packaged tile (the streaming kernel, K split over the waves), against the oracle on the
    whole output."""
    torch.manual_seed(0)
    x = torch.randn(16, 8192, device=DEV).bfloat16()
    w = (0.02 * torch.randn(8192, 8192, device=DEV)).bfloat16()
    bias = (0.02 * torch.randn(8192, device=DEV)).bfloat16()
    fn = lambda x, w, b: tj.gelu(tj.linear(x, w, b))  # noqa: E731
    f = tj.jit(fn)
    out = f(x, w, bias)
    assert f.compiled(x, w, bias).matmul_configs[0].SPLIT_K > 1
    (orc,) = oracle.run(fn, x.float().cpu(), w.float().cpu(), bias.float().cpu())
    close_lowp(out, orc, tol=2e-2)


def test_config5_attention_full_size_sampled_heads():
    """Config 5's attention core at its full shape, [4, 32, 2048, 128] bf16 with the 1/sqrt(128)
    scale, through the fused flash kernel (8 waves, ping-pong, 32 key blocks), against an fp32
    reference on four (batch, head) pairs; the rows of every head sum the values with weights
    that sum to 1, so the output's mean over keys is also checked on all heads."""
    torch.manual_seed(0)
    q, k, v = [torch.randn(4, 32, 2048, 128, device=DEV).bfloat16() for _ in range(3)]
    fn = lambda q, k, v: tj.matmul(tj.softmax(tj.matmul(q, tj.transpose(k, -1, -2)) * (128 ** -0.5)), v)  # noqa: E731
    f = tj.jit(fn)
    out = f(q, k, v)
    cp = f.compiled(q, k, v)
    assert cp.num_kernels == 1 and "attention" in cp.launches[0].name
    for b, h in ((0, 0), (1, 7), (2, 19), (3, 31)):
        qf, kf, vf = q[b, h].float(), k[b, h].float(), v[b, h].float()
        ref = torch.softmax(qf @ kf.t().contiguous() * (128 ** -0.5), dim=-1) @ vf
        close_lowp(out[b, h], ref, tol=2e-2)
    # convex combinations of V's rows: every output lies inside V's per-column range
    lo, hi = v.float().amin(dim=2, keepdim=True), v.float().amax(dim=2, keepdim=True)
    o = out.float()
    assert bool(((o >= lo - 1e-2) & (o <= hi + 1e-2)).all())


def _config5_batch0_fp32(args):
    """Config 5's layer evaluated in float32 by torch for batch 0."""
    x, g1, wq, wk, wv, wo, g2, w1, w2 = [a.float() for a in args]
    x = x[:1]
    S, D, H = x.shape[1], x.shape[2], 32

    def rms(t, g):
        return t * torch.rsqrt((t * t).mean(-1, keepdim=True) + 1e-6) * g

    def heads(t):
        return t.reshape(1, S, H, D // H).transpose(1, 2).contiguous()

    h = rms(x, g1)
    q, k, v = heads(h @ wq.t().contiguous()), heads(h @ wk.t().contiguous()), heads(h @ wv.t().contiguous())
    pr = torch.softmax(q @ k.transpose(-1, -2).contiguous() * (D // H) ** -0.5, dim=-1)
    o = (pr @ v).transpose(1, 2).reshape(1, S, D)
    x = x + o @ wo.t().contiguous()
    return x + F.gelu(rms(x, g2) @ w1.t().contiguous()) @ w2.t().contiguous()


def test_config5_block_full_size_batch0_vs_fp32():
    """Config 5's layer at its full shape ([4, 2048, 4096], 32 heads x 128, MLP 11008, bf16) on
    the packaged tiles, against a float32 torch evaluation of the same layer for batch 0 (the
    batches are independent), at the default bf16 bounds: the layer stores bf16 between its
    9 kernels (q, k, v, attention output, residual stream, normed activations, gelu output)
    and lands 3.3e-3 from float32 in norm, 3.9e-3 in its worst row."""
    import bench

    args = bench.block_inputs(torch, torch.device(DEV))
    f = tj.jit(bench._fn_block)
    out = f(*args)
    assert f.compiled(*args).num_kernels == 9
    close_lowp(out[:1], _config5_batch0_fp32(args), tol=3e-2)


def test_config5_block_full_size_under_graph_replay(monkeypatch):
    """Config 5's layer at full size as the bench times it under ``TENSORJIT_HIP_GRAPH=1``:
    two hipGraph replays (eager work between them) bit-identical to direct launches of the
    same program, and batch 0 against the float32 evaluation."""
    import bench

    monkeypatch.setenv("TENSORJIT_HIP_GRAPH", "1")
    args = bench.block_inputs(torch, torch.device(DEV))
    f = tj.jit(bench._fn_block)
    cp = f.compiled(*args)
    assert cp.use_graph and cp.num_kernels == 9
    cp.use_graph = False
    direct = cp(*args)[0].clone()
    cp.use_graph = True
    replays = []
    for _ in range(2):
        replays.append(cp(*args)[0].clone())
        torch.cuda.synchronize()
        _ = (args[0] * 2).sum().item()          # eager work between replays
    assert cp.stats["graph_replays"] >= 2
    for r in replays:
        assert torch.equal(r, direct)
    close_lowp(replays[-1][:1], _config5_batch0_fp32(args), tol=3e-2)


def test_config5_block_with_fused_attention_vs_oracle():
    """Config 5's layer at head dim 64 (so the attention chain and its head transposes
    fuse into one flash kernel, and the second residual into the down-projection's
    epilogue: 9 kernels), bf16 vs the fp32 oracle of the reference plan, and hipGraph
    replays equal to eager launches."""
    import bench

    torch.manual_seed(0)
    args = bench.block_inputs(torch, torch.device(DEV), B=1, S=256, D=2048, F=512)
    f = tj.jit(bench._fn_block)
    out = f(*args)
    cp = f.compiled(*args)
    assert cp.num_kernels == 9 and any("attention" in l.name for l in cp.launches)
    (ref,) = oracle.run(bench._fn_block, *[a.float().cpu() for a in args])
    close_lowp(out, ref, tol=3e-2)
    cp.use_graph = False
    eager = cp(*args)[0].clone()
    cp.use_graph = True
    for _ in range(3):
        assert torch.equal(cp(*args)[0], eager)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_epilogue_reading_the_gemm_operand_is_exact(dt):
    """``x + linear(x, w)``: the residual is the product's own A operand (one kernel
    input read by the K loop and by the epilogue), on one tiling of each schedule --
    persistent / direct-to-LDS / ping-pong / register-staged / decode for 16-bit, 32x32
    and 16x16 tiles and a K split for fp32 -- exact on small-integer data (fp32 sums of
    integers are exact, rounded once to the storage type as the reference is)."""
    from tensorjit.backends import hip_backend as hb
    from tensorjit.runtime.autotune import MatmulConfig as C

    torch.manual_seed(0)
    if dt == torch.bfloat16:
        cases = [((512, 512), C(256, 256, 64, 4, 2, 2, 16, 1, 8, 0, 0, 1, 1, 8)),
                 ((512, 512), C(256, 256, 64, 4, 2, 2, 16, 1, 8, 0, 0, 1)),
                 ((300, 512), C(256, 256, 64, 8, 2, 4, 32, 1, 8, 3)),
                 ((300, 520), C(128, 128, 32, 4, 2, 2, 32)),
                 ((16, 4096), C(16, 32, 64, 4, 1, 1, 16, 4, 0)),
                 ((7, 520), C(16, 32, 64, 4, 1, 1, 16, 4, 0))]
    else:
        cases = [((300, 520), C(128, 128, 32, 4, 2, 2, 32)), ((300, 520), C(64, 64, 32, 4, 2, 2, 16)),
                 ((128, 512), C(64, 64, 32, 4, 2, 2, 16, 1, 8, 0, 0, 0, 4))]
    fn = lambda x, w: x + tj.linear(x, w)  # noqa: E731
    for (m, k), cfg in cases:
        x = torch.randint(-2, 3, (m, k), device=DEV).to(dt)
        w = torch.randint(-2, 3, (k, k), device=DEV).to(dt)
        mm = C_lower(fn, x, w).kernels[0].anchor
        assert hb.config_ok(cfg, hb.compute_dtype(mm), mm), cfg
        print(f"x + linear(x, w) {m}x{k} {cfg}", flush=True)
        out = _run_with_config(fn, [x, w], cfg)
        ref = (x.double() + x.double() @ w.double().t()).to(dt)
        assert torch.equal(out, ref), ((m, k), cfg)
    # the default path (tj.jit, packaged table / cost model) too
    x = torch.randint(-2, 3, (256, 512), device=DEV).to(dt)
    w = torch.randint(-2, 3, (512, 512), device=DEV).to(dt)
    assert torch.equal(tj.jit(fn)(x, w), (x.double() + x.double() @ w.double().t()).to(dt))


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_elementwise_kernel_behind_a_gemm_joins_its_epilogue(dt, monkeypatch):
    """``h + linear(relu(h), w2)`` with ``h = x + linear(x, w1)``: the reference plan
    leaves the last add as its own kernel (joining h's kernel would form a cycle); the
    backend moves it into the second GEMM's epilogue (2 kernels instead of 3), against
    the oracle of the reference plan, and the switch keeps the 3 kernels."""
    torch.manual_seed(0)
    x = torch.randn(256, 512, device=DEV).to(dt)
    w1, w2 = [(0.05 * torch.randn(512, 512, device=DEV)).to(dt) for _ in range(2)]
    fn = lambda x, a, b: (lambda h: h + tj.linear(tj.relu(h), b))(x + tj.linear(x, a))  # noqa: E731
    f = tj.jit(fn)
    out = f(x, w1, w2)
    assert f.compiled(x, w1, w2).num_kernels == 2
    (ref,) = oracle.run(fn, *[t.float().cpu() for t in (x, w1, w2)])
    if dt == torch.float32:
        close_f32(out, ref, scale=1e-5)
    else:
        close_lowp(out, ref, tol=2e-2)
    monkeypatch.setenv("TENSORJIT_HIP_GEMM_EPILOGUE", "0")
    f3 = tj.jit(fn)
    out3 = f3(x, w1, w2)
    assert f3.compiled(x, w1, w2).num_kernels == 3
    if dt == torch.float32:
        close_f32(out3, out, scale=1e-5)


def test_config5_transformer_block_small_bf16_vs_oracle():
    """Config 5's layer (RMSNorm, q/k/v, attention with materialised scores, out-proj +
    residual, RMSNorm, gelu MLP + residual) at a small shape, bf16 vs the fp32 oracle."""
    import bench

    torch.manual_seed(0)
    args = bench.block_inputs(torch, torch.device(DEV), B=2, S=64, D=256, F=512)
    f = tj.jit(bench._fn_block)
    out = f(*args)
    assert f.compiled(*args).num_kernels == 15          # the second residual joins the down-projection
    (ref,) = oracle.run(bench._fn_block, *[a.float().cpu() for a in args])
    close_lowp(out, ref, tol=3e-2)
    # graph replay of the same program gives the same bits as eager launches
    cp = f.compiled(*args)
    cp.use_graph = False
    eager = cp(*args)[0].clone()
    cp.use_graph = True
    for _ in range(3):
        assert torch.equal(cp(*args)[0], eager)


def _run_with_config(fn, args, cfg, calls=1):
    """Compile ``fn`` for ``args`` with its single matmul forced to tile config ``cfg``;
    ``calls`` > 1 runs that one program that many times and returns every output."""
    from tensorjit.backends import hip_backend as hb
    from tensorjit.compiler import lower
    from tensorjit.frontend.tracer import tensor_type_of
    from tensorjit.runtime import hip as rt

    p = lower(tj.trace(fn, [tensor_type_of(a) for a in args]), "hip")
    (k,) = p.kernels
    src, launches = hb.generate(p, {0: cfg})
    code = hb.compile_source(src, hb.arch_of(0))
    # the kernel's parameters follow its own input order, not the traced function's
    gin = {id(n): j for j, n in enumerate(p.graph.inputs)}
    order = [gin[id(p.resolve(n))] for n in k.inputs]
    assert [tuple(n.shape) for n in k.inputs] == [tuple(args[j].shape) for j in order]
    refs = [[(rt.INPUT, j) for j in order] + [(rt.OUTPUT, 0)]]
    ws, arena = hb.workspace_layout(launches, 0)          # split-K GEMMs: partials + a sum launch
    prog = rt.NativeHipProgram(0, code, [l.name for l in launches], [(l.grid, l.block, 0) for l in launches],
                               hb.launch_args(launches, refs, ws), arena, len(args), 1)
    outs = []
    for _ in range(calls):
        outs.append(torch.empty(k.outputs[0].shape, device=DEV, dtype=args[0].dtype))
        prog.run([a.data_ptr() for a in args], [outs[-1].data_ptr()], torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return outs[0] if calls == 1 else outs


@pytest.mark.parametrize("tb", [True, False])
def test_every_bf16_tile_config_is_exact_on_integer_data(tb):
    """Every candidate tiling (incl. the ping-pong schedule and the skinny kernel) on
    a shape with ragged M / N / K edges, exact on small-integer data."""
    from tensorjit.backends import hip_backend as hb
    from tensorjit.runtime.autotune import HIP_CANDIDATES

    torch.manual_seed(0)
    for m, n, kk in [(300, 520, 136), (100, 72, 40), (16, 200, 512), (300, 520, 192)]:
        a = torch.randint(-2, 3, (m, kk), device=DEV).bfloat16()
        b = torch.randint(-2, 3, (n, kk) if tb else (kk, n), device=DEV).bfloat16()
        fn = (lambda x, y: tj.linear(x, y)) if tb else (lambda x, y: tj.matmul(x, y))
        ref = (a.double() @ (b.double().t() if tb else b.double())).bfloat16()
        mm = C_lower(fn, a, b).kernels[0].anchor
        tried = 0
        for cfg in HIP_CANDIDATES:
            if not hb.config_ok(cfg, hb.compute_dtype(mm), mm):
                continue
            out = _run_with_config(fn, [a, b], cfg)
            assert torch.equal(out, ref), (m, n, kk, tb, cfg)
            tried += 1
        assert tried >= (3 if m > 16 else 1)


@pytest.mark.parametrize("tb", [True, False])
def test_every_fp32_tile_config_is_exact_on_integer_data(tb):
    """Every fp32 candidate tiling -- 32x32x2 and 16x16x4 MFMA tiles, K split over
    workgroups, direct-to-LDS tiles -- on shapes with ragged M / N / K edges, exact on
    small-integer data (every partial sum is an integer below 2^24, so any summation order
    gives the same bits)."""
    from tensorjit.backends import hip_backend as hb
    from tensorjit.runtime.autotune import HIP_F32_CANDIDATES

    torch.manual_seed(0)
    mi32 = ksplit = direct = 0
    for m, n, kk in [(300, 520, 136), (100, 72, 40), (130, 260, 1024)]:
        a = torch.randint(-2, 3, (m, kk), device=DEV).float()
        b = torch.randint(-2, 3, (n, kk) if tb else (kk, n), device=DEV).float()
        fn = (lambda x, y: tj.linear(x, y)) if tb else (lambda x, y: tj.matmul(x, y))
        ref = (a.double() @ (b.double().t() if tb else b.double())).float()
        mm = C_lower(fn, a, b).kernels[0].anchor
        tried = 0
        for cfg in HIP_F32_CANDIDATES:
            if not hb.config_ok(cfg, hb.compute_dtype(mm), mm):
                continue
            out = _run_with_config(fn, [a, b], cfg)
            assert torch.equal(out, ref), (m, n, kk, tb, cfg)
            tried += 1
            mi32 += cfg.MI == 32
            ksplit += cfg.KSPLIT > 1
            direct += cfg.DIRECT
        assert tried >= 4, (m, n, kk)
    assert mi32 >= 4 * 3 and ksplit >= 4 and direct >= (3 if tb else 0)


def test_config4_fp32_full_size_on_its_packaged_tile_vs_oracle():
    """Config 4's fp32 variant, gelu(x @ w.T + bias) at 4096^3, through ``tj.jit`` on the tile
    the packaged table holds for it (direct-to-LDS 128x128x32 with 16x16x4 MFMAs): the
    oracle on a 64-row sample at the fp32 bound, and a float64 product on the whole output."""
    from tensorjit.backends import hip_backend as hb
    from tensorjit.runtime.autotune import MatmulConfig
    from tensorjit.runtime.cache import packaged_entry

    torch.manual_seed(0)
    x = torch.randn(4096, 4096, device=DEV)
    w = 0.02 * torch.randn(4096, 4096, device=DEV)
    bias = 0.02 * torch.randn(4096, device=DEV)
    fn = lambda x, w, b: tj.gelu(tj.linear(x, w, b))  # noqa: E731
    f = tj.jit(fn)
    out = f(x, w, bias)
    cp = f.compiled(x, w, bias)
    entry = packaged_entry(hb.matmul_key(cp.program.kernels[0], cp.arch))
    assert entry is not None and cp.matmul_configs[0] == MatmulConfig.from_dict(entry["config"])
    assert cp.matmul_configs[0].DIRECT == 1 and cp.matmul_configs[0].MI == 16
    rows = torch.arange(0, 4096, 64, device=DEV)
    (orc,) = oracle.run(fn, x[rows].cpu(), w.cpu(), bias.cpu())
    close_f32(out[rows], orc)
    ref = F.gelu(F.linear(x.double(), w.double(), bias.double()))
    close_f32(out, ref)


@pytest.mark.parametrize("use_graph", [False, True])
def test_config1_mlp_full_size_vs_oracle(use_graph, monkeypatch):
    """Config 1, the README MLP block at [512, 768] -> 3072 fp32 on its packaged tiles (the
    down-projection split 4 ways over K), against the oracle at the fp32 bound -- on every
    call, in eager launches and in hipGraph replays."""
    monkeypatch.setenv("TENSORJIT_HIP_GRAPH", "1" if use_graph else "0")
    torch.manual_seed(0)
    x = torch.randn(512, 768, device=DEV)
    g = 1 + 0.1 * torch.randn(768, device=DEV)
    w1, b1 = 0.02 * torch.randn(3072, 768, device=DEV), 0.02 * torch.randn(3072, device=DEV)
    w2, b2 = 0.02 * torch.randn(768, 3072, device=DEV), 0.02 * torch.randn(768, device=DEV)
    args = [x, g, w1, b1, w2, b2]
    f = tj.jit(MLP)
    for step in range(3):
        xs = x + step
        (ref,) = oracle.run(MLP, xs.cpu(), *[a.cpu() for a in args[1:]])
        out = f(xs, *args[1:])
        close_f32(out, ref)
    cp = f.compiled(*args)
    assert cp.num_kernels == 3 and cp.stats["graph_replays"] == (3 if use_graph else 0)
    assert cp.matmul_configs[2].KSPLIT == 4 and len(cp.launches) == 3    # the last workgroup sums


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_on_device_autotune_times_candidates_and_persists_the_winner(dt, monkeypatch, tmp_path):
    """``tune=True`` for a GEMM shape absent from the packaged table: the backend compiles and
    times the cost model's best candidates on device buffers, stores the winner in a fresh
    autotune store, runs with it (checked against the oracle), and a later compile of the same
    shape reads the stored choice instead of tuning again.  Reference flow:
    tensorjit/runtime/autotune.py:83-118; its test tests/test_cuda_backend.py:68-85."""
    import json

    from tensorjit.backends import hip_backend as hb
    from tensorjit.runtime.autotune import MatmulConfig
    from tensorjit.runtime.cache import packaged_entry

    monkeypatch.delenv("TENSORJIT_NO_AUTOTUNE", raising=False)
    monkeypatch.delenv("TENSORJIT_RETUNE", raising=False)
    monkeypatch.setenv("TENSORJIT_CACHE_DIR", str(tmp_path / "fresh"))
    torch.manual_seed(0)
    m, n, k = (320, 576, 448) if dt == torch.bfloat16 else (200, 264, 384)
    x = torch.randn(m, k, device=DEV).to(dt)
    w = (0.05 * torch.randn(n, k, device=DEV)).to(dt)
    b = (0.05 * torch.randn(n, device=DEV)).to(dt)
    fn = lambda x, w, b: tj.gelu(tj.linear(x, w, b))  # noqa: E731
    f = tj.jit(fn, tune=True)
    out = f(x, w, b)
    cp = f.compiled(x, w, b)
    key = hb.matmul_key(cp.program.kernels[0], cp.arch)
    assert packaged_entry(key) is None
    stored = json.loads((tmp_path / "fresh" / "autotune.json").read_text())[key]
    assert MatmulConfig.from_dict(stored["config"]) == cp.matmul_configs[0]
    assert 0 < stored["ms"] < 1e3
    (orc,) = oracle.run(fn, x.float().cpu(), w.float().cpu(), b.float().cpu())
    if dt == torch.float32:
        close_f32(out, orc)
    else:
        close_lowp(out, orc)

    def no_tuning(*a, **kw):
        raise AssertionError("a stored choice must not be tuned again")

    monkeypatch.setattr(hb.HipProgram, "_autotune", no_tuning)
    again = tj.jit(fn, tune=True)
    assert torch.equal(again(x, w, b), out)
    assert again.compiled(x, w, b).matmul_configs[0] == cp.matmul_configs[0]


def test_bf16_gemm_gelu_epilogue_is_within_its_bound_of_the_exact_gelu():
    """A bf16 GEMM whose epilogue applies gelu uses tj_gelu16 (erf by A&S 7.1.25).  With
    identity weights each product is its input exactly, so over every bf16 value of
    magnitude 2^-100 to 8 (smaller inputs would give fp32 denormals) each output must be
    the exact gelu of its input to within half a bf16 unit plus the formula's bound,
    1.3e-5 |x|."""
    pos = torch.arange(0x0D80, 0x4101, dtype=torch.int32)                # bf16 in [2^-100, 8]
    bits = torch.cat([pos, pos | 0x8000, torch.zeros(1, dtype=torch.int32)])
    vals = bits.to(torch.int16).view(torch.bfloat16)
    n = -(-vals.numel() // 256) * 256
    x = torch.zeros(n, dtype=torch.bfloat16)
    x[:vals.numel()] = vals
    a = x.reshape(-1, 256).to(DEV)
    w = torch.eye(256, dtype=torch.bfloat16, device=DEV)
    f = tj.jit(lambda p, q: tj.gelu(tj.linear(p, q)))
    out = f(a, w)
    assert "tj_gelu16(" in f.compiled(a, w).source.split("tj_gelu16(float x)")[1]
    xd = a.double().cpu()
    exact = 0.5 * xd * torch.special.erfc(-xd / math.sqrt(2.0))
    err = (out.double().cpu() - exact).abs()
    bound = 2.0 ** -8 * exact.abs() + 1.3e-5 * xd.abs() + 1e-30
    worst = int(torch.argmax(err - bound))
    assert bool((err <= bound).all()), (float(xd.reshape(-1)[worst]), float(out.reshape(-1)[worst]),
                                        float(exact.reshape(-1)[worst]))


@pytest.mark.parametrize("case", ["f32_residual", "f32_ragged_gelu", "bf16_batched", "f16_ragged_bias_gelu",
                                  "skinny_bias_gelu"])
def test_k_split_gemm_matches_reference(case, monkeypatch):
    """K split over workgroups: fp32 partial tiles in the arena workspace, summed (in a
    fixed order) by the last workgroup of each tile (or, for the skinny kernel and with
    ``TENSORJIT_HIP_KSPLIT_FUSED=0``, by a second launch) that applies the fused epilogue;
    compared with an fp32 reference on three calls of one program (the workspace is reused
    without clearing; the tile counters must be back at zero after each call), bit-identical
    between the calls and between the two forms."""
    from tensorjit.runtime.autotune import MatmulConfig

    torch.manual_seed(0)
    if case == "f32_residual":
        x, w, r = torch.randn(512, 3072, device=DEV), 0.02 * torch.randn(768, 3072, device=DEV), torch.randn(512, 768, device=DEV)
        fn, args = (lambda a, b, c: tj.linear(a, b) + c), [x, w, r]
        ref, tol = x @ w.t() + r, 1e-5
        cfgs = [(64, 64, 32, 4, 2, 2, 16, 1, 8, 0, 0, 0, 8), (32, 32, 64, 4, 2, 2, 16, 1, 8, 0, 0, 0, 4)]
    elif case == "f32_ragged_gelu":
        x, w, b = torch.randn(200, 1024, device=DEV), 0.05 * torch.randn(300, 1024, device=DEV), torch.randn(300, device=DEV)
        fn, args = (lambda a, bb, c: tj.gelu(tj.linear(a, bb, c))), [x, w, b]
        ref, tol = torch.nn.functional.gelu(x @ w.t() + b), 1e-5
        cfgs = [(32, 64, 64, 4, 2, 2, 16, 1, 8, 0, 0, 0, 4), (64, 64, 32, 4, 2, 2, 16, 1, 8, 0, 0, 0, 8)]
    elif case == "bf16_batched":
        a = torch.randn(3, 136, 512, device=DEV).bfloat16()
        b = torch.randn(3, 200, 512, device=DEV).bfloat16()
        fn, args = (lambda p, q: tj.matmul(p, tj.transpose(q, 1, 2))), [a, b]
        ref, tol = a.float() @ b.float().transpose(1, 2).contiguous(), 2e-2
        cfgs = [(64, 64, 64, 4, 2, 2, 16, 1, 8, 0, 0, 0, 4), (128, 128, 32, 4, 2, 2, 32, 1, 8, 0, 0, 0, 2)]
    elif case == "f16_ragged_bias_gelu":
        x, w = torch.randn(200, 2048, device=DEV).half(), (0.03 * torch.randn(328, 2048, device=DEV)).half()
        b = torch.randn(328, device=DEV).half()
        fn, args = (lambda a, bb, c: tj.gelu(tj.linear(a, bb, c))), [x, w, b]
        ref, tol = torch.nn.functional.gelu(x.float() @ w.float().t() + b.float()), 2e-2
        cfgs = [(64, 64, 64, 4, 2, 2, 16, 1, 8, 0, 0, 0, 4), (32, 64, 64, 4, 2, 2, 16, 1, 8, 0, 0, 0, 8)]
    else:
        x, w, b = torch.randn(16, 8192, device=DEV).bfloat16(), (0.02 * torch.randn(4096, 8192, device=DEV)).bfloat16(), \
            torch.randn(4096, device=DEV).bfloat16()
        fn, args = (lambda a, bb, c: tj.gelu(tj.linear(a, bb, c))), [x, w, b]
        ref, tol = torch.nn.functional.gelu(x.float() @ w.float().t() + b.float()), 2e-2
        cfgs = [(16, 64, 256, 8, 1, 1, 16, 8, 0, 0, 0, 0, 4), (16, 32, 256, 8, 1, 1, 16, 8, 0, 0, 0, 0, 2)]
    for vals in cfgs:
        cfg = MatmulConfig(*vals)
        print(f"k-split {case} {vals}", flush=True)
        monkeypatch.setenv("TENSORJIT_HIP_KSPLIT_FUSED", "1")
        outs = [o.float() for o in _run_with_config(fn, args, cfg, calls=3)]
        if tol == 1e-5:
            close_f32(outs[0], ref, what=f"{case} {vals}")
        else:
            close_lowp(outs[0], ref, tol=tol, what=f"{case} {vals}")
        for out in outs[1:]:
            assert torch.equal(out, outs[0]), (case, vals)      # fixed summation order
        monkeypatch.setenv("TENSORJIT_HIP_KSPLIT_FUSED", "0")
        two = _run_with_config(fn, args, cfg).float()
        assert torch.equal(two, outs[0]), (case, vals)         # same order in both forms


DIRECT_CFGS = [(256, 256, 64, 4, 2, 2, 32, 1, 8, 0, 0, 1), (256, 128, 64, 4, 2, 2, 32, 1, 8, 0, 0, 1),
               (256, 256, 64, 4, 2, 2, 16, 1, 8, 0, 0, 1), (256, 128, 64, 4, 2, 2, 16, 1, 8, 0, 0, 1),
               (128, 64, 64, 4, 2, 2, 16, 1, 4, 0, 0, 1), (128, 128, 64, 4, 2, 2, 32, 1, 8, 0, 0, 1)]
# fp32 operands: 32-deep K tiles (the same 128-byte rows), 16x16x4 MFMAs
DIRECT_F32_CFGS = [(128, 128, 32, 4, 2, 2, 16, 1, 8, 0, 0, 1), (256, 128, 32, 4, 2, 2, 16, 1, 8, 0, 0, 1),
                   (128, 256, 32, 4, 2, 2, 16, 1, 8, 0, 0, 1), (64, 64, 32, 4, 2, 2, 16, 1, 8, 0, 0, 1)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("case", ["one_tile", "two_tiles", "three_tiles", "ragged", "batched", "shared_weight",
                                  "bias_gelu", "residual"])
def test_direct_lds_gemm_matches_reference(case, dtype):
    """The direct-to-LDS schedule (buffer loads straight into swizzled LDS, one wave per
    SIMD): the peeled prologue / tail for 1-3 K tiles, rows past M and N (zero-filled by
    the buffer range check), batched operands and a fused epilogue, against an fp32
    reference with the 16-bit tolerance."""
    from tensorjit.backends import hip_backend as hb
    from tensorjit.runtime.autotune import MatmulConfig

    torch.manual_seed(0)
    shapes = {"one_tile": (256, 256, 64), "two_tiles": (256, 512, 128), "three_tiles": (512, 256, 192),
              "ragged": (300, 520, 320), "batched": (200, 136, 256), "shared_weight": (300, 392, 192),
              "bias_gelu": (384, 640, 448), "residual": (520, 264, 256)}
    m, n, kk = shapes[case]
    if case == "shared_weight":
        # a batch of activations times one weight (batch stride 0 for B), as every projection of a layer
        a = torch.randn(3, m, kk, device=DEV).to(dtype)
        b = torch.randn(n, kk, device=DEV).to(dtype)
        fn = lambda x, y: tj.linear(x, y)
        args, ref = [a, b], a.float() @ b.float().t()
    elif case == "batched":
        a = torch.randn(2, 3, m, kk, device=DEV).to(dtype)
        b = torch.randn(2, 3, n, kk, device=DEV).to(dtype)
        fn = lambda x, y: tj.matmul(x, tj.transpose(y, 2, 3))
        args, ref = [a, b], a.float() @ b.float().transpose(2, 3).contiguous()
    elif case == "bias_gelu":
        a = torch.randn(m, kk, device=DEV).to(dtype)
        b = (0.05 * torch.randn(n, kk, device=DEV)).to(dtype)
        bias = torch.randn(n, device=DEV).to(dtype)
        fn = lambda x, y, z: tj.gelu(tj.linear(x, y, z))
        args, ref = [a, b, bias], torch.nn.functional.gelu(a.float() @ b.float().t() + bias.float())
    elif case == "residual":
        a = torch.randn(m, kk, device=DEV).to(dtype)
        b = torch.randn(n, kk, device=DEV).to(dtype)
        res = torch.randn(m, n, device=DEV).to(dtype)
        fn = lambda x, y, z: tj.linear(x, y) + z
        args, ref = [a, b, res], a.float() @ b.float().t() + res.float()
    else:
        a = torch.randn(m, kk, device=DEV).to(dtype)
        b = torch.randn(n, kk, device=DEV).to(dtype)
        fn = lambda x, y: tj.linear(x, y)
        args, ref = [a, b], a.float() @ b.float().t()
    mm = C_lower(fn, *args).kernels[0].anchor
    for vals in DIRECT_F32_CFGS if dtype == torch.float32 else DIRECT_CFGS:
        cfg = MatmulConfig(*vals)
        assert hb.config_ok(cfg, hb.compute_dtype(mm), mm), (case, cfg)
        for _ in range(2):      # twice: a race between loads and reads shows as run-to-run differences
            out = _run_with_config(fn, args, cfg).float()
            if dtype == torch.float32:
                close_f32(out, ref, what=f"{case} {dtype} {cfg}")
            else:
                close_lowp(out, ref, what=f"{case} {dtype} {cfg}")


REF_BENCH = {
    # the reference GPU benchmark's workloads at hidden D (reference benchmarks/bench.py:20-52)
    "bias_gelu": (lambda x, b: tj.gelu(x + b), lambda T, D: [(T, 4 * D), (4 * D,)], [1.0, 1.0]),
    "softmax": (lambda t: tj.softmax(t), lambda T, D: [(8, min(T, 2048), min(T, 2048))], [3.0]),
    "layernorm": (lambda x, g, b: tj.layer_norm(x, g, b), lambda T, D: [(T, D), (D,), (D,)], [1.0, 1.0, 1.0]),
    "rmsnorm": (lambda x, g: tj.rms_norm(x, g), lambda T, D: [(T, D), (D,)], [1.0, 1.0]),
    "linear_gelu": (lambda x, w, b: tj.gelu(tj.linear(x, w, b)), lambda T, D: [(T, D), (4 * D, D), (4 * D,)],
                    [1.0, 0.03, 0.03]),
}


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("seq", [256, 4096])
@pytest.mark.parametrize("name", sorted(REF_BENCH))
def test_reference_benchmark_workloads_vs_oracle(name, seq, dt):
    """The workloads the reference GPU table times (hidden 1024, seq 256 and 4096), as
    bench.py's reference_gpu_table runs them, against the fp32 oracle."""
    fn, shapes, scale = REF_BENCH[name]
    tdt = torch.bfloat16 if dt == "bf16" else torch.float32
    gen = torch.Generator(device=DEV).manual_seed(seq)
    args = [(torch.randn(s_, device=DEV, generator=gen) * c).to(tdt) for s_, c in zip(shapes(seq, 1024), scale)]
    print(f"reference workload {name} seq {seq} {dt}", flush=True)
    # fp32 GEMM: a 1024-term dot product per output
    check_vs_oracle(fn, *args, scale=1e-5 * (2 if name == "linear_gelu" else 1))


@pytest.mark.parametrize("dt,seq", [("bf16", 256), ("bf16", 1024), ("bf16", 4096), ("f32", 256), ("f32", 4096)])
def test_reference_table_mlp_block_on_its_packaged_tiles(dt, seq):
    """The reference benchmark's mlp_block at hidden 1024 (reference benchmarks/bench.py:
    20-52) on the packaged tiles swept for its two GEMMs (K split 4 ways, direct-to-LDS
    128 x 64 tiles, ...), against a float64 evaluation."""
    from tensorjit.backends import hip_backend as hb
    from tensorjit.runtime.autotune import MatmulConfig
    from tensorjit.runtime.cache import packaged_entry

    tdt = torch.bfloat16 if dt == "bf16" else torch.float32
    gen = torch.Generator(device=DEV).manual_seed(seq)
    shapes = [(seq, 1024), (1024,), (4096, 1024), (4096,), (1024, 4096), (1024,)]
    scale = [1.0, 1.0, 0.03, 0.03, 0.015, 0.03]
    args = [(torch.randn(s_, device=DEV, generator=gen) * c).to(tdt) for s_, c in zip(shapes, scale)]
    f = tj.jit(MLP)
    out = f(*args)
    cp = f.compiled(*args)
    assert len(cp.matmul_configs) == 2
    packaged = 0
    for idx, cfg in cp.matmul_configs.items():
        entry = packaged_entry(hb.matmul_key(cp.program.kernels[idx], cp.arch))
        if entry is not None:
            packaged += 1
            assert cfg == MatmulConfig.from_dict(entry["config"])
    assert packaged >= 1
    x, g, w1, b1, w2, b2 = [a.double().cpu() for a in args]
    h = torch.nn.functional.layer_norm(x, (1024,), g)
    ref = x + torch.nn.functional.linear(torch.nn.functional.gelu(torch.nn.functional.linear(h, w1, b1)), w2, b2)
    if dt == "bf16":
        # the LayerNorm and gelu outputs are stored in bf16 between the kernels
        close_lowp(out, ref, norm=1e-2, what=f"mlp_block {dt} {seq}")
    else:
        close_f32(out, ref, scale=1e-5 * 2, what=f"mlp_block {dt} {seq}")


def C_lower(fn, *args):
    from tensorjit.compiler import lower
    from tensorjit.frontend.tracer import tensor_type_of

    return lower(tj.trace(fn, [tensor_type_of(a) for a in args]), "hip")


@pytest.mark.parametrize("case", ["plain_two_tiles_each", "bias_gelu_uneven", "residual_short_k", "plain_long_k",
                                  "batch_folded_residual", "batch_row_broadcast", "f16_bias_gelu"])
def test_persistent_direct_gemm_matches_the_direct_kernel(case):
    """The persistent direct-to-LDS kernel (workgroups looping over output tiles, the next
    tile's first K tiles prefetched under the epilogue) gives bit-identical results to the
    one-tile-per-workgroup direct kernel with the same tiling (same MFMA order), on
    small-integer data where both must equal the exact product: several tiles per
    workgroup, workgroups with unequal tile counts, the shortest K loop (4 K tiles), an
    epilogue with preloaded bias and one that loads a residual per element, a batched
    projection folded into one GEMM over (batch x M) rows, and a residual broadcast over
    the batch (which does not fold: the direct kernel is generated instead).  The
    integer products are exact in fp32, so the base kernel's output is the reference
    rounded once to the 16-bit storage type."""
    from tensorjit.runtime.autotune import MatmulConfig

    torch.manual_seed(0)
    # (batch, M, N, K, epilogue, workgroups): 16 tiles on 8 workgroups (XCD order); 15
    # tiles on 8 (plain order, one workgroup runs one tile); 4 K tiles; 16 K tiles; a
    # [3, 256, .] activation (12 tiles on 8 workgroups)
    bt, m, n, kk, epi, G = {"plain_two_tiles_each": ((), 1024, 1024, 384, "plain", 8),
                            "bias_gelu_uneven": ((), 768, 1280, 640, "gelu", 8),
                            "residual_short_k": ((), 512, 1024, 256, "res", 8),
                            "plain_long_k": ((), 1024, 512, 1024, "plain", 8),
                            "batch_folded_residual": ((3,), 256, 1024, 256, "res", 8),
                            "batch_row_broadcast": ((3,), 256, 512, 256, "rowres", 8),
                            "f16_bias_gelu": ((), 512, 768, 512, "gelu", 8)}[case]
    dt = torch.float16 if case.startswith("f16") else torch.bfloat16
    print(f"persistent gemm {case} {bt}x{m}x{n}x{kk} {epi} G={G} {dt}", flush=True)
    a = torch.randint(-3, 4, (*bt, m, kk), device=DEV).to(dt)
    b = torch.randint(-3, 4, (n, kk), device=DEV).to(dt)
    if epi == "gelu":
        bias = torch.randint(-8, 9, (n,), device=DEV).to(dt)
        fn, args = (lambda x, y, z: tj.gelu(tj.linear(x, y, z))), [a, b, bias]
        ref = torch.nn.functional.gelu(a.float() @ b.float().t() + bias.float())
    elif epi in ("res", "rowres"):
        res = torch.randint(-8, 9, (*bt, m, n) if epi == "res" else (m, n), device=DEV).to(dt)
        fn, args = (lambda x, y, z: tj.linear(x, y) + z), [a, b, res]
        ref = a.float() @ b.float().t() + res.float()
    else:
        fn, args = (lambda x, y: tj.linear(x, y)), [a, b]
        ref = a.float() @ b.float().t()
    base = MatmulConfig(256, 256, 64, 4, 2, 2, 16, 1, 8, 0, 0, 1)
    pers = MatmulConfig(256, 256, 64, 4, 2, 2, 16, 1, 8, 0, 0, 1, 1, G)
    mm = C_lower(fn, *args).kernels[0].anchor
    assert hb_config_ok(pers, mm)
    from tensorjit.backends import hip_backend as hb

    launches = hb.generate(C_lower(fn, *args), {0: pers})[1]
    assert (launches[0].meta.get("persistent") is None) == (epi == "rowres"), case
    want = _run_with_config(fn, args, base)
    for _ in range(2):          # twice: a race between the prefetches and the reads shows as a difference
        got = _run_with_config(fn, args, pers)
        assert torch.equal(got, want), case
    # both round the exact fp32 sums to 16 bits once: within half an ulp of the reference
    close_lowp(want.float(), ref, what=case)


def hb_config_ok(cfg, mm):
    from tensorjit.backends import hip_backend as hb

    return hb.config_ok(cfg, hb.compute_dtype(mm), mm)


def test_tensors_past_two_to_the_31_elements():
    """Iteration spaces of 2^31 elements and more take 64-bit offsets: a pointwise
    chain, an RMSNorm, a column sum and a split full sum over [2^21 + 3, 1024] bf16, and a
    GEMM whose [65536, 32768]
    output has 2^31 elements, each checked against the oracle on its first rows and on
    the rows whose offsets are past 2^31."""
    torch.manual_seed(0)
    rows = 2**21 + 3
    x = torch.randn(rows, 1024, device=DEV).bfloat16()
    g = (1 + 0.1 * torch.randn(1024, device=DEV)).bfloat16()
    fn = lambda t, w: (t * 2.0 + 1.0, tj.rms_norm(t, w))  # noqa: E731
    print("past 2^31: pointwise + rms", flush=True)
    y, r = tj.jit(fn)(x, g)
    for sl in (slice(0, 64), slice(rows - 64, rows)):
        ry, rr = oracle.run(fn, x[sl].float().cpu(), g.float().cpu())
        close_lowp(y[sl], ry, tol=1e-2)
        close_lowp(r[sl], rr, tol=2e-2)
    del x, y, r
    # a column reduction and a split full reduction over the same 2^31 + 3072 elements:
    # small integers keep every partial exact, so both match torch bit for bit
    xi = torch.randint(-3, 4, (rows, 1024), device=DEV).bfloat16()
    print("past 2^31: column sum and split sum", flush=True)
    fc = tj.jit(lambda t: tj.sum(t, axis=0))
    assert fc.compiled(xi).launches[0].meta["family"] == "colreduce"
    assert torch.equal(fc(xi), xi.float().sum(0).bfloat16())
    fs = tj.jit(lambda t: tj.sum(tj.reshape(t, rows * 1024)))
    assert fs.compiled(xi).launches[0].meta["splits"] > 1
    assert torch.equal(fs(xi).float().reshape(()), xi.float().sum().bfloat16().float())
    del xi
    torch.cuda.empty_cache()
    a = torch.randn(65536, 64, device=DEV).bfloat16()
    w = torch.randn(32768, 64, device=DEV).bfloat16()
    print("past 2^31: gemm output", flush=True)
    out = tj.jit(lambda p, q: tj.linear(p, q))(a, w)
    for sl in (slice(0, 32), slice(65536 - 32, 65536)):
        ref = a[sl].float() @ w.float().t()
        close_lowp(out[sl], ref, tol=2e-2)
