"""tj_hip_program_run_static: the allocation-free variant of tj_hip_program_run.

Same kernels, same launch order, intermediates in the library's static per-GPU
arena instead of the program's own: outputs must equal tj_hip_program_run's bit for
bit, on two calls in a row with the second program smaller than the first (the
static arena then still holds the first call's larger contents), a fresh program's
first call issued under stream capture, and a program whose arena exceeds the static
one is refused before any launch.
"""
import pytest
import torch

import tensorjit as tj
from tensorjit.runtime import hip as rt

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(autouse=True)
def _env(monkeypatch, tmp_path_factory):
    if not (torch.cuda.is_available() and torch.version.hip):
        pytest.skip("needs a ROCm GPU")
    monkeypatch.setenv("TENSORJIT_NO_AUTOTUNE", "1")
    monkeypatch.setenv("TENSORJIT_CACHE_DIR", str(tmp_path_factory.getbasetemp() / "tjcache"))


def _mlp(x, g, w1, b1, w2, b2):
    return x + tj.linear(tj.gelu(tj.linear(tj.layer_norm(x, g), w1, b1)), w2, b2)


def _inputs(rows, d=768, f=3072, seed=0):
    gen = torch.Generator(device=DEV).manual_seed(seed)
    shapes = [(rows, d), (d,), (f, d), (f,), (d, f), (d,)]
    scale = [1.0, 0.1, 0.02, 0.02, 0.02, 0.02]
    return [torch.randn(s, device=DEV, generator=gen) * c for s, c in zip(shapes, scale)]


def _both(cp, args):
    """Outputs of tj_hip_program_run and tj_hip_program_run_static for the same inputs."""
    stream = torch.cuda.current_stream().cuda_stream
    ins = [a.contiguous() for a in args]
    outs = [[torch.empty(s, dtype=d, device=DEV) for s, d in cp._out_specs] for _ in range(2)]
    ip = [t.data_ptr() for t in ins]
    cp.native.run(ip, [t.data_ptr() for t in outs[0]], stream)
    cp.native.run_static(ip, [t.data_ptr() for t in outs[1]], stream)
    torch.cuda.synchronize()
    return outs


def test_static_arena_run_matches_the_allocating_run():
    f = tj.jit(_mlp)
    big = _inputs(512)             # arena: LayerNorm + gelu outputs + 4-way split-K partials
    cp_big = f.compiled(*big)      # (summed by each tile's last workgroup: 3 launches)
    assert 0 < cp_big.arena_bytes <= rt.STATIC_ARENA_BYTES and len(cp_big.launches) == 3
    small = _inputs(64, seed=1)
    cp_small = f.compiled(*small)
    assert 0 < cp_small.arena_bytes < cp_big.arena_bytes
    for cp, args in ((cp_big, big), (cp_small, small), (cp_big, _inputs(512, seed=2))):
        ref, got = _both(cp, args)
        for r, o in zip(ref, got):
            assert torch.equal(r, o)
        torch.testing.assert_close(got[0], cp(*args)[0], atol=0, rtol=0)


def test_first_static_run_of_a_fresh_program_under_stream_capture():
    """tj_hip_program_create looks the static arena up, so a fresh program's very first
    tj_hip_program_run_static may be issued under stream capture (torch.cuda.graph):
    every replay of that graph, with eager work in between, equals tj_hip_program_run's
    output bit for bit."""
    cp = tj.jit(_mlp).compiled(*_inputs(256, seed=6))
    args = _inputs(256, seed=6)
    assert cp.native.stats()["calls"] == 0 and 0 < cp.arena_bytes <= rt.STATIC_ARENA_BYTES
    ip = [a.data_ptr() for a in args]
    got = [torch.empty(s, dtype=d, device=DEV) for s, d in cp._out_specs]
    want = [torch.empty(s, dtype=d, device=DEV) for s, d in cp._out_specs]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        cp.native.run_static(ip, [t.data_ptr() for t in got], torch.cuda.current_stream().cuda_stream)
    cp.native.run(ip, [t.data_ptr() for t in want], torch.cuda.current_stream().cuda_stream)
    for _ in range(3):
        for t in got:
            t.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip(got, want))
        _ = (args[0] * 2).sum().item()          # eager work between replays


def test_static_arena_run_of_key_split_attention():
    """The fused attention with key splits keeps its partial rows in the workspace: in
    the static arena they match the allocating run bit for bit, a larger split program
    first and a smaller one after it."""
    fn = lambda q, k, v: tj.matmul(tj.softmax(tj.matmul(q, tj.transpose(k, -1, -2)) * 0.088), v)  # noqa: E731
    f = tj.jit(fn)
    gen = torch.Generator(device=DEV).manual_seed(3)
    cases = [[torch.randn(s, device=DEV, generator=gen).bfloat16() for s in [(2, 2, 1000, 128)] * 3],
             [torch.randn(s, device=DEV, generator=gen).bfloat16() for s in [(1, 2, 300, 64), (1, 2, 1280, 64),
                                                                             (1, 2, 1280, 64)]]]
    sizes = []
    for args in cases:
        cp = f.compiled(*args)
        assert [l.meta["family"] for l in cp.launches] == ["attention", "attention_combine"]
        assert 0 < cp.arena_bytes <= rt.STATIC_ARENA_BYTES
        sizes.append(cp.arena_bytes)
        ref, got = _both(cp, args)
        assert torch.equal(ref[0], got[0])
    assert sizes[1] < sizes[0]


def test_static_arena_run_of_split_row_reductions():
    """A reduction split over workgroups keeps its partials in the workspace: in the
    static arena the sum and max match the allocating run bit for bit, a program with
    more partials first and one with fewer after it."""
    f = tj.jit(lambda t: (tj.sum(t * t, axis=-1), tj.max(t, axis=-1)))
    gen = torch.Generator(device=DEV).manual_seed(4)
    sizes = []
    for shape in [(4, 1 << 20), (1, 140000)]:
        x = torch.randn(shape, device=DEV, generator=gen)
        cp = f.compiled(x)
        assert [l.meta["family"] for l in cp.launches] == ["row", "row_combine"] * 2
        assert 0 < cp.arena_bytes <= rt.STATIC_ARENA_BYTES
        sizes.append(cp.arena_bytes)
        ref, got = _both(cp, [x])
        assert torch.equal(ref[0], got[0]) and torch.equal(ref[1], got[1])
        assert torch.equal(got[1], x.amax(-1))
    assert sizes[1] < sizes[0]


def test_static_arena_run_of_column_reductions():
    """A column reduction's partials live in the workspace too: in the static arena the
    column sum and max match the allocating run bit for bit, a program with more partials
    first and one with fewer after it."""
    f = tj.jit(lambda t: (tj.sum(t, axis=0), tj.max(t, axis=0)))
    gen = torch.Generator(device=DEV).manual_seed(5)
    sizes = []
    for shape in [(8192, 4096), (3000, 1000)]:
        x = torch.randn(shape, device=DEV, generator=gen)
        cp = f.compiled(x)
        assert [l.meta["family"] for l in cp.launches] == ["colreduce", "colreduce_combine"] * 2
        assert 0 < cp.arena_bytes <= rt.STATIC_ARENA_BYTES
        sizes.append(cp.arena_bytes)
        ref, got = _both(cp, [x])
        assert torch.equal(ref[0], got[0]) and torch.equal(ref[1], got[1])
        assert torch.equal(got[1], x.amax(0))
    assert sizes[1] < sizes[0]


def test_programs_larger_than_the_static_arena_are_refused():
    args = _inputs(16384)          # 48 MiB LayerNorm output + 192 MiB gelu output
    cp = tj.jit(_mlp).compiled(*args)
    assert cp.arena_bytes > rt.STATIC_ARENA_BYTES
    out = torch.zeros(cp._out_specs[0][0], device=DEV)
    with pytest.raises(rt.HipError, match="static arena"):
        cp.native.run_static([a.data_ptr() for a in args], [out.data_ptr()], torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert not bool(out.any())     # refused before any launch
