"""Static arena planner (reference tests/test_runtime_and_planner.py:18-51)."""
import tensorjit as tj
import tensorjit.compiler as C
from tensorjit.ir import TensorType
from tensorjit.passes.memory_planner import ALIGN, plan_memory


def _prog(fn, *shapes):
    return C.lower(tj.trace(fn, [TensorType(s) for s in shapes]), "hip")


def test_planner_shares_storage_between_disjoint_lifetimes():
    def chain(x):
        y = x
        for _ in range(6):
            y = tj.matmul(tj.softmax(tj.gelu(y * 1.1 + 0.1)), x)
        return y

    plan = plan_memory(_prog(chain, (256, 256)))
    assert plan.naive_bytes > 2 * plan.arena_bytes
    assert plan.savings > 0.5
    assert all(b.offset % ALIGN == 0 for b in plan.buffers.values())


def test_planner_never_overlaps_live_buffers():
    def mlp(x, g, w1, b1, w2, b2):
        return x + tj.linear(tj.gelu(tj.linear(tj.layer_norm(x, g), w1, b1)), w2, b2)

    plan = plan_memory(_prog(mlp, (512, 256), (256,), (1024, 256), (1024,), (256, 1024), (256,)))
    bufs = list(plan.buffers.values())
    for i, a in enumerate(bufs):
        for b in bufs[i + 1:]:
            alive_together = not (a.last < b.first or b.last < a.first)
            overlap = not (a.offset + a.size <= b.offset or b.offset + b.size <= a.offset)
            assert not (alive_together and overlap)
    # the LayerNorm output and the GELU output are both live at the second matmul
    assert plan.arena_bytes == sum(b.size for b in bufs)


def test_planner_mlp_config1_arena_is_ln_plus_gelu():
    def mlp(x, g, w1, b1, w2, b2):
        return x + tj.linear(tj.gelu(tj.linear(tj.layer_norm(x, g), w1, b1)), w2, b2)

    plan = plan_memory(_prog(mlp, (512, 768), (768,), (3072, 768), (3072,), (768, 3072), (768,)))
    assert plan.arena_bytes == 512 * 768 * 4 + 512 * 3072 * 4
    # LN out (k0..k1) placed first at 0, GELU out (k1..k2) after it: both live at k1
    assert sorted(b.offset for b in plan.buffers.values()) == [0, 512 * 768 * 4]


def test_planner_excludes_graph_outputs():
    plan = plan_memory(_prog(lambda x: (tj.exp(x), tj.exp(x) + 1.0), (64,)))
    assert all("add" not in b.node.name for b in plan.buffers.values())


def test_planner_best_fit_prefers_the_tightest_gap():
    # k0: a (8 KiB, dies at k1), b (1 KiB, lives to k3); k1: c (4 KiB, dies k2)
    # k2: d (1 KiB) must take the 1 KiB-or-larger gap that fits best.
    def f(x, y):
        a = tj.exp(x)                 # [2048] f32 = 8 KiB
        b = tj.exp(y)                 # [256]  f32 = 1 KiB
        c = tj.sum(a.reshape(2, 1024), keepdim=True) + 0.0
        return c, b
    plan = plan_memory(_prog(f, (2048,), (256,)))
    sizes = sorted(b.size for b in plan.buffers.values())
    assert all(s % ALIGN == 0 for s in sizes)
    assert plan.arena_bytes <= plan.naive_bytes
