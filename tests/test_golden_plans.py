"""The optimised graph, kernel plan and memory plan of every benchmark workload equal
the reference's own, as recorded in tests/golden/plans.json by the reference's passes
(tests/golden/make_plans.py), run with the hip backend's row-fusion limit (32768; the
reference's cuda backend stops at 8192, and the recorded plans of rows up to 8192 are the
same under either).  The plans must match node for node, kernel for kernel and byte for
byte in the arena, rows of 12000-32768 elements included.  The one deliberate departure
(a column value read along the rows of a square tensor) is pinned as such."""
import json
import sys
from pathlib import Path

import pytest

import bench
import tensorjit as tj
from tensorjit import ir
from tensorjit.compiler import lower
from tensorjit.passes.memory_planner import plan_memory

GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))
import plan_cases  # noqa: E402

FIXTURE = json.loads((GOLDEN / "plans.json").read_text())


def test_fixture_covers_every_case():
    from tensorjit.compiler import ROW_FUSION_MAX_N

    # this repository's package, not the reference's, is the one under test
    assert Path(tj.__file__).resolve().parts[-3] == "mlir-gpu-kernel-compiler_amd"
    assert FIXTURE["reference_backend"] == plan_cases.REFERENCE_BACKEND
    assert FIXTURE["row_fusion_max_n"] == plan_cases.ROW_FUSION_MAX_N == ROW_FUSION_MAX_N[plan_cases.BACKEND]
    assert sorted(FIXTURE["cases"]) == sorted(c[0] for c in plan_cases.CASES)
    assert sorted(FIXTURE["divergent"]) == sorted(c[0] for c in plan_cases.DIVERGENT)
    # the wide-row cases are one row kernel each up to the limit, and not past it
    for name, _, args, _ in plan_cases.CASES:
        n = args[0][0][-1]
        if n > 8192:
            kinds = [k["kind"] for k in FIXTURE["cases"][name]["kernels"]]
            assert (kinds == ["row"]) == (n <= plan_cases.ROW_FUSION_MAX_N), (name, kinds)


@pytest.mark.parametrize("name,fn_name,args,env", plan_cases.CASES, ids=[c[0] for c in plan_cases.CASES])
def test_plan_matches_the_reference(name, fn_name, args, env, monkeypatch):
    monkeypatch.delenv("TENSORJIT_NO_ROW_FUSION", raising=False)
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    program = lower(plan_cases.trace_case(tj, ir, getattr(bench, fn_name), args), plan_cases.BACKEND)
    got = json.loads(json.dumps(plan_cases.describe(program, plan_memory(program))))
    want = FIXTURE["cases"][name]
    assert got["graph"] == want["graph"]
    assert got["kernels"] == want["kernels"]
    assert got["aliases"] == want["aliases"]
    assert got["memory"] == want["memory"]


@pytest.mark.parametrize("name,fn_name,args,ref_kinds,hip_kinds", plan_cases.DIVERGENT,
                         ids=[c[0] for c in plan_cases.DIVERGENT])
def test_plan_departs_from_the_reference_only_where_documented(name, fn_name, args, ref_kinds, hip_kinds,
                                                               monkeypatch):
    """Same optimised graph; the reference's row kernel, which would apply a per-column
    value per row, is a reduction and a pointwise kernel over the same nodes here; every
    other kernel is the reference's."""
    monkeypatch.delenv("TENSORJIT_NO_ROW_FUSION", raising=False)
    program = lower(plan_cases.trace_case(tj, ir, getattr(plan_cases, fn_name), args), plan_cases.BACKEND)
    got = json.loads(json.dumps(plan_cases.describe(program, plan_memory(program))))
    want = FIXTURE["divergent"][name]
    assert got["graph"] == want["graph"]
    assert [k["kind"] for k in want["kernels"]] == ref_kinds
    assert [k["kind"] for k in got["kernels"]] == hip_kinds
    rows = [k for k in want["kernels"] if k["kind"] == "row"]
    split = [k for k in got["kernels"] if k not in want["kernels"]]
    assert sorted(n for k in rows for n in k["nodes"]) == sorted(n for k in split for n in k["nodes"])
    assert [k for k in got["kernels"] if k in want["kernels"]] == [k for k in want["kernels"] if k not in rows]


def test_a_changed_plan_is_caught(monkeypatch):
    """The comparison is not vacuous: fusing config 2 without row fusion (two kernels)
    differs from the recorded one-kernel plan."""
    name, fn_name, args, _ = next(c for c in plan_cases.CASES if c[0] == "c2_eltwise_f32")
    monkeypatch.setenv("TENSORJIT_NO_ROW_FUSION", "1")
    program = lower(plan_cases.trace_case(tj, ir, getattr(bench, fn_name), args), plan_cases.BACKEND)
    got = json.loads(json.dumps(plan_cases.describe(program, plan_memory(program))))
    assert got["kernels"] != FIXTURE["cases"][name]["kernels"]
