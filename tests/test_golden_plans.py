"""The optimised graph, kernel plan and memory plan of every benchmark workload equal
the reference's own, as recorded in tests/golden/plans.json by the reference's passes
(tests/golden/make_plans.py).  The hip backend lowers with the same row-fusion limit as
the reference's cuda backend, so the plans must match node for node, kernel for kernel
and byte for byte in the arena."""
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
    # this repository's package, not the reference's, is the one under test
    assert Path(tj.__file__).resolve().parts[-3] == "mlir-gpu-kernel-compiler_amd"
    assert FIXTURE["reference_backend"] == plan_cases.REFERENCE_BACKEND
    assert sorted(FIXTURE["cases"]) == sorted(c[0] for c in plan_cases.CASES)


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


def test_a_changed_plan_is_caught(monkeypatch):
    """The comparison is not vacuous: fusing config 2 without row fusion (two kernels)
    differs from the recorded one-kernel plan."""
    name, fn_name, args, _ = next(c for c in plan_cases.CASES if c[0] == "c2_eltwise_f32")
    monkeypatch.setenv("TENSORJIT_NO_ROW_FUSION", "1")
    program = lower(plan_cases.trace_case(tj, ir, getattr(bench, fn_name), args), plan_cases.BACKEND)
    got = json.loads(json.dumps(plan_cases.describe(program, plan_memory(program))))
    assert got["kernels"] != FIXTURE["cases"][name]["kernels"]
