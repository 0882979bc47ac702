"""Write ``plans.json``: the reference's own kernel plans and memory plans for the
benchmark workloads.

    python tests/golden/make_plans.py [REFERENCE_ROOT]      # default /root/reference

It imports the reference's ``tensorjit`` (pure Python: tracer, cleanup passes,
``fuse``/``row_fuse``, ``plan_memory``; nothing is compiled or run on a device), traces
each workload of ``plan_cases.CASES`` and ``plan_cases.DIVERGENT`` with it, lowers it with
the reference's own ``fuse(optimize(graph))`` and ``row_fuse`` at the hip backend's
row-fusion limit (``plan_cases.ROW_FUSION_MAX_N``, 32768; the reference's cuda backend
uses 8192, which gives the same plans for rows of at most 8192 elements) and records the
result through ``plan_cases.describe``.  The tests compare this repository's plans with
the file; they never import the reference.  Run in the build container only (the
reference is not on the GPU box).
"""
from __future__ import annotations

import json
import os
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]


def main(ref_root: str) -> None:
    ref = Path(ref_root).resolve()
    sys.path.insert(0, str(ref))
    import tensorjit as tj  # the reference package

    if not Path(tj.__file__).resolve().is_relative_to(ref):
        raise SystemExit(f"imported {tj.__file__}, not the reference under {ref}")
    from tensorjit import ir
    from tensorjit.passes import fuse, optimize, row_fuse
    from tensorjit.passes.memory_planner import plan_memory

    # bench.py's workload functions run `import tensorjit` when called: the module
    # already imported above (the reference) is the one they get
    sys.path.insert(0, str(ROOT))
    sys.path.insert(0, str(HERE))
    import bench
    import plan_cases

    def lower(graph):
        # the reference's lower() (reference tensorjit/compiler.py:37-42) at the hip limit
        program = fuse(optimize(graph))
        if os.environ.get("TENSORJIT_NO_ROW_FUSION") != "1":
            program = row_fuse(program, max_n=plan_cases.ROW_FUSION_MAX_N)
        return program

    out = {"generator": "tests/golden/make_plans.py", "reference_backend": plan_cases.REFERENCE_BACKEND,
           "row_fusion_max_n": plan_cases.ROW_FUSION_MAX_N, "cases": {}, "divergent": {}}
    cases = [(c, "cases", getattr(bench, c[1])) for c in plan_cases.CASES]
    cases += [((name, fn_name, args, {}), "divergent", getattr(plan_cases, fn_name))
              for name, fn_name, args, _, _ in plan_cases.DIVERGENT]
    for (name, _, args, env), where, fn in cases:
        saved = {k: os.environ.get(k) for k in env}
        os.environ.update(env)
        try:
            program = lower(plan_cases.trace_case(tj, ir, fn, args))
            out[where][name] = plan_cases.describe(program, plan_memory(program))
        finally:
            for k, v in saved.items():
                if v is None:
                    os.environ.pop(k, None)
                else:
                    os.environ[k] = v
        print(f"{name}: {len(program.kernels)} kernels, arena {out[where][name]['memory']['arena_bytes']} B")
    (HERE / "plans.json").write_text(json.dumps(out, separators=(",", ":"), sort_keys=True) + "\n")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
