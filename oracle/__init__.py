"""CPU oracle for the tensorjit hip backend — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU baseline
use this package, as the checker / CPU timing baseline.  The product path
(``tensorjit`` and its hip backend) never imports it.

``oracle.run(fn, *tensors)`` traces ``fn`` with fp32 types, lowers it with
tensorjit's own passes (the shared upstream of every backend) and executes the
resulting kernel program through the C restatement of the reference ``c``
backend (``oracle/c_backend.py``).

What pins it: float64 closed forms per op family (``tests/test_oracle.py``), and a
plan-free float64 evaluation of the traced graph node by node
(``tests/graph_eval.py``) that random programs of every fuzz generator must match
(``tests/test_graph_fuzz.py``), so a fusion plan that computes something other than
the ops' meaning fails even though the oracle and the hip path share it.
"""
from __future__ import annotations

import torch

from .c_backend import OracleProgram, compile_program, generate  # noqa: F401


def lower_f32(fn, *shapes, backend: str = "hip"):
    """Trace ``fn`` over fp32 inputs of ``shapes`` and lower it to a fused program."""
    import tensorjit as tj
    from tensorjit.compiler import lower
    from tensorjit.ir import TensorType

    return lower(tj.trace(fn, [TensorType(tuple(s)) for s in shapes]), backend)


def run(fn, *tensors: torch.Tensor) -> list[torch.Tensor]:
    """fp32 CPU result of ``fn`` on (upcast copies of) ``tensors``."""
    prog = compile_program(lower_f32(fn, *[t.shape for t in tensors]))
    return prog(*[t.detach().float().cpu() for t in tensors])
