"""CPU oracle: a restatement of the reference ``c`` backend (C11 + OpenMP).

TEST INFRASTRUCTURE ONLY.  Nothing in the product (the ``tensorjit`` package
and its hip backend) imports, links or runs this file; only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg do, as the
checker and as the CPU timing baseline.

What it restates (reference ``tensorjit/backends/c_backend.py``):

* fp32 only; any other dtype raises ``NotImplementedError`` (``:77-80``).
* gelu through the Abramowitz & Stegun 7.1.26 erf with ``|x|`` clamped at 4
  (``:44-56``; published formula, |error| < 1.5e-7).
* expression semantics per op (``tensorjit/backends/common.py:65-85``):
  ``where`` tests ``!= 0``, ``rsqrt`` is ``1/sqrtf``, ``relu`` is
  ``fmaxf(x, 0)``, sigmoid/silu through ``expf``.
* reductions: ``sum``/``mean`` accumulate in fp32 from 0, ``mean`` divides by N
  at the end, ``max`` starts from -inf (``:133-183``).
* row kernels run their stages in order per row with per-row temporaries
  (``:424-564``); matmul applies the epilogue per output element after the
  fp32 dot product (``:186-304``).
* built with ``gcc -O3 -ffast-math -march=native -fopenmp -std=c11`` (``:318``).

The C text is this file's own (loop structure, names and GEMM blocking
differ from the reference's generator); the arithmetic each op performs is
the reference's.
"""
from __future__ import annotations

import ctypes
import hashlib
import math
import os
import shutil
import subprocess
import tempfile
from pathlib import Path

import torch

C_PRELUDE = r"""
#include <math.h>
#include <stdlib.h>
#include <string.h>
#define OR_EXPORT __attribute__((visibility("default")))
/* Abramowitz & Stegun 7.1.26: erf(x) ~ 1 - (a1 t + a2 t^2 + ... + a5 t^5) exp(-x^2), t = 1/(1 + p x). */
static inline float or_erf(float x) {
  const float s = x < 0.0f ? -1.0f : 1.0f;
  float z = fabsf(x);
  z = z > 4.0f ? 4.0f : z;
  const float t = 1.0f / (1.0f + 0.3275911f * z);
  const float poly = t * (0.254829592f + t * (-0.284496736f + t * (1.421413741f + t * (-1.453152027f + t * 1.061405429f))));
  return s * (1.0f - poly * expf(-z * z));
}
"""

C_EXPR = {
    "neg": "(-{0})",
    "exp": "expf({0})",
    "log": "logf({0})",
    "sqrt": "sqrtf({0})",
    "rsqrt": "(1.0f / sqrtf({0}))",
    "tanh": "tanhf({0})",
    "relu": "fmaxf({0}, 0.0f)",
    "sigmoid": "(1.0f / (1.0f + expf(-({0}))))",
    "gelu": "(0.5f * {0} * (1.0f + or_erf({0} * 0.70710678118654752f)))",
    "silu": "({0} / (1.0f + expf(-({0}))))",
    "abs": "fabsf({0})",
    "add": "({0} + {1})",
    "sub": "({0} - {1})",
    "mul": "({0} * {1})",
    "div": "({0} / {1})",
    "pow": "powf({0}, {1})",
    "maximum": "fmaxf({0}, {1})",
    "minimum": "fminf({0}, {1})",
    "where": "(({0}) != 0.0f ? ({1}) : ({2}))",
}

BUILD_DIR = Path(__file__).resolve().parent / "_build"


def _lit(v: float) -> str:
    if v != v:
        return "NAN"
    if math.isinf(v):
        return "(-INFINITY)" if v < 0 else "INFINITY"
    return f"{v!r}f"


def _strides(shape) -> list[int]:
    out, step = [], 1
    for d in reversed(shape):
        out.append(step)
        step *= d
    return out[::-1]


def _read_strides(inp, consumer, iter_shape) -> list[int]:
    """Strides used to read ``inp`` at each point of ``iter_shape``."""
    cs = _strides(inp.shape)
    if consumer is not None and consumer.op == "transpose":
        return [cs[p] for p in consumer.attrs["perm"]]
    lead = len(iter_shape) - len(inp.shape)
    return [0] * lead + [0 if inp.shape[d] == 1 and iter_shape[lead + d] != 1 else cs[d] for d in range(len(inp.shape))]


def _offset(idx: list[str], st: list[int]) -> str:
    terms = [f"{v}*{s}L" for v, s in zip(idx, st) if s]
    return " + ".join(terms) if terms else "0"


class _K:
    """Per-kernel naming: external inputs x{j}, nodes t{j}, outputs y{j}."""

    def __init__(self, k, idx):
        self.k, self.idx = k, idx
        self.name = {id(n): f"x{j}" for j, n in enumerate(k.inputs)}
        self.name.update({id(n): f"t{j}" for j, n in enumerate(k.nodes)})

    def expr(self, n, local):
        args = []
        for i in n.inputs:
            if i.op == "const" and i.shape == ():
                args.append(_lit(i.attrs["value"]))
            else:
                args.append(local[id(i)])
        return C_EXPR[n.op].format(*args)

    def header(self):
        lines = [f"OR_EXPORT void k{self.idx}(void** a) {{"]
        for j, n in enumerate(self.k.inputs):
            lines.append(f"  const float* restrict {self.name[id(n)]}p = (const float*)a[{j}];")
        for j, _ in enumerate(self.k.outputs):
            lines.append(f"  float* restrict y{j}p = (float*)a[{len(self.k.inputs) + j}];")
        return lines

    def consumer(self, n, nodes):
        return next((c for c in nodes if n in c.inputs), None)


def _gen_pointwise(kk: _K, nodes, shape) -> str:
    k = kk.k
    rank = len(shape)
    idx = [f"i{d}" for d in range(rank)]
    L = kk.header()
    if rank >= 2:
        L.append("  #pragma omp parallel for schedule(static)")
    for d in range(rank):
        if d == rank - 1:
            L.append("  #pragma omp simd")
        L.append(f"  for (long i{d} = 0; i{d} < {shape[d]}L; ++i{d}) {{")
    local = {}
    for n in k.inputs:
        st = _read_strides(n, kk.consumer(n, nodes), shape)
        L.append(f"    const float {kk.name[id(n)]} = {kk.name[id(n)]}p[{_offset(idx, st)}];")
        local[id(n)] = kk.name[id(n)]
    for n in nodes:
        val = local[id(n.inputs[0])] if n.op in ("transpose", "broadcast_to") else kk.expr(n, local)
        L.append(f"    const float {kk.name[id(n)]} = {val};")
        local[id(n)] = kk.name[id(n)]
    cs = _strides(shape)
    for j, o in enumerate(k.outputs):
        L.append(f"    y{j}p[{_offset(idx, cs)}] = {kk.name[id(o)]};")
    L += ["  }"] * rank
    L.append("}")
    return "\n".join(L)


def _gen_rows(kk: _K, stages, rows, N) -> str:
    """Row kernel or stand-alone reduction: per row, run every stage in order."""
    k = kk.k
    nrows = math.prod(rows) if rows else 1
    vshape = tuple(rows) + (N,)
    inside = {id(n) for n in k.nodes}
    out_of = {id(o): j for j, o in enumerate(k.outputs)}
    stage_of = {id(n): si for si, st in enumerate(stages) for n in st.nodes}
    scalar_ids = set()   # reduction results, their epilogues, scalar stages (by position)
    for st in stages:
        if st.kind == "reduce":
            scalar_ids |= {id(n) for n in st.nodes[st.nodes.index(st.anchor):]}
        elif tuple(st.iter_shape) != vshape:
            scalar_ids |= {id(n) for n in st.nodes}
    is_vec = lambda n: id(n) in inside and id(n) not in scalar_ids  # noqa: E731
    # row values another stage reads, or a per-row node reads (only with N == 1, where a
    # row is one element), go through a row buffer
    anchors = {id(st.anchor) for st in stages if st.kind == "reduce"}   # read their input in the row loop
    temps = [n for si, st in enumerate(stages) for n in st.nodes
             if is_vec(n) and id(n) not in out_of
             and any(stage_of.get(id(u), si) != si or not (is_vec(u) or id(u) in anchors)
                     for u in n.users if id(u) in inside)]
    temp_of = {id(n): i for i, n in enumerate(temps)}
    rstr = _strides(rows)
    ridx = [f"r{d}" for d in range(len(rows))]

    def vec_ref(n, i="n"):
        if id(n) in out_of:
            return f"y{out_of[id(n)]}p[r * {N}L + {i}]"
        return f"w{temp_of[id(n)]}[{i}]"

    L = kk.header()
    L.append("  #pragma omp parallel")
    L.append("  {")
    for i in range(len(temps)):
        L.append(f"  float* restrict w{i} = (float*)malloc(sizeof(float) * {N});")
    L.append("  #pragma omp for schedule(static)")
    L.append(f"  for (long r = 0; r < {nrows}L; ++r) {{")
    for d, s in enumerate(rstr):
        L.append(f"    const long r{d} = (r / {s}L) % {rows[d]}L;")
    scal = [n for n in k.nodes if not is_vec(n)]
    if scal:
        L.append("    float " + ", ".join(kk.name[id(n)] for n in scal) + ";")

    def vec_loads(st, used_nodes):
        out, local = [], {}
        for n in st.inputs:
            if not any(n in m.inputs for m in used_nodes):
                continue
            if id(n) in inside:
                local[id(n)] = vec_ref(n) if is_vec(n) else kk.name[id(n)]
            else:
                strd = _read_strides(n, kk.consumer(n, used_nodes), vshape)
                out.append(f"const float {kk.name[id(n)]}v = {kk.name[id(n)]}p[{_offset(ridx + ['n'], strd)}];")
                local[id(n)] = f"{kk.name[id(n)]}v"
        return out, local

    def scalar_loads(st, used_nodes, shape, local):
        out = []
        idx = ridx + (["0"] * (len(shape) - len(rows)))
        for n in list(st.inputs) + [i for m in used_nodes for i in m.inputs if is_vec(i)]:
            if id(n) in local or not any(n in m.inputs for m in used_nodes):
                continue
            if id(n) in inside and is_vec(n):
                local[id(n)] = vec_ref(n, "0")      # N == 1: the row's one element
            elif id(n) in inside:
                local[id(n)] = kk.name[id(n)]
            else:
                strd = _read_strides(n, kk.consumer(n, used_nodes), shape)
                out.append(f"    const float {kk.name[id(n)]}s = {kk.name[id(n)]}p[{_offset(idx, strd)}];")
                local[id(n)] = f"{kk.name[id(n)]}s"
        return out

    for si, st in enumerate(stages):
        L.append(f"    /* stage {si}: {st.kind} {[n.op for n in st.nodes]} */")
        if st.kind == "reduce":
            red = st.anchor
            pos = st.nodes.index(red)
            pro, epi = st.nodes[:pos], st.nodes[pos + 1:]
            loads, local = vec_loads(st, pro + [red])
            body = list(loads)
            for n in pro:
                body.append(f"const float {kk.name[id(n)]} = {kk.expr(n, local)};")
                local[id(n)] = kk.name[id(n)]
                if id(n) in out_of:
                    body.append(f"y{out_of[id(n)]}p[r * {N}L + n] = {kk.name[id(n)]};")
                elif id(n) in temp_of:
                    body.append(f"w{temp_of[id(n)]}[n] = {kk.name[id(n)]};")
            xv = local[id(red.inputs[0])]
            if red.op == "max":
                init, upd, clause = "-INFINITY", f"acc = fmaxf(acc, {xv});", "max"
            else:
                init, upd, clause = "0.0f", f"acc += {xv};", "+"
            body.append(upd)
            L.append("    {")
            L.append(f"    float acc = {init};")
            L.append(f"    #pragma omp simd reduction({clause}:acc)")
            L.append(f"    for (long n = 0; n < {N}L; ++n) {{")
            L += ["      " + s for s in body]
            L.append("    }")
            if red.op == "mean":
                L.append(f"    acc = acc / {float(N)!r}f;")
            L.append(f"    {kk.name[id(red)]} = acc;")
            L.append("    }")
            if id(red) in out_of:
                L.append(f"    y{out_of[id(red)]}p[r] = {kk.name[id(red)]};")
            elocal = {id(red): kk.name[id(red)]}
            L += scalar_loads(st, epi, tuple(red.shape), elocal)
            for n in epi:
                L.append(f"    {kk.name[id(n)]} = {kk.expr(n, elocal)};")
                elocal[id(n)] = kk.name[id(n)]
                if id(n) in out_of:
                    L.append(f"    y{out_of[id(n)]}p[r] = {kk.name[id(n)]};")
        elif tuple(st.iter_shape) == vshape:
            loads, local = vec_loads(st, st.nodes)
            body = list(loads)
            for n in st.nodes:
                body.append(f"const float {kk.name[id(n)]} = {kk.expr(n, local)};")
                local[id(n)] = kk.name[id(n)]
                if id(n) in out_of:
                    body.append(f"y{out_of[id(n)]}p[r * {N}L + n] = {kk.name[id(n)]};")
                elif id(n) in temp_of:
                    body.append(f"w{temp_of[id(n)]}[n] = {kk.name[id(n)]};")
            L.append("    #pragma omp simd")
            L.append(f"    for (long n = 0; n < {N}L; ++n) {{")
            L += ["      " + s for s in body]
            L.append("    }")
        else:
            local = {}
            L += scalar_loads(st, st.nodes, tuple(st.iter_shape), local)
            for n in st.nodes:
                L.append(f"    {kk.name[id(n)]} = {kk.expr(n, local)};")
                local[id(n)] = kk.name[id(n)]
                if id(n) in out_of:
                    L.append(f"    y{out_of[id(n)]}p[r] = {kk.name[id(n)]};")
    L.append("  }")
    for i in range(len(temps)):
        L.append(f"  free(w{i});")
    L += ["  }", "}"]
    return "\n".join(L)


def _gen_matmul(kk: _K) -> str:
    """C = A @ op(B) in fp32 (blocked over rows of A), then the epilogue per element."""
    k = kk.k
    mm = k.anchor
    a, b = mm.inputs
    tb = bool(mm.attrs.get("trans_b"))
    M, K = a.shape[-2], a.shape[-1]
    N = b.shape[-2] if tb else b.shape[-1]
    out_shape = tuple(mm.shape)
    bshape = out_shape[:-2]
    nb = math.prod(bshape) if bshape else 1

    def bst(t):
        cs = _strides(t.shape)
        lead = len(bshape) - (len(t.shape) - 2)
        return [0] * lead + [0 if t.shape[d] == 1 and bshape[lead + d] != 1 else cs[d] for d in range(len(t.shape) - 2)]

    bidx = [f"b{d}" for d in range(len(bshape))]
    bcs = _strides(bshape)
    A, B = kk.name[id(a)], kk.name[id(b)]
    epi = [n for n in k.nodes if n is not mm]
    L = kk.header()
    L.append("  #pragma omp parallel")
    L.append("  {")
    L.append(f"  float* restrict row = (float*)malloc(sizeof(float) * {N});")
    L.append("  #pragma omp for collapse(2) schedule(static)")
    L.append(f"  for (long bi = 0; bi < {nb}L; ++bi)")
    L.append(f"  for (long i = 0; i < {M}L; ++i) {{")
    for d, s in enumerate(bcs):
        L.append(f"    const long b{d} = (bi / {s}L) % {bshape[d]}L;")
    L.append(f"    const float* restrict Ar = {A}p + ({_offset(bidx, bst(a))}) + i * {K}L;")
    L.append(f"    const float* restrict Bm = {B}p + ({_offset(bidx, bst(b))});")
    if tb:
        L.append(f"    for (long j = 0; j < {N}L; ++j) {{")
        L.append("      const float* restrict Br = Bm + j * %dL;" % K)
        L.append("      float s = 0.0f;")
        L.append("      #pragma omp simd reduction(+:s)")
        L.append(f"      for (long q = 0; q < {K}L; ++q) s += Ar[q] * Br[q];")
        L.append("      row[j] = s;")
        L.append("    }")
    else:
        L.append(f"    for (long j = 0; j < {N}L; ++j) row[j] = 0.0f;")
        L.append(f"    for (long q = 0; q < {K}L; ++q) {{")
        L.append("      const float av = Ar[q];")
        L.append(f"      const float* restrict Br = Bm + q * {N}L;")
        L.append("      #pragma omp simd")
        L.append(f"      for (long j = 0; j < {N}L; ++j) row[j] += av * Br[j];")
        L.append("    }")
    L.append("    #pragma omp simd")
    L.append(f"    for (long j = 0; j < {N}L; ++j) {{")
    local = {id(mm): kk.name[id(mm)]}
    L.append(f"      const float {kk.name[id(mm)]} = row[j];")
    oidx = bidx + ["i", "j"]
    # the inputs the epilogue reads -- an operand of the product included
    # (``x + linear(x, w)``).  The reference's c backend drops both operands from its
    # epilogue inputs (tensorjit/backends/c_backend.py:215), so its generated C does not
    # compile for that graph; this restatement reads them like any other input.
    used = {id(i) for n in epi for i in n.inputs}
    for n in k.inputs:
        if id(n) not in used:
            continue
        strd = _read_strides(n, kk.consumer(n, epi), out_shape)
        L.append(f"      const float {kk.name[id(n)]} = {kk.name[id(n)]}p[{_offset(oidx, strd)}];")
        local[id(n)] = kk.name[id(n)]
    for n in epi:
        L.append(f"      const float {kk.name[id(n)]} = {kk.expr(n, local)};")
        local[id(n)] = kk.name[id(n)]
    ocs = _strides(out_shape)
    for j, o in enumerate(k.outputs):
        L.append(f"      y{j}p[{_offset(oidx, ocs)}] = {kk.name[id(o)]};")
    L += ["    }", "  }", "  free(row);", "  }", "}"]
    return "\n".join(L)


def generate(program) -> str:
    parts = [C_PRELUDE]
    for idx, k in enumerate(program.kernels):
        for n in k.nodes + k.inputs:
            if n.dtype.value != "f32":
                raise NotImplementedError(f"the C oracle is fp32 only (got {n.dtype.value} at {n.name})")
        kk = _K(k, idx)
        if k.kind in ("elementwise", "copy"):
            parts.append(_gen_pointwise(kk, k.nodes, tuple(k.iter_shape)))
        elif k.kind == "reduce":
            x = k.anchor.inputs[0]
            parts.append(_gen_rows(kk, [k], tuple(x.shape[:-1]), x.shape[-1]))
        elif k.kind == "row":
            parts.append(_gen_rows(kk, k.stages, tuple(k.rows), k.n))
        elif k.kind == "matmul":
            parts.append(_gen_matmul(kk))
        else:
            raise NotImplementedError(k.kind)
    return "\n\n".join(parts)


FLAGS = ["-O3", "-shared", "-fPIC", "-ffast-math", "-march=native", "-fopenmp", "-std=c11"]


def build(source: str) -> ctypes.CDLL:
    tag = hashlib.sha256(("oracle-v2\0" + source).encode()).hexdigest()[:20]
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    so = BUILD_DIR / f"oracle_{tag}.so"
    if not so.exists():
        cc = os.environ.get("CC") or shutil.which("gcc")
        if not cc:
            raise RuntimeError("the C oracle needs gcc")
        with tempfile.TemporaryDirectory() as td:
            src = Path(td) / "k.c"
            src.write_text(source)
            tmp = Path(td) / "k.so"
            r = subprocess.run([cc, *FLAGS, str(src), "-o", str(tmp), "-lm"], capture_output=True, text=True)
            if r.returncode:
                raise RuntimeError(f"oracle C compile failed:\n{r.stderr}\n{source}")
            shutil.move(str(tmp), so)
    return ctypes.CDLL(str(so))


def gen_runner(program, plan, in_index: dict[int, int], out_index: dict[int, int]) -> str:
    """``tj_run(in, out, arena)``: every kernel of the program in order, each argument
    resolved at generation time to caller input i, caller output j or arena + offset --
    the execution model of the reference's native runtime (``csrc/runtime.cpp:46-110``:
    pre-resolved INPUT/OUTPUT/ARENA references, one planned arena, one call per program)."""
    lines = ["void tj_run(void* const* in, void* const* out, char* arena) {"]
    for idx, k in enumerate(program.kernels):
        refs = []
        for n in list(k.inputs) + list(k.outputs):
            src = program.resolve(n)
            if id(src) in in_index:
                refs.append(f"in[{in_index[id(src)]}]")
            elif id(src) in out_index:
                refs.append(f"out[{out_index[id(src)]}]")
            else:
                off = plan.offset(src)
                if off is None:
                    raise RuntimeError(f"{n.name}: no storage in the oracle's plan")
                refs.append(f"(void*)(arena + {off})")
        lines.append(f"  {{ void* a[] = {{{', '.join(refs) or '0'}}}; k{idx}(a); }}")
    lines.append("}")
    return "\n".join(lines)


class OracleProgram:
    """Runs a fused program on CPU fp32 tensors through the generated C: one native call
    per program call (``tj_run``), intermediates in one planned arena reused by every call."""

    def __init__(self, program):
        from tensorjit.passes.memory_planner import plan_memory

        self.program = program
        g = program.graph
        self.plan = plan_memory(program)
        in_index = {id(n): i for i, n in enumerate(g.inputs)}
        returned = {id(program.resolve(o)) for o in g.outputs}
        self._out_nodes = []
        for k in program.kernels:
            for o in k.outputs:
                if id(o) in returned and id(o) not in in_index and all(o is not x for x in self._out_nodes):
                    self._out_nodes.append(o)
        out_index = {id(o): j for j, o in enumerate(self._out_nodes)}
        self.source = generate(program) + "\n\n" + gen_runner(program, self.plan, in_index, out_index)
        self.lib = build(self.source)
        self._run = self.lib.tj_run
        self._run.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_void_p), ctypes.c_void_p]
        self._run.restype = None
        # torch's CPU allocations are 64-byte aligned, the planner's alignment
        self.arena = torch.empty(max(self.plan.arena_bytes, 64), dtype=torch.uint8)

    def __call__(self, *inputs: torch.Tensor) -> list[torch.Tensor]:
        g = self.program.graph
        if len(inputs) != len(g.inputs):
            raise TypeError(f"expected {len(g.inputs)} inputs, got {len(inputs)}")
        ins = []
        for node, t in zip(g.inputs, inputs):
            if tuple(t.shape) != tuple(node.shape):
                raise ValueError(f"{node.name}: expected {node.shape}, got {tuple(t.shape)}")
            ins.append(t.detach().to("cpu", torch.float32).contiguous())
        outs = [torch.empty(o.shape, dtype=torch.float32) for o in self._out_nodes]
        cin = (ctypes.c_void_p * max(len(ins), 1))(*[t.data_ptr() for t in ins])
        cout = (ctypes.c_void_p * max(len(outs), 1))(*[t.data_ptr() for t in outs])
        self._run(cin, cout, self.arena.data_ptr())
        env = {id(n): t for n, t in zip(g.inputs, ins)}
        env.update({id(o): t for o, t in zip(self._out_nodes, outs)})
        result = []
        for o in g.outputs:
            src = self.program.resolve(o)
            if id(src) in env:
                t = env[id(src)]
            elif src.op == "const":
                t = torch.full(src.shape, src.attrs["value"], dtype=torch.float32)
            else:
                raise RuntimeError(f"output {o.name} was not produced")
            result.append(t.reshape(o.shape))
        return result


def compile_program(program) -> OracleProgram:
    return OracleProgram(program)
