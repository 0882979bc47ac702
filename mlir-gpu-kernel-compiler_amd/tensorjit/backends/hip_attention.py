"""Fused attention for the hip backend: ``matmul(q, kᵀ)·scale → softmax → matmul(·, v)``.

The reference passes plan attention as three kernels (a batched ``matmul`` with
``trans_b`` and a scale epilogue, a 4-stage softmax ``row`` kernel, a batched NN
``matmul``), materialising the ``[B, H, S, S]`` scores and probabilities in
memory.  ``fuse_attention`` recognises that chain in the planned program (the
passes themselves are unchanged) and replaces it with one ``attention`` kernel,
so the scores never leave the chip and the memory planner no longer reserves
arena space for them.

``gen_attention`` emits a gfx950 flash-attention forward kernel: a workgroup of
4 waves owns 128 query rows (32 per wave) of one (batch, head); key/value blocks
of 64 rows stream through double-buffered LDS.  Each wave computes the scores
transposed, ``Sᵀ = K·Qᵀ`` (MFMA 32x32x16, queries as columns), so every lane owns
one query column: the online-softmax max / sum need one cross-lane exchange
(``lane ^ 32``) per block, the rescale of the output accumulator is a per-lane
multiply, and the probabilities go from the score accumulator straight into the
B operand of ``Oᵀ += Vᵀ·Pᵀ`` without an LDS round trip.  For that, V is stored
transposed in LDS with the keys of every 16-key chunk permuted (bits 2 and 3 of
the key offset swapped) so one 16-byte read returns the keys in the order the
score accumulator holds them.
"""
from __future__ import annotations

import math
import os

from ..ir import DType, Node
from ..passes import Kernel, Program
from .hip_prelude import CTYPE

BQ_PER_WAVE = 32
WAVES = 4
BKV = 64
MAX_HEAD_DIM = 128


# ---------------------------------------------------------------------------
# pattern: matmul(q, k, trans_b)[* scale] -> softmax row kernel -> matmul(p, v)
# ---------------------------------------------------------------------------


def _scalar_const(n: Node) -> float | None:
    return n.attrs["value"] if n.op == "const" and n.shape == () else None


def _score_scale(k1: Kernel) -> float | None:
    """The scale of ``k1 = matmul(q, k, trans_b)`` followed by at most one scalar multiply."""
    mm = k1.anchor
    if k1.kind != "matmul" or not mm.attrs.get("trans_b"):
        return None
    if k1.nodes == [mm]:
        return 1.0
    if len(k1.nodes) != 2 or k1.nodes[1].op != "mul":
        return None
    a, b = k1.nodes[1].inputs
    other = b if a is mm else a if b is mm else None
    return None if other is None else _scalar_const(other)


def _is_last_axis_reduce(n: Node, op: str, x: Node) -> bool:
    if n.op != op or n.inputs != [x] or not n.attrs.get("keepdim"):
        return False
    axis = n.attrs.get("axis", -1)
    return axis in (-1, len(x.shape) - 1)


def _is_softmax_row(k2: Kernel, s: Node) -> Node | None:
    """``k2`` is exactly ``exp(s - max(s)) / sum(exp(...))`` over the last axis; returns its output."""
    if k2.kind != "row" or [n.op for n in k2.nodes] != ["max", "sub", "exp", "sum", "div"]:
        return None
    mx, sub, ex, sm, div = k2.nodes
    ok = (_is_last_axis_reduce(mx, "max", s) and sub.inputs == [s, mx] and ex.inputs == [sub]
          and _is_last_axis_reduce(sm, "sum", ex) and div.inputs == [ex, sm])
    return div if ok and k2.outputs == [div] else None


def _only_used_by(n: Node, users: list[Node], graph_outputs: set[int]) -> bool:
    ids = {id(u) for u in users}
    return id(n) not in graph_outputs and all(id(u) in ids for u in n.users)


def match_attention(program: Program, i3: int) -> dict | None:
    """If kernel ``i3`` is the PV product of a fusable attention chain, describe it."""
    kernels = program.kernels
    k3 = kernels[i3]
    if k3.kind != "matmul" or k3.nodes != [k3.anchor] or k3.anchor.attrs.get("trans_b"):
        return None
    mm3 = k3.anchor
    p, v = mm3.inputs
    producer = {id(o): i for i, k in enumerate(kernels) for o in k.outputs}
    i2 = producer.get(id(p))
    if i2 is None or i2 >= i3:
        return None
    k2 = kernels[i2]
    if len(k2.inputs) != 1:
        return None
    s = k2.inputs[0]
    if _is_softmax_row(k2, s) is not p:
        return None
    i1 = producer.get(id(s))
    if i1 is None or i1 >= i2:
        return None
    k1 = kernels[i1]
    scale = _score_scale(k1)
    if scale is None or k1.outputs != [s]:
        return None
    outs = {id(program.resolve(o)) for o in program.graph.outputs}
    if not (_only_used_by(s, k2.nodes, outs) and _only_used_by(p, [mm3], outs)):
        return None
    q, kk = k1.anchor.inputs
    dt = q.dtype
    if dt not in (DType.bf16, DType.f16) or kk.dtype != dt or v.dtype != dt or mm3.dtype != dt:
        return None
    if len(q.shape) < 2 or not (q.shape[:-2] == kk.shape[:-2] == v.shape[:-2] == mm3.shape[:-2]):
        return None
    Sq, D = q.shape[-2:]
    Sk, Dv = kk.shape[-2], v.shape[-1]
    if kk.shape[-1] != D or v.shape[-2] != Sk or tuple(p.shape[-2:]) != (Sq, Sk):
        return None
    if D % 16 or D > MAX_HEAD_DIM or Dv % 32 or Dv > MAX_HEAD_DIM or Sq < 1 or Sk < 1:
        return None
    if math.prod(q.shape[:-2]) > 65535:         # one (batch, head) per grid row
        return None
    return {"i1": i1, "i2": i2, "i3": i3, "q": q, "k": kk, "v": v, "out": mm3, "scale": float(scale),
            "nodes": k1.nodes + k2.nodes + k3.nodes}


def fuse_attention(program: Program) -> Program:
    """Replace every fusable attention chain by one ``attention`` kernel at the PV
    product's position (its inputs are live there; the scores and probabilities
    have no other user).  ``TENSORJIT_HIP_ATTENTION=0`` keeps the three kernels."""
    if os.environ.get("TENSORJIT_HIP_ATTENTION", "1") == "0":
        return program
    kernels = list(program.kernels)
    changed = False
    i3 = 0
    while i3 < len(kernels):
        cur = Program(program.graph, kernels, program.aliases)
        m = match_attention(cur, i3)
        if m is None:
            i3 += 1
            continue
        fused = Kernel("attention", nodes=m["nodes"], anchor=m["out"], inputs=[m["q"], m["k"], m["v"]],
                       outputs=list(kernels[i3].outputs))
        fused.attn = {"scale": m["scale"]}  # type: ignore[attr-defined]
        kernels[i3] = fused
        for i in sorted((m["i1"], m["i2"]), reverse=True):
            del kernels[i]
        i3 -= 2
        changed = True
    return Program(program.graph, kernels, program.aliases) if changed else program


# ---------------------------------------------------------------------------
# gfx950 flash-attention forward
# ---------------------------------------------------------------------------


def _perm16(x: str) -> str:
    """Position of key offset ``x`` inside its 16-key chunk (bits 2 and 3 swapped)."""
    return f"((({x}) & ~12u) | ((({x}) & 4u) << 1) | ((({x}) & 8u) >> 1))"


def gen_attention(k: Kernel, idx: int) -> tuple[str, "Launch"]:  # noqa: F821
    from .hip_kernels import Launch

    q, kk, v = k.inputs
    out = k.outputs[0]
    scale = k.attn["scale"]  # type: ignore[attr-defined]
    dt = q.dtype
    T = CTYPE[dt]
    batch = math.prod(q.shape[:-2]) if len(q.shape) > 2 else 1
    Sq, D = q.shape[-2:]
    Sk, Dv = kk.shape[-2], v.shape[-1]
    NW, THREADS = WAVES, WAVES * 64
    BQ = BQ_PER_WAVE * NW
    KB = -(-Sk // BKV)
    DP, VP = D + 8, BKV + 8                     # 16-byte row padding: conflict-free fragment reads
    opvec = "tj_bf16x8" if dt == DType.bf16 else "tj_f16x8"
    mfma = "__builtin_amdgcn_mfma_f32_32x32x16_bf16" if dt == DType.bf16 else "__builtin_amdgcn_mfma_f32_32x32x16_f16"
    KC = BKV * D // 8 // THREADS                  # 16-byte K chunks per lane per block
    VC = BKV * Dv // 8 // THREADS
    assert KC * THREADS * 8 == BKV * D and VC * THREADS * 8 == BKV * Dv
    idx_t = "unsigned long" if batch * max(Sq, Sk) * max(D, Dv) >= 2**31 else "unsigned int"
    ragged = Sk % BKV != 0
    bdims = "x".join(str(d) for d in q.shape[:-2]) or "1"
    fname = f"tj{idx}_attention_{bdims}x{Sq}x{Sk}x{D}_{dt.value}_flash"
    cs = scale * 1.4426950408889634            # scores scaled into exp2's domain
    if dt == DType.bf16:
        pack4 = "tj_f2bf2({0}, {1}) | ((unsigned long)tj_f2bf2({2}, {3}) << 32)"
    else:
        pack4 = ("(unsigned long)(tj_f2h({0}) | (tj_f2h({1}) << 16)) | "
                 "((unsigned long)(tj_f2h({2}) | (tj_f2h({3}) << 16)) << 32)")

    # two waves per SIMD (two workgroups per CU): one wave's softmax arithmetic runs
    # under the other's MFMAs; the compiler then keeps everything in 256 VGPRs
    L = [f'extern "C" __global__ void __launch_bounds__({THREADS}) __attribute__((amdgpu_waves_per_eu(2, 2))) {fname}(',
         f"    const {T}* __restrict__ in0_p, const {T}* __restrict__ in1_p, const {T}* __restrict__ in2_p,",
         f"    {T}* __restrict__ out0_p) {{",
         f"  __shared__ __attribute__((aligned(16))) {T} Ks[2][{BKV}][{DP}];",
         f"  __shared__ __attribute__((aligned(16))) {T} Vs[2][{Dv}][{VP}];",
         "  const unsigned int tid = threadIdx.x, lane = tid % 64u, wave = tid / 64u;",
         "  const unsigned int g = lane / 32u, col = lane % 32u;",
         f"  const {idx_t} bh = blockIdx.y;",
         f"  const {T}* __restrict__ Qb = in0_p + bh * {Sq * D}u;",
         f"  const {T}* __restrict__ Kb = in1_p + bh * {Sk * D}u;",
         f"  const {T}* __restrict__ Vb = in2_p + bh * {Sk * Dv}u;",
         f"  {T}* __restrict__ Ob = out0_p + bh * {Sq * Dv}u;",
         f"  const unsigned int qrow = blockIdx.x * {BQ}u + wave * 32u + col;",
         f"  const unsigned int qc = qrow < {Sq}u ? qrow : {Sq - 1}u;",
         # Q as the B operand of S^T = K Q^T: chunk c holds Q[q][c*16 + g*8 .. +8]
         f"  {opvec} qf[{D // 16}];",
         "#pragma unroll",
         f"  for (int c = 0; c < {D // 16}; ++c) qf[c] = *(const {opvec}*)&Qb[qc * {D}u + c * 16 + g * 8u];",
         f"  tj_f32x16 o[{Dv // 32}];",
         "#pragma unroll",
         f"  for (int u = 0; u < {Dv // 32}; ++u) o[u] = (tj_f32x16)(0.0f);",
         "  float m_run = -__builtin_inff(), l_run = 0.0f;",
         f"  tj_u32x4 rk[{KC}], rv[{VC}];"]

    def load(blk: str) -> list[str]:
        out_l = ["#pragma unroll", f"  for (int i = 0; i < {KC}; ++i) {{",
                 f"    const unsigned int c = i * {THREADS}u + tid, row = c / {D // 8}u, d8 = (c % {D // 8}u) * 8u;",
                 f"    unsigned int key = ({blk}) * {BKV}u + row;"]
        if ragged:
            out_l.append(f"    key = key < {Sk}u ? key : {Sk - 1}u;")
        out_l += [f"    rk[i] = *(const tj_u32x4*)&Kb[key * {D}u + d8];", "  }",
                  "#pragma unroll", f"  for (int i = 0; i < {VC}; ++i) {{",
                  # consecutive lanes take consecutive keys: the transposing 2-byte LDS
                  # stores below then hit consecutive addresses
                  f"    const unsigned int c = i * {THREADS}u + tid, row = c % {BKV}u, d8 = (c / {BKV}u) * 8u;",
                  f"    unsigned int key = ({blk}) * {BKV}u + row;"]
        if ragged:
            out_l.append(f"    key = key < {Sk}u ? key : {Sk - 1}u;")
        out_l += [f"    rv[i] = *(const tj_u32x4*)&Vb[key * {Dv}u + d8];", "  }"]
        return out_l

    def store(buf: str) -> list[str]:
        out_l = ["#pragma unroll", f"  for (int i = 0; i < {KC}; ++i) {{",
                 f"    const unsigned int c = i * {THREADS}u + tid, row = c / {D // 8}u, d8 = (c % {D // 8}u) * 8u;",
                 f"    *(tj_u32x4*)&Ks[{buf}][row][d8] = rk[i];", "  }",
                 "#pragma unroll", f"  for (int i = 0; i < {VC}; ++i) {{",
                 f"    const unsigned int c = i * {THREADS}u + tid, row = c % {BKV}u, d8 = (c / {BKV}u) * 8u;",
                 f"    const unsigned int pos = (row & ~15u) | {_perm16('row & 15u')};",
                 "#pragma unroll", "    for (int w = 0; w < 4; ++w) {",
                 "      const unsigned int x_ = rv[i][w];"]
        lo, hi = "(unsigned short)(x_ & 0xffffu)", "(unsigned short)(x_ >> 16)"
        if dt == DType.f16:
            lo, hi = f"__builtin_bit_cast(_Float16, {lo})", f"__builtin_bit_cast(_Float16, {hi})"
        out_l += [f"      Vs[{buf}][d8 + 2 * w][pos] = {lo};", f"      Vs[{buf}][d8 + 2 * w + 1][pos] = {hi};",
                  "    }", "  }"]
        return out_l

    L += load("0u")
    L += store("0")
    if KB > 1:
        L += load("1u")
    L.append("  __syncthreads();")
    L.append(f"  for (int j = 0; j < {KB}; ++j) {{")
    L.append("    const int buf = j & 1;")
    # S^T = K Q^T over D in 16-wide chunks: tile t covers keys t*32 .. t*32+31
    L += [f"    tj_f32x16 s[{BKV // 32}];",
          "#pragma unroll",
          f"    for (int t = 0; t < {BKV // 32}; ++t) s[t] = (tj_f32x16)(0.0f);",
          "#pragma unroll",
          f"    for (int c = 0; c < {D // 16}; ++c)",
          "#pragma unroll",
          f"      for (int t = 0; t < {BKV // 32}; ++t)",
          f"        s[t] = {mfma}(*(const {opvec}*)&Ks[buf][t * 32 + col][c * 16 + g * 8u], qf[c], s[t], 0, 0, 0);"]
    # online softmax, one query column per lane (its 32 keys here + lane ^ 32's 32)
    L += ["    float mx = -__builtin_inff();",
          "#pragma unroll",
          f"    for (int t = 0; t < {BKV // 32}; ++t)",
          "#pragma unroll",
          "      for (int r = 0; r < 16; ++r) {",
          f"        float x = s[t][r] * {cs!r}f;"]
    if ragged:
        L.append(f"        if (j * {BKV} + t * 32 + (r / 4) * 8 + (int)g * 4 + r % 4 >= {Sk}) x = -__builtin_inff();")
    L += ["        s[t][r] = x;",
          "        mx = fmaxf(mx, x);",
          "      }",
          "    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));",
          "    const float m_new = fmaxf(m_run, mx);",
          "    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);",
          "    float rs = 0.0f;",
          "#pragma unroll",
          f"    for (int t = 0; t < {BKV // 32}; ++t)",
          "#pragma unroll",
          "      for (int r = 0; r < 16; ++r) {",
          "        const float e = __builtin_amdgcn_exp2f(s[t][r] - m_new);",
          "        s[t][r] = e;",
          "        rs += e;",
          "      }",
          "    rs += __shfl_xor(rs, 32, 64);",
          "    l_run = l_run * alpha + rs;",
          "    m_run = m_new;",
          "#pragma unroll",
          f"    for (int u = 0; u < {Dv // 32}; ++u) o[u] *= alpha;"]
    # O^T += V^T P^T: chunk ch = 2t + h holds keys t*32 + 16h .. +15 (in the permuted order)
    L += ["#pragma unroll",
          f"    for (int t = 0; t < {BKV // 32}; ++t)",
          "#pragma unroll",
          "      for (int h = 0; h < 2; ++h) {",
          "        tj_u32x4 pw;",
          "#pragma unroll",
          "        for (int w = 0; w < 4; ++w) pw[w] = "
          + ("tj_f2bf2(s[t][8 * h + 2 * w], s[t][8 * h + 2 * w + 1]);" if dt == DType.bf16 else
             "tj_f2h(s[t][8 * h + 2 * w]) | (tj_f2h(s[t][8 * h + 2 * w + 1]) << 16);"),
          f"        const {opvec} pf = __builtin_bit_cast({opvec}, pw);",
          "#pragma unroll",
          f"        for (int u = 0; u < {Dv // 32}; ++u)",
          f"          o[u] = {mfma}(*(const {opvec}*)&Vs[buf][u * 32 + col][(2 * t + h) * 16 + g * 8u], pf, o[u], 0, 0, 0);",
          "      }"]
    L.append(f"    if (j + 1 < {KB}) {{")
    L += ["    " + x for x in store("buf ^ 1")]
    L.append("    }")
    L.append(f"    if (j + 2 < {KB}) {{")
    L += ["    " + x for x in load("(unsigned int)(j + 2)")]
    L.append("    }")
    L.append("    __syncthreads();")
    L.append("  }")
    # O = O^T / l: lane holds 4 consecutive dv per (u, r/4) for its query
    L += [f"  if (qrow < {Sq}u) {{",
          "    const float inv = 1.0f / l_run;",
          "#pragma unroll",
          f"    for (int u = 0; u < {Dv // 32}; ++u)",
          "#pragma unroll",
          "      for (int r4 = 0; r4 < 4; ++r4) {",
          "        const unsigned int dv = u * 32 + r4 * 8 + g * 4u;",
          "        *(unsigned long*)&Ob[qrow * " + f"{Dv}u + dv] = "
          + pack4.format("o[u][r4 * 4] * inv", "o[u][r4 * 4 + 1] * inv", "o[u][r4 * 4 + 2] * inv",
                         "o[u][r4 * 4 + 3] * inv") + ";",
          "      }",
          "  }",
          "}"]
    lds = 2 * (BKV * DP + Dv * VP) * dt.itemsize
    flops = 2.0 * batch * Sq * Sk * (D + Dv)
    meta = {"family": "attention", "dtype": dt.value, "batch": batch, "Sq": Sq, "Sk": Sk, "D": D, "Dv": Dv,
            "scale": scale, "lds_bytes": lds, "flops": flops}
    return "\n".join(L), Launch(fname, (-(-Sq // BQ), batch, 1), (THREADS, 1, 1), 0, meta)
