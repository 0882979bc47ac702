"""Fused attention for the hip backend: ``matmul(q, kᵀ)·scale → softmax → matmul(·, v)``.

The reference passes plan attention as three kernels (a batched ``matmul`` with
``trans_b`` and a scale epilogue, a 4-stage softmax ``row`` kernel, a batched NN
``matmul``), materialising the ``[B, H, S, S]`` scores and probabilities in
memory.  ``fuse_attention`` recognises that chain in the planned program (the
passes themselves are unchanged) and replaces it with one ``attention`` kernel,
so the scores never leave the chip and the memory planner no longer reserves
arena space for them.

``gen_attention`` emits a gfx950 flash-attention forward kernel: a workgroup of
4 or 8 waves owns 32 query rows per wave of one (batch, head); key/value blocks
of 64 rows stream through double-buffered LDS.  Each wave computes the scores
transposed, ``Sᵀ = K·Qᵀ`` (MFMA 32x32x16, queries as columns), so every lane owns
half the keys of one query column: the online softmax exchanges nothing with the
other half (``lane ^ 32``) unless the running maximum has to move, the rescale of
the output accumulator is a per-lane multiply, and the probabilities go from the
score accumulator straight into the
B operand of ``Oᵀ += Vᵀ·Pᵀ`` without an LDS round trip.  V stays in its natural
``[key][d]`` layout in LDS; the ``Vᵀ`` operand is gathered with gfx950's
transposing LDS read ``ds_read_b64_tr_b16`` (within each 16 lanes, lane ``i``
receives element ``i % 4`` of the 8-byte rows loaded by lanes ``4e + i / 4``,
e = 0..3), two per fragment, in the key order of the score accumulator.  At head dim
128 with 8 waves (K/V moved into LDS by DMA) the same data flow runs on 16x16x32
MFMAs: a wave's 32 queries are two 16-query column tiles, a query's keys of a block
sit on four lanes (l % 16 + 16 g), and each K or Vᵀ fragment feeds one MFMA of each
tile.

Grids short of one workgroup per CU (few heads, long keys) split the key range: each
workgroup runs the same loop over an equal share of the key blocks and stores its
unnormalised output rows with their running reference and sum in a workspace, and a
second launch combines the splits (weights ``2^(m_s - max m)``) and writes the output.
"""
from __future__ import annotations

import math
import os

from ..ir import DType, Node
from ..passes import Kernel, Program
from ..runtime.autotune import CU_COUNT
from .hip_prelude import CTYPE

BQ_PER_WAVE = 32
BKV = 64
MAX_HEAD_DIM = 128
# DMA schedule (head dim 128): how many fragment reads the score MFMAs (K) and the PV
# MFMAs (Vᵀ) keep in flight ahead of themselves, pinned by sched_group_barrier (0: the
# compiler's own order).  Same box, interleaved, bit-identical outputs, [4,32,2048,128],
# (KS, PV): compiler's order 260.4 us, (2, 2) 248.9, (2, 3) 248.7, (3, 3) 249.3, (3, 4) 250.5,
# (2, 4) 250.8, (2, 6) 252.2, (1, 4) 256.5; another box: compiler's order 262.6, (0, 4)
# 256.4, (4, 0) 252.9, (4, 4) 250.5; [1,32,8192,128] 929.4 -> 878.9 at (2, 2)
KS_AHEAD = 2
PV_AHEAD = 2
# the same for the register-staged schedules (4 waves, and 8 waves below head dim 128); K
# reads ahead only from head dim 128.  Same box, bit-identical, (KS, PV): [1,16,2048,128]
# (4 waves, 128 workgroups) compiler's order 50.8 us, (2, 2) 46.1, (2, 0) 45.8; head dim 64
# [4,32,2048,64] 159.7 -> 157.4 at (0, 2), 8 waves 161.5 -> 159.3; 16 queries x 4096 keys
# [8,32,*,64] 47.9 -> 47.5 at (0, 2) but 55.1 at (2, 2)
KS_AHEAD_STAGED = 2
PV_AHEAD_STAGED = 2
SG_MFMA, SG_DS_READ = 0x008, 0x100

# The DMA schedule runs on 16x16x32 MFMAs (TENSORJIT_HIP_ATTENTION_MI16=0 keeps 32x32x16):
# each wave's 32 queries are two 16-query column tiles, and every K and Vᵀ fragment feeds
# one MFMA of each, so the LDS reads per FLOP stay those of the 32x32x16 form.  The card is
# power-limited, and a 16x16x32 stream on random data holds a higher clock (2197 against
# 1810 MHz for 32x32x16, one box).  Same box, interleaved, best of three, accuracy against
# fp32 unchanged (relative norm error 2.342e-3 for both): [4,32,2048,128] 247.6 -> 238.0 us,
# [1,32,2000,128] 65.0 -> 63.2, [1,32,8192,128] 893.6 -> 861.7.  Fragment reads in flight
# (KS, PV), bit-identical: (2, 2) 238.0 / 860.9 us ([4,32,2048,128] / [1,32,8192,128]),
# (1, 1) 262.6 / 944.8, (2, 1) 249.0 / 894.1, (2, 3) 237.8 / 859.8, (3, 3) 236.9 / 855.9,
# (3, 2) 236.6 / 854.1, (4, 4) 236.4 / 853.1 (254 VGPRs).
KS_AHEAD16 = 3
PV_AHEAD16 = 2
QUAD_HELPERS = r"""#ifndef TJ_QUAD_LANES
#define TJ_QUAD_LANES
// lanes l, l ^ 16, l ^ 32, l ^ 48 combined: v_permlane16_swap exchanges the odd and even
// 16-lane rows, v_permlane32_swap the halves; each step combines a pair in either order,
// so the four lanes end with the same bits
__device__ __forceinline__ float tj_quad_max(float x) {
  const unsigned int u = __builtin_bit_cast(unsigned int, x);
  const auto s = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return tj_pair_max(fmaxf(__builtin_bit_cast(float, (unsigned int)s[0]), __builtin_bit_cast(float, (unsigned int)s[1])));
}
typedef _Float16 tj_f16x2q __attribute__((ext_vector_type(2)));
// sum of the two 16-bit probabilities of a packed pair, added to acc (v_dot2c with ones)
__device__ __forceinline__ float tj_pair_acc_bf16(unsigned int p, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(tj_bf16x2, p), __builtin_bit_cast(tj_bf16x2, 0x3F803F80u), acc, false);
}
__device__ __forceinline__ float tj_pair_acc_f16(unsigned int p, float acc) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(tj_f16x2q, p), __builtin_bit_cast(tj_f16x2q, 0x3C003C00u), acc, false);
}
__device__ __forceinline__ float tj_quad_sum(float x) {
  const unsigned int u = __builtin_bit_cast(unsigned int, x);
  const auto s = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return tj_pair_sum(__builtin_bit_cast(float, (unsigned int)s[0]) + __builtin_bit_cast(float, (unsigned int)s[1]));
}
#endif
"""


def balance_enabled() -> bool:
    """16x16x32 DMA kernel: take each block's row sums from the 16-bit probabilities the
    PV MFMAs use (v_dot2 with ones) and the next block's extremes in the PV phase, instead
    of fp32 sums and extremes in the softmax phase.  Measured against fp32 reference
    attention the outputs are closer (the normaliser matches the weights applied: max
    error 2.8e-3 against 4.9e-3 of the largest output at [4,32,2048,128]); time equal."""
    return os.environ.get("TENSORJIT_HIP_ATTENTION_BALANCE", "1") != "0"


def mi16_enabled() -> bool:
    return os.environ.get("TENSORJIT_HIP_ATTENTION_MI16", "1") != "0"


# ---------------------------------------------------------------------------
# pattern: matmul(q, k, trans_b)[* scale] -> softmax row kernel -> matmul(p, v)
# ---------------------------------------------------------------------------


def _scalar_const(n: Node) -> float | None:
    return n.attrs["value"] if n.op == "const" and n.shape == () else None


def _score_scale(k1: Kernel) -> float | None:
    """The scale of ``k1 = matmul(q, k, trans_b)`` followed by at most one scalar multiply
    (either operand order) or one division of the scores by a nonzero scalar
    (``q @ kᵀ / sqrt(d)``, scale ``1 / c``; ``c / scores`` is not a scale)."""
    mm = k1.anchor
    if k1.kind != "matmul" or not mm.attrs.get("trans_b"):
        return None
    if k1.nodes == [mm]:
        return 1.0
    if len(k1.nodes) != 2 or k1.nodes[1].op not in ("mul", "div"):
        return None
    a, b = k1.nodes[1].inputs
    if k1.nodes[1].op == "div":
        c = _scalar_const(b) if a is mm else None
        return None if not c else 1.0 / c
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
    # K and V blocks are copied 16 bytes per lane: 64 keys x D (and x Dv) must cover the
    # 256 lanes of a 4-wave workgroup (8 waves need multiples of 64, as their layout does)
    if D % 32 or D > MAX_HEAD_DIM or Dv % 32 or Dv > MAX_HEAD_DIM or Sq < 1 or Sk < 1:
        return None
    if math.prod(q.shape[:-2]) > 65535 or scale == 0.0:   # one (batch, head) per grid row
        return None
    if math.prod(q.shape[:-2]) * max(Sq, Sk) * max(D, Dv) >= 2**32:   # 32-bit element offsets
        return None
    return {"i1": i1, "i2": i2, "i3": i3, "q": q, "k": kk, "v": v, "out": mm3, "scale": float(scale),
            "nodes": k1.nodes + k2.nodes + k3.nodes}


def _bshd_source(program: Program, t: Node, users_ok: set[int], outs: set[int]) -> tuple[int, Node] | None:
    """If ``t`` is a copy kernel's ``transpose(perm=(0,2,1,3))`` of a contiguous
    [B, S, H, D] value used only inside the fused chain, return (kernel index, source):
    the attention kernel can read the source through strides instead."""
    if t.op != "transpose" or tuple(t.attrs.get("perm", ())) != (0, 2, 1, 3) or len(t.shape) != 4:
        return None
    if id(t) in outs or not all(id(u) in users_ok for u in t.users):
        return None
    for i, k in enumerate(program.kernels):
        if k.kind == "copy" and k.nodes == [t] and k.outputs == [t]:
            return i, t.inputs[0]
    return None


def _bshd_sink(program: Program, o: Node, outs: set[int]) -> tuple[int, Node] | None:
    """If the attention output's only user is a copy kernel's transpose back to
    [B, S, H, D], return (kernel index, that transpose): the kernel writes it directly."""
    if id(o) in outs or len(o.users) != 1:
        return None
    t = o.users[0]
    if t.op != "transpose" or tuple(t.attrs.get("perm", ())) != (0, 2, 1, 3) or len(t.shape) != 4:
        return None
    for i, k in enumerate(program.kernels):
        if k.kind == "copy" and k.nodes == [t] and k.outputs == [t] and k.inputs == [o]:
            return i, t
    return None


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
        # head transposes on either side: read q/k/v from, and write o to, [B, S, H, D]
        outs = {id(cur.resolve(o)) for o in program.graph.outputs}
        fused_ids = {id(n) for n in m["nodes"]}
        drop = [m["i1"], m["i2"]]
        ins, layouts, nodes, seen = [], [], list(m["nodes"]), {}
        for x in (m["q"], m["k"], m["v"]):
            src = seen.get(id(x)) or _bshd_source(cur, x, fused_ids, outs)
            if src is not None:
                seen[id(x)] = src
                if src[0] not in drop:
                    drop.append(src[0])
                    nodes.insert(0, x)
                ins.append(src[1])
                layouts.append("bshd")
            else:
                ins.append(x)
                layouts.append("bhsd")
        out, out_layout = m["out"], "bhsd"
        sink = _bshd_sink(cur, m["out"], outs)
        if sink is not None:
            drop.append(sink[0])
            out, out_layout = sink[1], "bshd"
            nodes.append(sink[1])
        fused = Kernel("attention", nodes=nodes, anchor=m["out"], inputs=ins, outputs=[out])
        fused.attn = {"scale": m["scale"], "layouts": layouts, "out_layout": out_layout}  # type: ignore[attr-defined]
        kernels[i3] = fused
        for i in sorted(drop, reverse=True):
            del kernels[i]
        i3 = kernels.index(fused) + 1
        changed = True
        continue
    return Program(program.graph, kernels, program.aliases) if changed else program


# ---------------------------------------------------------------------------
# gfx950 flash-attention forward
# ---------------------------------------------------------------------------


XCDS = 8


def _tile_lines(nq: int, batch: int, idx_t: str) -> list[str]:
    """Workgroup -> (batch*head ``bh``, query tile ``qt``).  Workgroups are dealt to the
    8 XCDs round-robin; in groups of 8 heads the ``nq`` query tiles of one head share
    ``blockIdx.x % 8``, so they run on one XCD and its L2 serves the head's K and V once
    instead of once per XCD."""
    if nq > 1 and batch % XCDS == 0:
        return [f"  const unsigned int grp = blockIdx.x / {XCDS * nq}u, rem = blockIdx.x % {XCDS * nq}u;",
                f"  const {idx_t} bh = grp * {XCDS}u + rem % {XCDS}u;",
                f"  const unsigned int qt = rem / {XCDS}u;"]
    return [f"  const {idx_t} bh = blockIdx.x / {nq}u;", f"  const unsigned int qt = blockIdx.x % {nq}u;"]


def attention_layout(batch: int, Sq: int, D: int, Dv: int) -> tuple[int, int]:
    """(waves per workgroup, 32-row query tiles per wave).

    8 waves in two ping-pong groups share every K/V block between 256 queries (half the
    L2->CU traffic of 4 waves) while on each SIMD one group's softmax arithmetic runs
    under the other group's MFMAs; 4 independent waves per workgroup (128 queries, two
    workgroups per CU) otherwise.  Measured on MI355X (bf16): ping-pong is faster at head
    dims 128 once its grid fills the 256 CUs ([4,32,2048,128] 270 vs 299 us, [1,32,4096,128]
    255 vs 288, [8,32,1024,128] 154 vs 176, [2,8,4096,128] with exactly 256 workgroups
    128 vs 146); 4 waves are faster with fewer ping-pong workgroups ([1,16,2048,128] 51 vs
    55 us, [4,8,512,128] 16 vs 20) and at head dim 64 ([4,32,2048,64] 162 vs 169,
    [16,16,512,64] 27 vs 31; equal at [2,16,2048,64]).  TENSORJIT_HIP_ATTENTION_WAVES=4
    or 8 forces a schedule (8 needs head dims that are multiples of 64).  Two query
    tiles per wave would halve the LDS fragment reads per FLOP, but its accumulators do
    not fit beside the softmax operands in the 256 VGPRs the rescale arithmetic needs
    (the compiler spills)."""
    pingpong_ok = D % 64 == 0 and Dv % 64 == 0
    forced = os.environ.get("TENSORJIT_HIP_ATTENTION_WAVES")
    if forced in ("4", "8"):
        return (8 if forced == "8" and pingpong_ok else 4), 1
    if pingpong_ok and min(D, Dv) >= 128 and Sq >= 512 and batch * -(-Sq // 256) >= CU_COUNT:
        return 8, 1
    return 4, 1


def attention_splits(tiles: int, KB: int, pingpong: bool) -> int:
    """Key-range splits per (batch*head, query tile) for grids that leave CUs idle: with
    ``tiles`` workgroups short of one per CU, each workgroup takes an equal share of the
    key blocks (``KB`` divisible by the split count, at least 2 blocks each) and writes
    unnormalised partial outputs with their running maxima and sums; a second launch
    combines them.  The smallest split count that reaches 256 workgroups, else the largest
    one that divides ``KB``; 1 for the ping-pong schedule and for full grids.
    TENSORJIT_HIP_ATTENTION_SPLITS=n forces n where it divides ``KB`` into >= 2-block parts."""
    forced = os.environ.get("TENSORJIT_HIP_ATTENTION_SPLITS", "")
    ok = [n for n in range(2, 33) if KB % n == 0 and KB // n >= 2]
    if pingpong:
        return 1
    if forced.isdigit():
        return int(forced) if int(forced) in ok else 1
    if tiles >= CU_COUNT or not ok:
        return 1
    return next((n for n in ok if tiles * n >= CU_COUNT), ok[-1])


def _split_tile_lines(nq: int, batch: int, NS: int, KBL: int, idx_t: str) -> list[str]:
    """Workgroup -> (``bh``, ``qt``) and, with key splits, the split's first key block
    ``kb0``: the (batch*head, split) pairs are the XCD-grouped "heads" of ``_tile_lines``,
    so the query tiles that share a key range share an XCD's L2."""
    if NS == 1:
        return _tile_lines(nq, batch, idx_t)
    lines = [x.replace(" bh = ", " vh = ") for x in _tile_lines(nq, batch * NS, idx_t)]
    return lines + [f"  const {idx_t} bh = vh / {NS}u;", f"  const unsigned int kb0 = (unsigned int)(vh % {NS}u) * {KBL}u;"]


def gen_attention(k: Kernel, idx: int) -> tuple[str, "Launch"]:  # noqa: F821
    from .hip_kernels import Launch

    q, kk, v = k.inputs
    out = k.outputs[0]
    scale = k.attn["scale"]  # type: ignore[attr-defined]
    layouts = k.attn.get("layouts", ["bhsd"] * 3)  # type: ignore[attr-defined]
    out_layout = k.attn.get("out_layout", "bhsd")  # type: ignore[attr-defined]

    def logical(n: Node, layout: str) -> tuple[tuple, int, int]:
        """(batch dims, rows, row length) of an operand as [.., rows, d]."""
        if layout == "bshd":
            B, S_, H, d = n.shape
            return (B, H), S_, d
        return tuple(n.shape[:-2]), n.shape[-2], n.shape[-1]

    qb_dims, Sq, D = logical(q, layouts[0])
    _, Sk, _ = logical(kk, layouts[1])
    _, _, Dv = logical(v, layouts[2])
    dt = q.dtype
    T = CTYPE[dt]
    batch = math.prod(qb_dims) if qb_dims else 1

    def base_stride(layout: str, rows: int, d: int, n: Node) -> tuple[str, int]:
        """Offset of (batch*head ``bh``)'s [rows, d] matrix and its row stride."""
        if layout == "bshd":
            H = n.shape[2]
            return f"(bh / {H}u) * {rows * H * d}u + (bh % {H}u) * {d}u", H * d
        return f"bh * {rows * d}u", d

    (qoff, qst), (koff, kst) = base_stride(layouts[0], Sq, D, q), base_stride(layouts[1], Sk, D, kk)
    (voff, vst), (ooff, ost) = base_stride(layouts[2], Sk, Dv, v), base_stride(out_layout, Sq, Dv, out)
    NW, QT = attention_layout(batch, Sq, D, Dv)
    assert QT == 1, "one query tile per wave"
    THREADS = NW * 64
    # 8 waves: two groups of 4 a phase apart (ping-pong) over 3 LDS stages
    pingpong = NW == 8
    NST = 3 if pingpong else 2
    BQ = BQ_PER_WAVE * QT * NW
    KB = -(-Sk // BKV)
    nq = -(-Sq // BQ)
    NS = attention_splits(batch * nq, KB, pingpong)
    KBL = KB // NS                              # key blocks per workgroup
    kb0 = "" if NS == 1 else "kb0 + "           # the workgroup's first key block
    DP = D + 8                                  # 16-byte row padding: conflict-free fragment reads
    # V rows: a transposing read touches 8 rows x 64 bytes; a pitch of 32 or 96 (mod 128)
    # elements puts rows r and r+1..r+3 on disjoint bank ranges
    VP = Dv + next(p for p in (0, 32, 64, 96) if (Dv + p) % 128 in (32, 96))
    opvec = "tj_bf16x8" if dt == DType.bf16 else "tj_f16x8"
    mfma = "__builtin_amdgcn_mfma_f32_32x32x16_bf16" if dt == DType.bf16 else "__builtin_amdgcn_mfma_f32_32x32x16_f16"
    KC = BKV * D // 8 // THREADS                  # 16-byte K chunks per lane per block
    VC = BKV * Dv // 8 // THREADS
    assert KC * THREADS * 8 == BKV * D and VC * THREADS * 8 == BKV * Dv
    idx_t = "unsigned long" if batch * max(Sq, Sk) * max(D, Dv) >= 2**31 else "unsigned int"
    assert batch * max(Sq, Sk) * max(D, Dv) < 2**32, "32-bit element offsets"
    ragged = Sk % BKV != 0
    bdims = "x".join(str(d) for d in qb_dims) or "1"
    fname = f"tj{idx}_attention_{bdims}x{Sq}x{Sk}x{D}_{dt.value}_flash"
    cs = scale * 1.4426950408889634            # scores scaled into exp2's domain
    if dt == DType.bf16:
        pack4 = "tj_f2bf2({0}, {1}) | ((unsigned long)tj_f2bf2({2}, {3}) << 32)"
    else:
        pack4 = ("(unsigned long)(tj_f2h({0}) | (tj_f2h({1}) << 16)) | "
                 "((unsigned long)(tj_f2h({2}) | (tj_f2h({3}) << 16)) << 32)")

    # head dim 128, ping-pong: K and V blocks go straight from memory into LDS (DMA)
    dma = (pingpong and D == 128 and Dv == 128 and NS == 1
           and os.environ.get("TENSORJIT_HIP_ATTENTION_DMA", "1") != "0"
           and Sk * kst * 2 < 2**31 and Sk * vst * 2 < 2**31)
    mi16 = dma and mi16_enabled()
    balanced = mi16 and balance_enabled()
    mfma16 = "__builtin_amdgcn_mfma_f32_16x16x32_bf16" if dt == DType.bf16 else "__builtin_amdgcn_mfma_f32_16x16x32_f16"
    if dma:
        NST = 4
        lds_decl = [f"  __shared__ __attribute__((aligned(1024))) char {a}{s}[{BKV * 256}];"
                    for a in ("Ks", "Vs") for s in range(NST)]
    else:
        lds_decl = [f"  __shared__ __attribute__((aligned(16))) {T} Ks[{NST}][{BKV}][{DP}];",
                    f"  __shared__ __attribute__((aligned(16))) {T} Vs[{NST}][{BKV}][{VP}];"]

    def dma_setup_lines() -> list[str]:
        """Wave w (group gq = w / 4) moves rows gq*32 + (w % 4)*8 + q*4 .. +3 (q = 0, 1) of
        every K and V block: one ``buffer_load_dwordx4 ... lds`` writes 1 KiB of LDS, four
        256-byte rows, lane l at byte 16 l.  Rows are not padded; lane l fetches 16-byte
        chunk (l % 16) ^ f(row) of its row, so position p of a stored row holds chunk
        p ^ f(row), f = (row & 15) ^ ((row >> 4) & 1) for K and ((row ^ (row >> 2)) & 3) << 2
        for V.  The offsets (block included) go in the lane's voffset, which the descriptor's
        range checks: rows past the last key read zeros.  Fragment addresses: K row ``col``
        of tile t, chunk 2c + g, sits at (2c + g) ^ f(col) = (g ^ f(col)) ^ 2c; 16 rows in a
        row hold a chunk at 16 distinct positions and 32 rows of one parity too, so a
        fragment read meets no bank twice whether the LDS serves it 8, 16 or 32 lanes at a
        time (the padded layout's property; f = (row >> 1) & 15 held only for 32).  A transposing
        Vᵀ read takes rows 16 ch + 8 s + vr (vr = 4g + (lane % 16) / 4) and chunk 4u + vcl:
        f = ((vr % 4) ^ (2s + g)) << 2, so chunk 4u + vcl sits at ((4u) ^ vsw) + vcl for
        the first read (s = 0) and at that of tile u ^ 2 for the second.  The transposing
        reads are served a half-wave (32 lanes of 8 bytes) at a time over 256 bytes of
        banks: a swizzle that keeps the 4 rows of a half-wave apart only within 512 bytes,
        f = ((row >> 1) & 3) << 2, measured 3.4e7 bank-conflict cycles per launch at
        [4,32,2048,128] against 0 for the padded rows.

        With 16x16x32 MFMAs (``mi16``) the K layout is kept: a fragment read takes K rows
        16t + lane % 16, chunk 4c + lane / 16, at (4c + g16) ^ r16 ^ (t & 1), and 16 rows
        of one parity again hold 16 distinct positions per chunk pair.  A transposing Vᵀ
        read takes rows 32 ch + 16 s + 4 g16 + (lane % 16) / 4 and columns 16 u + 4 (lane % 4)
        .. +3, i.e. 8 rows x 2 chunks per half-wave and 16 rows per wave, so V is stored
        with f = h(row) << 1, h = (row & 7) ^ ((row >> 3) & 1): position 2 (u ^ h) + j for
        chunk 2u + j, distinct over the 8 rows of a half-wave and over the 8 rows of each
        parity in the wave (the 512-byte model)."""
        # V's chunk swizzle follows the transposing reads of the MFMA form
        vsw_row = "((((r & 7u) ^ ((r >> 3) & 1u))) << 1)" if mi16 else "(((r ^ (r >> 2)) & 3u) << 2)"
        dma_lines_ = ["  const unsigned int wv = __builtin_amdgcn_readfirstlane(wave), gq = wv / 4u;",
                      f"  const __amdgpu_buffer_rsrc_t rsK = __builtin_amdgcn_make_buffer_rsrc((void*)Kb, (short)0, {Sk * kst * 2}, 0x00020000);",
                      f"  const __amdgpu_buffer_rsrc_t rsV = __builtin_amdgcn_make_buffer_rsrc((void*)Vb, (short)0, {Sk * vst * 2}, 0x00020000);",
                      "  unsigned int voK[2], voV[2], dmo[2];",
                      "#pragma unroll",
                      "  for (int q = 0; q < 2; ++q) {",
                      "    dmo[q] = (gq * 32u + (wv % 4u) * 8u + (unsigned int)q * 4u) * 256u;",
                      "    const unsigned int r = gq * 32u + (wv % 4u) * 8u + (unsigned int)q * 4u + lane / 16u;",
                      f"    voK[q] = (r * {kst}u + ((lane % 16u) ^ (r & 15u) ^ ((r >> 4) & 1u)) * 8u) * 2u;",
                      f"    voV[q] = (r * {vst}u + ((lane % 16u) ^ {vsw_row}) * 8u) * 2u;",
                      "  }"]
        if mi16:
            return dma_lines_ + [
                "  const unsigned int kx16 = r16 * 256u + ((g16 ^ r16) << 4);",
                "  const unsigned int vr16 = g16 * 4u + (lane % 16u) / 4u, vh16 = (vr16 & 7u) ^ ((vr16 >> 3) & 1u);",
                f"  unsigned int va16[{Dv // 16}];",
                "#pragma unroll",
                f"  for (int u = 0; u < {Dv // 16}; ++u)",
                "    va16[u] = vr16 * 256u + (((((unsigned int)u ^ vh16) << 1) | ((lane % 4u) >> 1)) << 4) + (lane % 2u) * 8u;"]
        return dma_lines_ + [
                "  const unsigned int kx = col * 256u + ((g ^ (col & 15u) ^ ((col >> 4) & 1u)) << 4);",
                "  const unsigned int vr = g * 4u + (lane % 16u) / 4u, vsw = (((lane % 16u) / 4u) ^ g) << 2;",
                "  const unsigned int vcl = ((lane / 16u) % 2u) * 2u + (lane % 4u) / 2u;",
                "  unsigned int va[4];",
                "#pragma unroll",
                "  for (int u = 0; u < 4; ++u)",
                "    va[u] = vr * 256u + (lane % 2u) * 8u + ((((unsigned int)u * 4u) ^ vsw) + vcl) * 16u;"]

    def dma_lines(which: str, blk: str, stage: int) -> list[str]:
        """This wave's two DMA loads of key block ``blk`` (K or V) into ``stage``."""
        rs, vo, st = ("rsK", "voK", kst) if which == "k" else ("rsV", "voV", vst)
        arr = "Ks" if which == "k" else "Vs"
        return [f"__builtin_amdgcn_raw_ptr_buffer_load_lds({rs}, (__attribute__((address_space(3))) void*)"
                f"({arr}{stage} + dmo[{q}]), 16, {vo}[{q}] + ({blk}) * {BKV * st * 2}u, 0, 0, 0);" for q in range(2)]

    # two waves per SIMD: one wave's softmax arithmetic runs under the other's MFMAs;
    # the compiler then keeps everything in 256 VGPRs
    occ = 2
    # the two halves of a query's keys (lanes l and l ^ 32) combine through the prelude's
    # tj_pair_max / tj_pair_sum (v_permlane32_swap), shared by every attention kernel of a program
    L = [f'extern "C" __global__ void __launch_bounds__({THREADS}) __attribute__((amdgpu_waves_per_eu({occ}, {occ}))) {fname}(',
         f"    const {T}* __restrict__ in0_p, const {T}* __restrict__ in1_p, const {T}* __restrict__ in2_p,",
         f"    {T}* __restrict__ out0_p{', float* __restrict__ ws_p' if NS > 1 else ''}) {{",
         *lds_decl,
         "  const unsigned int tid = threadIdx.x, lane = tid % 64u, wave = tid / 64u;",
         "  const unsigned int g = lane / 32u, col = lane % 32u;",
         *_split_tile_lines(nq, batch, NS, KBL, idx_t),
         f"  const {T}* __restrict__ Qb = in0_p + ({qoff});",
         f"  const {T}* __restrict__ Kb = in1_p + ({koff});",
         f"  const {T}* __restrict__ Vb = in2_p + ({voff});",
         f"  {T}* __restrict__ Ob = out0_p + ({ooff});"]
    if mi16:
        # 16x16x32: query tile h of this wave is rows qrow0 + h*16 (lane column lane % 16);
        # Q as the B operand of S^T = K Q^T: chunk c holds Q[row][c*32 + g16*8 .. +8]
        L += ["  const unsigned int r16 = lane % 16u, g16 = lane / 16u;",
              f"  const unsigned int qrow0 = qt * {BQ}u + wave * 32u + r16;",
              f"  {opvec} qf[2][{D // 32}];",
              f"  tj_f32x4 o[2][{Dv // 16}];",
              "  float m_run[2], l_run[2];",
              *(["  float mbn[2];"] if balanced else []),
              "#pragma unroll",
              "  for (int h = 0; h < 2; ++h) {",
              f"    const unsigned int qc = qrow0 + h * 16u < {Sq}u ? qrow0 + h * 16u : {Sq - 1}u;",
              "#pragma unroll",
              f"    for (int c = 0; c < {D // 32}; ++c) qf[h][c] = *(const {opvec}*)&Qb[qc * {qst}u + c * 32 + g16 * 8u];",
              "#pragma unroll",
              f"    for (int u = 0; u < {Dv // 16}; ++u) o[h][u] = (tj_f32x4)(0.0f);",
              "    m_run[h] = -__builtin_inff();",
              "    l_run[h] = 0.0f;",
              "  }"]
    else:
        L += [
         # query tile q of this wave: rows qrow0 + q*32 .. +31, one per lane column
         f"  const unsigned int qrow0 = qt * {BQ}u + wave * {32 * QT}u + col;",
         # Q as the B operand of S^T = K Q^T: chunk c holds Q[row][c*16 + g*8 .. +8]
         f"  {opvec} qf[{QT}][{D // 16}];",
         f"  tj_f32x16 o[{QT}][{Dv // 32}];",
         f"  float m_run[{QT}], l_run[{QT}];",
         "#pragma unroll",
         f"  for (int q = 0; q < {QT}; ++q) {{",
         f"    const unsigned int qc = qrow0 + q * 32u < {Sq}u ? qrow0 + q * 32u : {Sq - 1}u;",
         "#pragma unroll",
         f"    for (int c = 0; c < {D // 16}; ++c) qf[q][c] = *(const {opvec}*)&Qb[qc * {qst}u + c * 16 + g * 8u];",
         "#pragma unroll",
         f"    for (int u = 0; u < {Dv // 32}; ++u) o[q][u] = (tj_f32x16)(0.0f);",
         "    m_run[q] = -__builtin_inff();",
         "    l_run[q] = 0.0f;",
         "  }"]
    if dma:
        L += dma_setup_lines()
    else:
        L.append(f"  tj_u32x4 rk[{KC}], rv[{VC}];")
        if PV_AHEAD_STAGED:
            L.append("  const unsigned int vrow0 = g * 4u + (lane % 16u) / 4u, vcol0 = ((lane / 16u) % 2u) * 16u + (lane % 4u) * 4u;")
    if pingpong and not dma:
        L.append("  const unsigned int gq = wave / 4u, gtid = tid % 256u;")

    def k_load(blk: str) -> list[str]:
        out_l = ["#pragma unroll", f"for (int i = 0; i < {KC}; ++i) {{",
                 f"  const unsigned int c = i * {THREADS}u + tid, row = c / {D // 8}u, d8 = (c % {D // 8}u) * 8u;",
                 f"  unsigned int key = ({kb0}{blk}) * {BKV}u + row;"]
        if ragged:
            out_l.append(f"  key = key < {Sk}u ? key : {Sk - 1}u;")
        return out_l + [f"  rk[i] = *(const tj_u32x4*)&Kb[key * {kst}u + d8];", "}"]

    def v_load(blk: str) -> list[str]:
        out_l = ["#pragma unroll", f"for (int i = 0; i < {VC}; ++i) {{",
                 f"  const unsigned int c = i * {THREADS}u + tid, row = c / {Dv // 8}u, d8 = (c % {Dv // 8}u) * 8u;",
                 f"  unsigned int key = ({kb0}{blk}) * {BKV}u + row;"]
        if ragged:
            out_l.append(f"  key = key < {Sk}u ? key : {Sk - 1}u;")
        return out_l + [f"  rv[i] = *(const tj_u32x4*)&Vb[key * {vst}u + d8];", "}"]

    def half_load(which: str, blk: str) -> list[str]:
        """This group's half (keys gq*32 .. +31) of a K or V block into rk / rv; the block
        index is clamped so the loads past the last block stay in bounds (unused)."""
        d, reg, base, st = (D, "rk", "Kb", kst) if which == "k" else (Dv, "rv", "Vb", vst)
        n = (BKV // 2) * d // 8 // 256
        out_l = ["#pragma unroll", f"for (int i = 0; i < {n}; ++i) {{",
                 f"  const unsigned int c = i * 256u + gtid, row = gq * {BKV // 2}u + c / {d // 8}u, d8 = (c % {d // 8}u) * 8u;",
                 f"  const unsigned int b_ = ({blk}) < {KB}u ? ({blk}) : {KB - 1}u;",
                 f"  unsigned int key = b_ * {BKV}u + row;"]
        if ragged:
            out_l.append(f"  key = key < {Sk}u ? key : {Sk - 1}u;")
        return out_l + [f"  {reg}[i] = *(const tj_u32x4*)&{base}[key * {st}u + d8];", "}"]

    def half_store(which: str, stage: str) -> list[str]:
        d, reg, arr = (D, "rk", "Ks") if which == "k" else (Dv, "rv", "Vs")
        n = (BKV // 2) * d // 8 // 256
        return ["#pragma unroll", f"for (int i = 0; i < {n}; ++i) {{",
                f"  const unsigned int c = i * 256u + gtid, row = gq * {BKV // 2}u + c / {d // 8}u, d8 = (c % {d // 8}u) * 8u;",
                f"  *(tj_u32x4*)&{arr}[{stage}][row][d8] = {reg}[i];", "}"]

    def k_store(stage: int) -> list[str]:
        return ["#pragma unroll", f"for (int i = 0; i < {KC}; ++i) {{",
                f"  const unsigned int c = i * {THREADS}u + tid, row = c / {D // 8}u, d8 = (c % {D // 8}u) * 8u;",
                f"  *(tj_u32x4*)&Ks[{stage}][row][d8] = rk[i];", "}"]

    def v_store(stage: int) -> list[str]:
        return ["#pragma unroll", f"for (int i = 0; i < {VC}; ++i) {{",
                f"  const unsigned int c = i * {THREADS}u + tid, row = c / {Dv // 8}u, d8 = (c % {Dv // 8}u) * 8u;",
                f"  *(tj_u32x4*)&Vs[{stage}][row][d8] = rv[i];", "}"]

    def scores(dst: str, stage: int) -> list[str]:
        """S^T = K Q^T over D in 16-wide chunks: tile t covers keys t*32 .. t*32+31."""
        if mi16:
            return scores16(dst, stage, KS_AHEAD16)
        ks_ahead = KS_AHEAD if dma else KS_AHEAD_STAGED if D >= 128 else 0
        if ks_ahead:
            return scores_pipelined(dst, stage, ks_ahead)
        return ["#pragma unroll", f"for (int q = 0; q < {QT}; ++q)", "#pragma unroll",
                f"  for (int t = 0; t < {BKV // 32}; ++t) {dst}[q][t] = (tj_f32x16)(0.0f);",
                "#pragma unroll", f"for (int c = 0; c < {D // 16}; ++c) {{", "#pragma unroll",
                f"  for (int t = 0; t < {BKV // 32}; ++t) {{",
                f"    const {opvec} kf = *(const {opvec}*)(Ks{stage} + t * {32 * 256}u + (kx ^ (c * 32u)));" if dma else
                f"    const {opvec} kf = *(const {opvec}*)&Ks[{stage}][t * 32 + col][c * 16 + g * 8u];",
                "#pragma unroll",
                f"    for (int q = 0; q < {QT}; ++q) {dst}[q][t] = {mfma}(kf, qf[q][c], {dst}[q][t], 0, 0, 0);",
                "  }", "}"]

    # online softmax, one query column per lane (its 32 keys here + lane ^ 32's 32).
    # The extreme is taken on the raw scores (max(s*cs) = cs*max(s) for cs > 0, min for
    # cs < 0) so the scale folds into the exponent's FMA.  Lazy rescaling: the running
    # reference max moves only when some lane's own block max exceeds it by more than 8
    # (exponents then stay <= 2^8); otherwise the output accumulator is left alone, and
    # no lane exchanges anything.  Only then are the two halves of a query's keys
    # combined (lane ^ 32, one v_permlane32_swap), so both lanes of a query keep the
    # same reference; each lane sums its own half of the row sum, combined once at the
    # end.
    ext, ext_init, masked = ("fmaxf", "-__builtin_inff()", "-__builtin_inff()") if cs > 0 else \
        ("fminf", "__builtin_inff()", "__builtin_inff()")

    def block_max(sc: str, j: int | None, pre: bool = False) -> list[str]:
        if mi16:
            return block_max16(sc, j, pre)
        mask = None
        if ragged and j == KBL - 1:
            mask = f"{j * BKV}" if NS == 1 else f"(int)kb0 * {BKV} + {j * BKV}"
        elif ragged and j is None and pingpong:
            mask = "(int)jj"
            mask = f"{mask} * {BKV}"
        out_l = [f"float mb[{QT}];", "bool grow = false;", "#pragma unroll", f"for (int q = 0; q < {QT}; ++q) {{",
                 f"  float mx = {ext_init};", "#pragma unroll", f"  for (int t = 0; t < {BKV // 32}; ++t)",
                 "#pragma unroll", "    for (int r = 0; r < 16; ++r) {"]
        if mask is not None:
            out_l.append(f"      if ({mask} + t * 32 + (r / 4) * 8 + (int)g * 4 + r % 4 >= {Sk}) {sc}[q][t][r] = {masked};")
        out_l += [f"      mx = {ext}(mx, {sc}[q][t][r]);", "    }",
                  f"  mb[q] = mx * {cs!r}f;",
                  "  grow = grow || mb[q] > m_run[q] + 8.0f;",
                  "}",
                  "if (__builtin_amdgcn_ballot_w64(grow)) {",
                  "#pragma unroll",
                  f"  for (int q = 0; q < {QT}; ++q) {{",
                  "    const float m_new = fmaxf(m_run[q], tj_pair_max(mb[q]));",
                  "    const float alpha = __builtin_amdgcn_exp2f(m_run[q] - m_new);",
                  "    l_run[q] *= alpha;",
                  "#pragma unroll",
                  f"    for (int u = 0; u < {Dv // 32}; ++u) o[q][u] *= alpha;",
                  "    m_run[q] = m_new;",
                  "  }",
                  "}"]
        return out_l

    def probs(sc: str) -> list[str]:
        """exp2 of the block's scores, the running sums, and the P^T operands (chunk 2t+h)."""
        cvt = ("tj_f2bf2({0}, {1})" if dt == DType.bf16 else "tj_f2h({0}) | (tj_f2h({1}) << 16)")
        if mi16:
            return probs16(sc, cvt, not balanced)
        return ["#pragma unroll", f"for (int q = 0; q < {QT}; ++q) {{",
                "  float rs = 0.0f;", "#pragma unroll", f"  for (int t = 0; t < {BKV // 32}; ++t)",
                "#pragma unroll", "    for (int h = 0; h < 2; ++h) {",
                "      tj_u32x4 pw;", "#pragma unroll", "      for (int w = 0; w < 4; ++w) {",
                f"        const float e0 = __builtin_amdgcn_exp2f(__builtin_fmaf({sc}[q][t][8 * h + 2 * w], {cs!r}f, -m_run[q]));",
                f"        const float e1 = __builtin_amdgcn_exp2f(__builtin_fmaf({sc}[q][t][8 * h + 2 * w + 1], {cs!r}f, -m_run[q]));",
                "        rs += e0 + e1;",
                "        pw[w] = " + cvt.format("e0", "e1") + ";",
                "      }",
                f"      pf[q][2 * t + h] = __builtin_bit_cast({opvec}, pw);",
                "    }",
                "  l_run[q] += rs;",
                "}"]

    def pv(stage: int, extra: list[str] | None = None) -> list[str]:
        """O^T += V^T P^T.  The V^T fragment of chunk ch holds keys ch*16 + g*4 + 0..3 then
        ch*16 + 8 + g*4 + 0..3 (the score accumulator's order) for d = u*32 + lane % 32,
        gathered by two transposing reads of V's natural rows.  ``extra``: independent
        code of the 16x16x32 form scheduled among the MFMAs."""
        if mi16:
            return pv16(stage, PV_AHEAD16, extra or [])
        if (PV_AHEAD if dma else PV_AHEAD_STAGED):
            return pv_pipelined(stage, PV_AHEAD if dma else PV_AHEAD_STAGED)
        if dma:
            rd = "__builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) tj_i16x4*)"
            return ["#pragma unroll", f"for (int ch = 0; ch < {BKV // 16}; ++ch) {{",
                    "#pragma unroll", f"  for (int u = 0; u < {Dv // 32}; ++u) {{",
                    f"    tj_i16x4 v0 = {rd}(Vs{stage} + ch * 4096u + va[u]));",
                    f"    tj_i16x4 v1 = {rd}(Vs{stage} + ch * 4096u + 2048u + va[u ^ 2]));",
                    f"    const {opvec} vv = __builtin_bit_cast({opvec}, __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7));",
                    "#pragma unroll",
                    f"    for (int q = 0; q < {QT}; ++q) o[q][u] = {mfma}(vv, pf[q][ch], o[q][u], 0, 0, 0);",
                    "  }", "}"]
        return ["#pragma unroll", f"for (int ch = 0; ch < {BKV // 16}; ++ch) {{",
                "  const unsigned int vrow = ch * 16 + g * 4u + (lane % 16u) / 4u;",
                "#pragma unroll", f"  for (int u = 0; u < {Dv // 32}; ++u) {{",
                "    const unsigned int vcol = u * 32 + ((lane / 16u) % 2u) * 16u + (lane % 4u) * 4u;",
                f"    tj_i16x4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) tj_i16x4*)&Vs[{stage}][vrow][vcol]);",
                f"    tj_i16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) tj_i16x4*)&Vs[{stage}][vrow + 8u][vcol]);",
                f"    const {opvec} vv = __builtin_bit_cast({opvec}, __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7));",
                "#pragma unroll",
                f"    for (int q = 0; q < {QT}; ++q) o[q][u] = {mfma}(vv, pf[q][ch], o[q][u], 0, 0, 0);",
                "  }", "}"]

    def iteration(j: str, jc: int | None, par: int, has_next: bool, store_k: bool, store_v: bool,
                  load_k: bool, load_v: bool) -> list[str]:
        """Block j: the softmax of S(j) runs while the MFMAs of S(j+1) are in flight,
        then O += P(j) V(j); K(j+2) and V(j+1) move from registers to LDS and the loads
        of K(j+3), V(j+2) are issued.  LDS: Ks[(j+1)%2] = K(j+1), Vs[j%2] = V(j)."""
        sc, sn = ("sA", "sB") if par == 0 else ("sB", "sA")
        out_l = block_max(sc, jc)
        if has_next:
            out_l += scores(sn, 1 - par)
        out_l += probs(sc)
        out_l += pv(par)
        if store_k:
            out_l += k_store(par)
        if store_v:
            out_l += v_store(1 - par)
        if load_k:
            out_l += k_load(f"({j}) + 3u")
        if load_v:
            out_l += v_load(f"({j}) + 2u")
        out_l.append("__syncthreads();")
        return out_l

    def double_buffer_body() -> list[str]:
        """All waves in step; one barrier per block (2 LDS stages)."""
        out = []
        # prologue: K(0), K(1), V(0) into LDS, S(0), then K(2) and V(1) into registers
        out += ["  " + x for x in k_load("0u") + k_store(0)]
        if KBL > 1:
            out += ["  " + x for x in k_load("1u") + k_store(1)]
        out += ["  " + x for x in v_load("0u") + v_store(0)]
        out.append("  __syncthreads();")
        out += ["  " + x for x in scores("sA", 0)]
        out.append("  __syncthreads();   // every wave has read Ks[0] before K(2) replaces it")
        if KBL > 2:
            out += ["  " + x for x in k_load("2u")]
        if KBL > 1:
            out += ["  " + x for x in v_load("1u")]
        # blocks 0 .. KBL-4 have every step; run them in even/odd pairs, then peel the rest
        npair = max(0, KBL - 3) // 2
        if npair:
            out.append(f"  for (unsigned int j = 0; j < {2 * npair}u; j += 2u) {{")
            out += ["    {"] + ["      " + x for x in iteration("j", None, 0, True, True, True, True, True)] + ["    }"]
            out += ["    {"] + ["      " + x for x in iteration("j + 1u", None, 1, True, True, True, True, True)] + ["    }"]
            out.append("  }")
        for j in range(2 * npair, KBL):
            out.append(f"  {{  // block {j}")
            out += ["    " + x for x in iteration(f"{j}u", j, j % 2, j + 1 < KBL, j + 2 < KBL, j + 1 < KBL, j + 3 < KBL,
                                                  j + 2 < KBL)]
            out.append("  }")
        return out

    def pp_iteration(jj: str, par: int, has_next: bool = True) -> list[str]:
        """One block for one wave group, as two phases separated by workgroup barriers.
        Phase A: softmax of S(j) with the MFMAs of S(j+1) (K(j+1) in stage (j+1)%3).
        Phase B: O += P(j) V(j) (stage j%3); this group's halves of K(j+3) and V(j+1) go
        to LDS, the loads of K(j+4) and V(j+2) are issued.  The other group runs the
        opposite phase meanwhile.  With group 1 one phase behind, a K block is written
        (phases 2j+1 and 2j+2) two phases before its first read (2j+4) and a V block
        (same phases) one phase before (2j+3); the stages they overwrite were last read
        in phase 2j-1 (K) and 2j-2 (V).  ``has_next``: S(j+1) exists (the last block
        skips it; the barriers stay, so the groups keep their phase offset)."""
        sc, sn = ("sA", "sB") if par == 0 else ("sB", "sA")
        out = block_max(sc, None)
        if has_next:
            out += scores(sn, f"(({jj}) + 1u) % 3u")
        out += probs(sc)
        out += ["__syncthreads();"]
        out += pv(f"({jj}) % 3u")
        # stores past the last block write stages no later block reads; loads are clamped
        out += half_store("k", f"({jj}) % 3u") + half_store("v", f"(({jj}) + 1u) % 3u")
        out += half_load("k", f"({jj}) + 4u") + half_load("v", f"({jj}) + 2u")
        out.append("__syncthreads();")
        return out

    def pingpong_body() -> list[str]:
        out = []
        # prologue (all waves): K(0..2), V(0) into LDS, S(0); then this group's halves
        # of K(3) and V(1) into registers; group 1 waits one extra barrier
        for b in range(min(3, KB)):
            out += ["  " + x for x in k_load(f"{b}u") + k_store(b)]
        out += ["  " + x for x in v_load("0u") + v_store(0)]
        out.append("  __syncthreads();")
        out += ["  " + x for x in scores("sA", 0)]
        out += ["  " + x for x in half_load("k", "3u") + half_load("v", "1u")]
        out.append("  if (gq == 1u) __syncthreads();")
        # pairs of blocks that all have a next block, then the last one or two peeled
        npair = (KB - 1) // 2
        if npair:
            out.append(f"  for (unsigned int jj = 0; jj < {2 * npair}u; jj += 2u) {{")
            out += ["    {"] + ["      " + x for x in pp_iteration("jj", 0)] + ["    }"]
            out += ["    {"] + ["      const unsigned int jj1 = jj + 1u;"] + \
                   ["      " + x.replace("(int)jj *", "(int)jj1 *") for x in pp_iteration("jj1", 1)] + ["    }"]
            out.append("  }")
        for j in range(2 * npair, KB):
            out.append(f"  {{  const unsigned int jj = {j}u;")
            out += ["    " + x for x in pp_iteration("jj", j % 2, j + 1 < KB)]
            out.append("  }")
        out.append("  if (gq == 0u) __syncthreads();")
        return out

    def scores_pipelined(dst: str, stage: int, ahead: int) -> list[str]:
        """The score MFMAs with the K fragment read of MFMA p + ``ahead`` issued after MFMA p
        (fragments in (c, t) order), pinned by ``sched_group_barrier``."""
        assert QT == 1
        n = (D // 16) * (BKV // 32)

        def read(p: int) -> str:
            c, t = divmod(p, BKV // 32)
            if dma:
                return f"const {opvec} kt{p} = *(const {opvec}*)(Ks{stage} + {t * 32 * 256}u + (kx ^ {c * 32}u));"
            return f"const {opvec} kt{p} = *(const {opvec}*)&Ks[{stage}][{t * 32}u + col][{c * 16}u + g * 8u];"

        out = [f"{dst}[0][{t}] = (tj_f32x16)(0.0f);" for t in range(BKV // 32)]
        out.append("{")
        sg = [f"__builtin_amdgcn_sched_group_barrier({SG_DS_READ}, {min(ahead, n)}, 0);"]
        out += [read(p) for p in range(min(ahead, n))]
        for p in range(n):
            c, t = divmod(p, BKV // 32)
            out.append(f"{dst}[0][{t}] = {mfma}(kt{p}, qf[0][{c}], {dst}[0][{t}], 0, 0, 0);")
            sg.append(f"__builtin_amdgcn_sched_group_barrier({SG_MFMA}, 1, 0);")
            if p + ahead < n:
                out.append(read(p + ahead))
                sg.append(f"__builtin_amdgcn_sched_group_barrier({SG_DS_READ}, 1, 0);")
        return out + sg + ["}"]

    def pv_pipelined(stage: int, ahead: int) -> list[str]:
        """The PV phase with the transposing reads of fragment p + ``ahead`` issued after the
        MFMA of fragment p (fragments in (ch, u) order), pinned by ``sched_group_barrier``;
        the score accumulator that PV follows is dead by then, so its registers hold them."""
        assert QT == 1
        rd = "__builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) tj_i16x4*)"
        n = (BKV // 16) * (Dv // 32)

        def reads(p: int) -> list[str]:
            ch, u = divmod(p, Dv // 32)
            if dma:
                return [f"const tj_i16x4 vt{p}a = {rd}(Vs{stage} + {ch * 4096}u + va[{u}]));",
                        f"const tj_i16x4 vt{p}b = {rd}(Vs{stage} + {ch * 4096 + 2048}u + va[{u ^ 2}]));"]
            return [f"const tj_i16x4 vt{p}{h} = {rd}&Vs[{stage}][{ch * 16 + 8 * i}u + vrow0][{u * 32}u + vcol0]);"
                    for i, h in enumerate("ab")]

        out, sg = ["{"], [f"__builtin_amdgcn_sched_group_barrier({SG_DS_READ}, {2 * min(ahead, n)}, 0);"]
        for p in range(min(ahead, n)):
            out += reads(p)
        for p in range(n):
            ch, u = divmod(p, Dv // 32)
            out.append(f"o[0][{u}] = {mfma}(__builtin_bit_cast({opvec}, __builtin_shufflevector(vt{p}a, vt{p}b, "
                       f"0, 1, 2, 3, 4, 5, 6, 7)), pf[0][{ch}], o[0][{u}], 0, 0, 0);")
            sg.append(f"__builtin_amdgcn_sched_group_barrier({SG_MFMA}, 1, 0);")
            if p + ahead < n:
                out += reads(p + ahead)
                sg.append(f"__builtin_amdgcn_sched_group_barrier({SG_DS_READ}, 2, 0);")
        return out + sg + ["}"]

    # --- 16x16x32 forms (DMA schedule): S[h][t] is the 16 x 16 score tile of keys 16t ..
    # 16t+15 and queries 16h .. 16h+15 of the wave; lane l holds keys 16t + 4 (l / 16) + i
    # (i = 0..3) of query column l % 16, so a query's 64 keys of a block sit on lanes
    # l % 16 + 16 g, g = 0..3, 16 per lane.  P^T chunk ch (keys 32ch .. 32ch+31) is the lane's
    # own S[h][2ch] and S[h][2ch+1]: MFMA k index 8g + m stands for key 32ch + 16(m / 4) + 4g
    # + m % 4, and the Vᵀ fragment is read in that key order.

    def scores16(dst: str, stage: int, ahead: int) -> list[str]:
        """S^T = K Q^T with 16x16x32 MFMAs: the K fragment of (d chunk c, key tile t) feeds
        both query tiles; the read of fragment p + ``ahead`` is issued after fragment p's
        two MFMAs (fragments in (c, t) order), pinned by ``sched_group_barrier``."""
        nt = BKV // 16
        n = (D // 32) * nt

        def read(p: int) -> str:
            c, t = divmod(p, nt)
            return f"const {opvec} kt{p} = *(const {opvec}*)(Ks{stage} + {t * 4096}u + (kx16 ^ {((4 * c) ^ (t & 1)) << 4}u));"

        out = [f"{dst}[{h}][{t}] = (tj_f32x4)(0.0f);" for h in range(2) for t in range(nt)]
        out.append("{")
        sg = [f"__builtin_amdgcn_sched_group_barrier({SG_DS_READ}, {min(ahead, n)}, 0);"]
        out += [read(p) for p in range(min(ahead, n))]
        for p in range(n):
            c, t = divmod(p, nt)
            out += [f"{dst}[{h}][{t}] = {mfma16}(kt{p}, qf[{h}][{c}], {dst}[{h}][{t}], 0, 0, 0);" for h in range(2)]
            sg.append(f"__builtin_amdgcn_sched_group_barrier({SG_MFMA}, 2, 0);")
            if p + ahead < n:
                out.append(read(p + ahead))
                sg.append(f"__builtin_amdgcn_sched_group_barrier({SG_DS_READ}, 1, 0);")
        return out + sg + ["}"]

    def lane_max16(sc: str, j: int | None, dst: str) -> list[str]:
        """The lane's own extremes of block ``j``'s scores (16 keys per query tile), scaled
        into exp2's domain, into ``dst``; keys past Sk in a ragged last block are masked."""
        mask = f"{j * BKV}" if ragged and j == KBL - 1 else None
        out_l = ["#pragma unroll", "for (int h = 0; h < 2; ++h) {",
                 f"  float mx = {ext_init};", "#pragma unroll", f"  for (int t = 0; t < {BKV // 16}; ++t)",
                 "#pragma unroll", "    for (int i = 0; i < 4; ++i) {"]
        if mask is not None:
            out_l.append(f"      if ({mask} + t * 16 + (int)g16 * 4 + i >= {Sk}) {sc}[h][t][i] = {masked};")
        return out_l + [f"      mx = {ext}(mx, {sc}[h][t][i]);", "    }", f"  {dst}[h] = mx * {cs!r}f;", "}"]

    def block_max16(sc: str, j: int | None, pre: bool) -> list[str]:
        """The lane's own block extremes (16 keys per query), lazy rescale as in the 32x32
        form; a rescale combines the four lanes of a query (``tj_quad_max``).  With ``pre``
        the extremes were taken in the previous phase (``mbn``)."""
        out_l = ["float mb[2];", "bool grow = false;"]
        out_l += ["mb[0] = mbn[0];", "mb[1] = mbn[1];"] if pre else lane_max16(sc, j, "mb")
        return out_l + ["#pragma unroll", "for (int h = 0; h < 2; ++h)",
                        "  grow = grow || mb[h] > m_run[h] + 8.0f;",
                        "if (__builtin_amdgcn_ballot_w64(grow)) {",
                        "#pragma unroll",
                        "  for (int h = 0; h < 2; ++h) {",
                        "    const float m_new = fmaxf(m_run[h], tj_quad_max(mb[h]));",
                        "    const float alpha = __builtin_amdgcn_exp2f(m_run[h] - m_new);",
                        "    l_run[h] *= alpha;",
                        "#pragma unroll",
                        f"    for (int u = 0; u < {Dv // 16}; ++u) o[h][u] *= alpha;",
                        "    m_run[h] = m_new;",
                        "  }",
                        "}"]

    def probs16(sc: str, cvt: str, with_sum: bool) -> list[str]:
        """exp2 of the block's scores, the running sums (``with_sum``), and P^T chunk ch of
        each query tile from the lane's own S[h][2ch] (k 0..3 of its group) and
        S[h][2ch+1] (k 4..7)."""
        return ["#pragma unroll", "for (int h = 0; h < 2; ++h) {",
                "  float rs = 0.0f;", "#pragma unroll", f"  for (int ch = 0; ch < {BKV // 32}; ++ch) {{",
                "    tj_u32x4 pw;", "#pragma unroll", "    for (int s = 0; s < 2; ++s)",
                "#pragma unroll", "      for (int w = 0; w < 2; ++w) {",
                f"        const float e0 = __builtin_amdgcn_exp2f(__builtin_fmaf({sc}[h][2 * ch + s][2 * w], {cs!r}f, -m_run[h]));",
                f"        const float e1 = __builtin_amdgcn_exp2f(__builtin_fmaf({sc}[h][2 * ch + s][2 * w + 1], {cs!r}f, -m_run[h]));",
                *(["        rs += e0 + e1;"] if with_sum else []),
                "        pw[2 * s + w] = " + cvt.format("e0", "e1") + ";",
                "      }",
                f"    pf[h][ch] = __builtin_bit_cast({opvec}, pw);",
                "  }",
                *(["  l_run[h] += rs;"] if with_sum else []),
                "}"]

    def rowsum16() -> list[str]:
        """The running sums from the 16-bit probabilities the PV MFMAs take (two per
        v_dot2 with ones), so the sum and the weights of O are the same numbers."""
        acc = "tj_pair_acc_bf16" if dt == DType.bf16 else "tj_pair_acc_f16"
        return ["#pragma unroll", "for (int h = 0; h < 2; ++h) {", "  float rs = 0.0f;",
                "#pragma unroll", f"  for (int ch = 0; ch < {BKV // 32}; ++ch) {{",
                f"    const tj_u32x4 pw = __builtin_bit_cast(tj_u32x4, pf[h][ch]);",
                "#pragma unroll", f"    for (int w = 0; w < 4; ++w) rs = {acc}(pw[w], rs);",
                "  }", "  l_run[h] += rs;", "}"]

    def pv16(stage: int, ahead: int, extra: list[str]) -> list[str]:
        """O^T += V^T P^T with 16x16x32 MFMAs: the Vᵀ fragment of (key chunk ch, dv tile u)
        holds dv 16u + lane % 16 and keys 32ch + 4 g16 + 0..3 (first read) then 32ch + 16 +
        4 g16 + 0..3 (second), and feeds both query tiles; reads of fragment p + ``ahead``
        after fragment p's MFMAs, fragments in (ch, u) order.  ``extra`` (code independent
        of the MFMAs) is placed before the scheduling groups, inside the same region."""
        rd = "__builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) tj_i16x4*)"
        nu = Dv // 16
        n = (BKV // 32) * nu

        def reads(p: int) -> list[str]:
            ch, u = divmod(p, nu)
            return [f"const tj_i16x4 vt{p}a = {rd}(Vs{stage} + {ch * 8192}u + va16[{u}]));",
                    f"const tj_i16x4 vt{p}b = {rd}(Vs{stage} + {ch * 8192 + 4096}u + va16[{u}]));"]

        out, sg = ["{"], [f"__builtin_amdgcn_sched_group_barrier({SG_DS_READ}, {2 * min(ahead, n)}, 0);"]
        for p in range(min(ahead, n)):
            out += reads(p)
        for p in range(n):
            ch, u = divmod(p, nu)
            out.append(f"const {opvec} vv{p} = __builtin_bit_cast({opvec}, __builtin_shufflevector(vt{p}a, vt{p}b, "
                       "0, 1, 2, 3, 4, 5, 6, 7));")
            out += [f"o[{h}][{u}] = {mfma16}(vv{p}, pf[{h}][{ch}], o[{h}][{u}], 0, 0, 0);" for h in range(2)]
            sg.append(f"__builtin_amdgcn_sched_group_barrier({SG_MFMA}, 2, 0);")
            if p + ahead < n:
                out += reads(p + ahead)
                sg.append(f"__builtin_amdgcn_sched_group_barrier({SG_DS_READ}, 2, 0);")
        return out + extra + sg + ["}"]

    def epilogue16_lines() -> list[str]:
        # O = O^T / l: lane holds dv 16u + 4 g16 + 0..3 of query 16h + lane % 16
        return ["#pragma unroll", "  for (int h = 0; h < 2; ++h) {",
                "    const unsigned int qrow = qrow0 + h * 16u;",
                "    const float l_tot = tj_quad_sum(l_run[h]);",
                f"    if (qrow < {Sq}u) {{",
                "      const float inv = 1.0f / l_tot;",
                "#pragma unroll",
                f"      for (int u = 0; u < {Dv // 16}; ++u) {{",
                "        const unsigned int dv = u * 16 + g16 * 4u;",
                "        *(unsigned long*)&Ob[qrow * " + f"{ost}u + dv] = "
                + pack4.format("o[h][u][0] * inv", "o[h][u][1] * inv", "o[h][u][2] * inv", "o[h][u][3] * inv") + ";",
                "      }",
                "    }",
                "  }",
                "}"]

    def phase_end(vm: int | None) -> list[str]:
        """End of a ping-pong phase in the DMA schedule: this wave's fragment reads are done
        and, with ``vm``, all but its ``vm`` youngest DMA loads have landed; then the
        workgroup barrier.  A plain ``s_barrier``: __syncthreads' workgroup fence would
        wait for every DMA load in flight."""
        imm = 0xC07F if vm is None else (vm & 15) | ((vm >> 4) << 14) | 0x70
        return ["__builtin_amdgcn_sched_barrier(0);", f"__builtin_amdgcn_s_waitcnt({hex(imm)});",
                "__builtin_amdgcn_s_barrier();", "__builtin_amdgcn_sched_barrier(0);"]

    def n_dma(x: int) -> int:
        """DMA loads a wave issues in phase B of block x: V(x+3) and K(x+4), two each."""
        return 2 * (x + 3 < KB) + 2 * (x + 4 < KB)

    def dma_block(j: str, jc: int, s: int, vm: int) -> list[str]:
        """Block ``jc`` (-1: a loop block, never the last) in stage s = j % 4 for one wave group.
        Phase A: softmax of S(j) with the MFMAs of S(j+1) (K(j+1), stage (s+1)%4); at its
        end the DMA loads of phase B(j-2) have landed (``vm``: those of B(j-1) may not).
        Phase B: V(j+3) into stage (s+3)%4 and K(j+4) into stage s are issued, then
        O += P(j) V(j).  With group 1 one phase behind group 0 (group 0 runs A(j) in phase
        2j, B(j) in 2j+1), the stage V(j+3) overwrites was last read in phase 2j (V(j-1)) and
        the one of K(j+4) in 2j-1 (K(j)), before either group issues into it (2j+1, 2j+2);
        loads of B(j) land by A(j+2) (phases 2j+4 and 2j+5), before the first read of
        K(j+4) (2j+6) and of V(j+3) (2j+7)."""
        par = (jc if jc >= 0 else s) % 2
        sc, sn = ("sA", "sB") if par == 0 else ("sB", "sA")
        has_next = jc < 0 or jc + 1 < KB
        out = block_max(sc, jc, balanced)
        if has_next:
            out += scores(sn, (s + 1) % 4)
        out += probs(sc)
        out += phase_end(vm)
        if jc < 0 or jc + 3 < KB:
            out += dma_lines("v", f"{j} + 3u", (s + 3) % 4)
        if jc < 0 or jc + 4 < KB:
            out += dma_lines("k", f"{j} + 4u", s)
        extra = []
        if balanced:
            # phase B carries part of the softmax: the sums of P(j) and the extremes of
            # S(j+1), which phase A would otherwise add to its exp2 work
            extra = rowsum16() + (lane_max16(sn, jc + 1 if jc >= 0 else None, "mbn") if has_next else [])
        out += pv(s, extra)
        out += phase_end(None)
        return out

    def dma_body() -> list[str]:
        """Ping-pong over 4 K and 4 V stages filled by DMA.  Prologue (all waves): K(0),
        K(1), V(0), then the loads phases B(-2) and B(-1) would have issued (V(1), K(2);
        V(2), K(3)); a barrier once K(0), K(1) and V(0) have landed; S(0); group 1 waits one
        extra barrier.  Blocks 0 .. 4n-1 (each followed by at least four more) run in a loop
        unrolled by four, so every stage is a compile-time array; the rest are peeled."""
        out = []
        first = dma_lines("k", "0u", 0) + (dma_lines("k", "1u", 1) if KB > 1 else []) + dma_lines("v", "0u", 0)
        for x in (-2, -1):
            if x + 3 < KB:
                out_v = dma_lines("v", f"{x + 3}u", (x + 3) % 4)
                first += out_v
            if x + 4 < KB:
                first += dma_lines("k", f"{x + 4}u", (x + 4) % 4)
        out += ["  " + x for x in first]
        out += ["  " + x for x in phase_end(n_dma(-2) + n_dma(-1))]
        out += ["  " + x for x in scores("sA", 0)]
        if balanced:
            out += ["  " + x for x in lane_max16("sA", 0, "mbn")]
        out += ["  if (gq == 1u) {"] + ["    " + x for x in phase_end(None)] + ["  }"]
        nquad = max(0, (KB - 4) // 4)
        if nquad:
            out.append(f"  for (unsigned int jj = 0; jj < {4 * nquad}u; jj += 4u) {{")
            for i in range(4):
                out += ["    {"] + [f"      const unsigned int j{i} = jj + {i}u;"]
                out += ["      " + x for x in dma_block(f"j{i}", -1, i, 4)] + ["    }"]
            out.append("  }")
        for j in range(4 * nquad, KB):
            out.append(f"  {{  // block {j}")
            out += ["    " + x for x in dma_block(f"{j}u", j, j % 4, n_dma(j - 1))]
            out.append("  }")
        out += ["  if (gq == 0u) {"] + ["    " + x for x in phase_end(None)] + ["  }"]
        return out

    def epilogue_lines() -> list[str]:
        # O = O^T / l: lane holds 4 consecutive dv per (u, r/4) for its query
        return ["#pragma unroll", f"  for (int q = 0; q < {QT}; ++q) {{",
                "    const unsigned int qrow = qrow0 + q * 32u;",
                "    const float l_tot = tj_pair_sum(l_run[q]);",
                f"    if (qrow < {Sq}u) {{",
                "      const float inv = 1.0f / l_tot;",
                "#pragma unroll",
                f"      for (int u = 0; u < {Dv // 32}; ++u)",
                "#pragma unroll",
                "        for (int r4 = 0; r4 < 4; ++r4) {",
                "          const unsigned int dv = u * 32 + r4 * 8 + g * 4u;",
                "          *(unsigned long*)&Ob[qrow * " + f"{ost}u + dv] = "
                + pack4.format("o[q][u][r4 * 4] * inv", "o[q][u][r4 * 4 + 1] * inv", "o[q][u][r4 * 4 + 2] * inv",
                               "o[q][u][r4 * 4 + 3] * inv") + ";",
                "        }",
                "    }",
                "  }",
                "}"]

    # key splits: partial rows [split][bh][Sq][Dv] (fp32, unnormalised), then the rows'
    # (running reference, sum) pairs [split][bh][Sq][2]
    ml_base = NS * batch * Sq * Dv

    def partial_epilogue_lines() -> list[str]:
        return ["#pragma unroll", f"  for (int q = 0; q < {QT}; ++q) {{",
                "    const unsigned int qrow = qrow0 + q * 32u;",
                "    const float l_tot = tj_pair_sum(l_run[q]);",
                f"    if (qrow < {Sq}u) {{",
                f"      const unsigned int prow = ((kb0 / {KBL}u) * {batch}u + (unsigned int)bh) * {Sq}u + qrow;",
                "#pragma unroll",
                f"      for (int u = 0; u < {Dv // 32}; ++u)",
                "#pragma unroll",
                "        for (int r4 = 0; r4 < 4; ++r4) {",
                "          tj_f32x4 w;",
                "          w[0] = o[q][u][r4 * 4]; w[1] = o[q][u][r4 * 4 + 1]; w[2] = o[q][u][r4 * 4 + 2]; w[3] = o[q][u][r4 * 4 + 3];",
                f"          *(tj_f32x4*)&ws_p[prow * {Dv}u + u * 32 + r4 * 8 + g * 4u] = w;",
                "        }",
                "      if (g == 0u) {",
                f"        ws_p[{ml_base}u + prow * 2u] = m_run[q];",
                f"        ws_p[{ml_base}u + prow * 2u + 1u] = l_tot;",
                "      }",
                "    }",
                "  }",
                "}"]

    if mi16:
        L += [f"  tj_f32x4 sA[2][{BKV // 16}], sB[2][{BKV // 16}];", f"  {opvec} pf[2][{BKV // 32}];"]
    else:
        L += [f"  tj_f32x16 sA[{QT}][{BKV // 32}], sB[{QT}][{BKV // 32}];", f"  {opvec} pf[{QT}][{BKV // 16}];"]
    L += dma_body() if dma else pingpong_body() if pingpong else double_buffer_body()
    L += epilogue16_lines() if mi16 else epilogue_lines() if NS == 1 else partial_epilogue_lines()
    lds = NST * BKV * 256 * 2 if dma else NST * BKV * (DP + VP) * dt.itemsize
    flops = 2.0 * batch * Sq * Sk * (D + Dv)
    meta = {"family": "attention", "dtype": dt.value, "batch": batch, "Sq": Sq, "Sk": Sk, "D": D, "Dv": Dv,
            "scale": scale, "lds_bytes": lds, "flops": flops, "splits": NS,
            "schedule": "pingpong-dma" if dma else "pingpong" if pingpong else "double-buffer",
            "mfma": "16x16x32" if mi16 else "32x32x16",
            "row_sums": "16-bit" if balanced else "fp32"}
    main = Launch(fname, (nq * batch * NS, 1, 1), (THREADS, 1, 1), 0, meta)
    if NS == 1:
        return (QUAD_HELPERS if mi16 else "") + "\n".join(L), main
    meta["workspace"] = (ml_base + NS * batch * Sq * 2) * 4
    meta["ws_arg"] = True
    # combine: one lane per 8 consecutive outputs of a row; weights 2^(m_s - max m) over
    # the splits, out = sum_s w_s * O_s / sum_s w_s * l_s
    runs = batch * Sq * (Dv // 8)
    cname = fname + "_combine"
    pack8 = ("tj_f2bf2({0}, {1})" if dt == DType.bf16 else "tj_f2h({0}) | (tj_f2h({1}) << 16)")
    C = [f'extern "C" __global__ void __launch_bounds__(256) {cname}(',
         f"    const {T}* __restrict__ in0_p, const {T}* __restrict__ in1_p, const {T}* __restrict__ in2_p,",
         f"    {T}* __restrict__ out0_p, const float* __restrict__ ws_p) {{",
         "  const unsigned int t = blockIdx.x * 256u + threadIdx.x;",
         f"  if (t >= {runs}u) return;",
         f"  const unsigned int d8 = (t % {Dv // 8}u) * 8u, row = t / {Dv // 8}u;",
         f"  const {idx_t} bh = row / {Sq}u;",
         f"  const unsigned int qrow = row % {Sq}u;",
         f"  {T}* __restrict__ Ob = out0_p + ({ooff});",
         f"  float mx = -__builtin_inff();",
         "#pragma unroll",
         f"  for (int sp = 0; sp < {NS}; ++sp) mx = fmaxf(mx, ws_p[{ml_base}u + (sp * {batch * Sq}u + row) * 2u]);",
         "  float lt = 0.0f, acc[8];",
         "#pragma unroll",
         "  for (int e = 0; e < 8; ++e) acc[e] = 0.0f;",
         "#pragma unroll",
         f"  for (int sp = 0; sp < {NS}; ++sp) {{",
         f"    const unsigned int prow = sp * {batch * Sq}u + row;",
         f"    const float w = __builtin_amdgcn_exp2f(ws_p[{ml_base}u + prow * 2u] - mx);",
         f"    lt += w * ws_p[{ml_base}u + prow * 2u + 1u];",
         f"    const tj_f32x4 a0 = *(const tj_f32x4*)&ws_p[prow * {Dv}u + d8];",
         f"    const tj_f32x4 a1 = *(const tj_f32x4*)&ws_p[prow * {Dv}u + d8 + 4u];",
         "#pragma unroll",
         "    for (int e = 0; e < 4; ++e) { acc[e] += w * a0[e]; acc[4 + e] += w * a1[e]; }",
         "  }",
         "  const float inv = 1.0f / lt;",
         "  tj_u32x4 pk;",
         "#pragma unroll",
         "  for (int e = 0; e < 4; ++e) {",
         "    const float lo = acc[2 * e] * inv, hi = acc[2 * e + 1] * inv;",
         "    pk[e] = " + pack8.format("lo", "hi") + ";",
         "  }",
         f"  *(tj_u32x4*)&Ob[qrow * {ost}u + d8] = pk;",
         "}"]
    cmeta = {"family": "attention_combine", "splits": NS, "ws_arg": True, "batch": batch, "Sq": Sq, "Dv": Dv}
    comb = Launch(cname, (-(-runs // 256), 1, 1), (256, 1, 1), 0, cmeta)
    return "\n".join(L) + "\n\n" + "\n".join(C), [main, comb]
