"""Kernel families 1 and 2 of the hip backend: pointwise loop nests and row kernels.

Both take a fused ``Kernel`` from the fusion passes and return HIP C++ text
plus the launch geometry.  Every size and stride is a literal; all compute
is fp32.

Family 1 (``elementwise`` / ``copy``; reference template
``tensorjit/backends/cuda_backend.py:142-160``): each lane owns 16-byte
vectors of the contiguous output.  A vector never crosses a row of the last
dim, so every input is read with one offset per vector: a 16-byte load when
its innermost stride is 1, one broadcast scalar when it is 0, a gather
otherwise.  ``U`` vectors per lane are loaded before any is computed so
several loads per lane are in flight.  Grid = one workgroup of
``POINTWISE_THREADS`` (128) lanes per ``128*U`` vectors (copies: 256 lanes; no
grid-stride loop; HIP's dispatcher spreads workgroups over all XCDs
round-robin).

Family 2 (``row`` and stand-alone ``reduce``; reference template
``tensorjit/backends/cuda_backend.py:168-289``): ``T`` lanes per row, each
owning ``NCH`` 16-byte chunks of it, chunk ``c`` at element ``(c*T + tid)*VEC``,
so each chunk load is coalesced.  Rows up to 4 KiB get one wave each (several
rows per workgroup), rows up to 16 KiB one workgroup with one chunk per lane,
longer rows several chunks per lane (``row_shape``).  External row inputs are
loaded once into VGPRs at kernel entry (the reference reloads them in every
stage) and values needed by later stages stay in VGPRs.  A reduction is a
per-lane partial, a wave64 DPP all-reduce and, with more than one wave per
row, one LDS exchange between the waves (one barrier, its own LDS slots per
reduction so consecutive reductions never race).  A row group without any
reduction is emitted as a flat family-1 loop nest over ``rows x N``.  A
stand-alone reduction over few long rows splits each row over workgroups
(``row_split``): partials into the workspace, then a combine launch per row.
"""
from __future__ import annotations

import os

import hashlib
import math
from dataclasses import dataclass, field

from ..ir import DType, Node
from ..passes import Kernel
from ..runtime.autotune import CU_COUNT
from .common import (access_strides, broadcast_strides, contiguous_strides, emit_expr, inner_stride, merged_dims,
                     offset_expr)
from .hip_prelude import CTYPE, vec_width

THREADS = 256


@dataclass
class Launch:
    name: str
    grid: tuple[int, int, int]
    block: tuple[int, int, int]
    shared: int = 0           # dynamic LDS bytes
    meta: dict = field(default_factory=dict)


@dataclass
class KernelGen:
    """Names for one kernel: external inputs ``in{j}``, nodes ``v{j}``, outputs ``out{j}``."""

    k: Kernel
    idx: int
    names: dict[int, str]

    @classmethod
    def of(cls, k: Kernel, idx: int) -> "KernelGen":
        names = {id(n): f"in{j}" for j, n in enumerate(k.inputs)}
        names.update({id(n): f"v{j}" for j, n in enumerate(k.nodes)})
        return cls(k, idx, names)

    @property
    def fname(self) -> str:
        """``tj<idx>_<kind>_<iteration shape>_<dtype>``: unique in the module, readable in profiles."""
        k = self.k
        if k.kind == "matmul":
            a, b = k.anchor.inputs
            M, K = a.shape[-2], a.shape[-1]
            N = b.shape[-2] if k.anchor.attrs.get("trans_b") else b.shape[-1]
            batch = math.prod(k.anchor.shape[:-2]) if len(k.anchor.shape) > 2 else 1
            dims = (f"{batch}x" if batch > 1 else "") + f"{M}x{N}x{K}" + ("_nt" if k.anchor.attrs.get("trans_b") else "_nn")
            dt = a.dtype.value
        else:
            shape = tuple(k.iter_shape)
            dims = "x".join(str(d) for d in shape) or "1"
            dt = (k.outputs[0].dtype if k.outputs else k.nodes[-1].dtype).value
        return f"tj{self.idx}_{k.kind}_{dims}_{dt}_{self._tag()}"

    def _tag(self) -> str:
        """Composite ops the kernel implements (ln, rms, softmax, linear), else a hash of its ops."""
        short = {"layer_norm": "ln", "rms_norm": "rms", "softmax": "softmax", "linear": "linear"}
        tags: list[str] = []
        for n in self.k.nodes:
            op = n.meta.get("composite", {}).get("op")
            if op and short.get(op, op) not in tags:
                tags.append(short.get(op, op))
        if tags:
            return "_".join(tags)
        ops = ",".join(n.op for n in self.k.nodes)
        return "op" + hashlib.sha1(ops.encode()).hexdigest()[:6]

    def params(self) -> str:
        ps = [f"const {CTYPE[n.dtype]}* __restrict__ {self.names[id(n)]}_p" for n in self.k.inputs]
        ps += [f"{CTYPE[o.dtype]}* __restrict__ out{j}_p" for j, o in enumerate(self.k.outputs)]
        return ", ".join(ps)

    def consumer(self, n: Node, nodes: list[Node]) -> Node:
        return next((c for c in nodes if n in c.inputs), nodes[0])


def _index_type(count: int) -> str:
    return "unsigned int" if count < 2**31 else "unsigned long"


def _kernel_dtype(k: Kernel) -> DType:
    """The storage dtype that sets the vector width (widest item wins)."""
    dts = [n.dtype for n in k.outputs] + [n.dtype for n in k.inputs]
    return max(dts, key=lambda d: d.itemsize) if dts else DType.f32


def _vec_for(row_len: int, numel: int, dtype: DType) -> int:
    w = vec_width(dtype)
    return w if row_len % w == 0 and numel % w == 0 else 1


# ---------------------------------------------------------------------------
# family 1: pointwise loop nest
# ---------------------------------------------------------------------------


# MI355X's last-level cache (MALL, "infinity cache") holds 256 MiB.  A kernel whose
# streamed inputs (read once, no broadcast dim) exceed that loads them with the
# nontemporal hint (no allocation in the caches they pass through): they cannot stay
# cached, and the hint measured faster, same kernels, interleaved: config 2 fp32 (512
# MiB in) 128.6 -> 120.3 us, RMSNorm bf16 (512 MiB in) 167.0 -> 163.8, a bf16 add of
# 2 x 512 MiB 258.5 -> 241.6.  Inputs that fit stay plain loads: whatever produced them
# (or the previous call) may have left them in the MALL.  Same box, both rounds, plain
# vs nontemporal: softmax fp32 [16384, 2048] (128 MiB in, 256 MiB of traffic) 37.6 vs
# 40.7 us, RMSNorm / LayerNorm bf16 [16384, 4096] 37.1-37.3 vs 42.3-45.1 / 38.2-39.5 vs
# 43.6-48.6, gelu fp32 [16384, 4096] (256 MiB in) 73.4-74.5 vs 78.3-81.5, config 2
# bf16 (256 MiB in) 64.1-68.7 vs 67.3-73.8.  Broadcast operands (re-read by every row)
# never take the hint.  TENSORJIT_HIP_NT_LOADS=0 / 1 forces it off / on for every
# streamed input.
MALL_BYTES = 256 << 20


def _flat_access(shape, strides) -> bool:
    """Are ``strides`` over ``shape`` the row-major strides of ``shape`` itself, or all
    zero (one scalar)?  Dims of size 1 take any stride."""
    contiguous = contiguous_strides(shape)
    return (all(d == 1 or s == c for d, s, c in zip(shape, strides, contiguous))
            or all(d == 1 or s == 0 for d, s in zip(shape, strides)))


def _streamed(shape, strides) -> bool:
    """Every element of the input is read once over ``shape``: no broadcast (stride-0) dim."""
    return all(st != 0 for d, st in zip(shape, strides) if d > 1)


def _nt_loads(streamed_input_bytes: int) -> bool:
    """Nontemporal loads for a kernel whose streamed inputs (each element read once) total
    ``streamed_input_bytes``."""
    forced = os.environ.get("TENSORJIT_HIP_NT_LOADS")
    if forced in ("0", "1"):
        return forced == "1"
    return streamed_input_bytes > MALL_BYTES


def _load_lines(src: str, ctype_ptr: str, off: str, inner: int, vec: int, dst: str, nt: bool = False) -> list[str]:
    """Lines that fill ``dst[0..vec)`` with fp32 values of one vector of input ``src``
    (``nt``: a contiguous vector load with the nontemporal hint)."""
    if vec == 1:
        return [f"{dst}[0] = tj_ld({src}_p[{off}]);"]
    if inner == 1:
        return [f"tj_ldv{'_nt' if nt else ''}({src}_p + ({off}), {dst});"]
    if inner == 0:
        return [f"{{ const float s_ = tj_ld({src}_p[{off}]);",
                f"  for (int j = 0; j < {vec}; ++j) {dst}[j] = s_; }}"]
    return [f"for (int j = 0; j < {vec}; ++j) {dst}[j] = tj_ld({src}_p[({off}) + j * {inner}u]);"]


# 16-byte vectors per lane in the pointwise and copy families.  One vector
# per lane measured fastest at every size (deeper unrolling loses 3-8% on
# config 2 and on a plain copy: the extra loads in flight per lane do not make
# up for fewer resident waves per CU).
POINTWISE_UNROLL = 1
# Lanes per workgroup of the pointwise family: config 2 (two streamed inputs,
# one output) ran 132.4 us in fp32 / 58.8 us in bf16 with 128-lane workgroups
# against 136.2 / 59.6 us with 256 and 133.7 / 58.5 with 512 (same box,
# interleaved, best of 8 rounds)
POINTWISE_THREADS = 128


def gen_pointwise(g: KernelGen, nodes: list[Node], iter_shape: tuple[int, ...]) -> tuple[str, Launch]:
    """Fused pointwise DAG ``nodes`` over ``iter_shape`` (elementwise kernels and
    reduction-free row groups)."""
    k = g.k
    numel = math.prod(iter_shape) if iter_shape else 1
    in_st = {id(n): access_strides(n, g.consumer(n, nodes), iter_shape) for n in k.inputs}
    # every input read contiguously over the whole iteration space (or as one scalar):
    # element e sits at offset e of each, so a vector may cross rows and its width
    # depends on the element count alone ([16384, 4095] fp32: 16-byte vectors, not scalars)
    flat = all(_flat_access(iter_shape, st) for st in in_st.values())
    row_len = numel if flat else (iter_shape[-1] if iter_shape else 1)
    vec = _vec_for(row_len, numel, _kernel_dtype(k))
    nvec = numel // vec
    unroll = POINTWISE_UNROLL
    per_block = POINTWISE_THREADS * unroll
    grid = max(1, -(-nvec // per_block))
    idx_t = _index_type(numel)
    guard = nvec % per_block != 0
    inside = {id(n) for n in nodes}
    streamed = {id(n) for n in k.inputs if _streamed(iter_shape, in_st[id(n)])}
    nt = _nt_loads(sum(math.prod(n.shape or (1,)) * n.dtype.itemsize for n in k.inputs if id(n) in streamed))

    L = [f'extern "C" __global__ __launch_bounds__({POINTWISE_THREADS}) void {g.fname}({g.params()}) {{',
         f"  const {idx_t} vbase = ({idx_t})blockIdx.x * {per_block}u + threadIdx.x;"]
    for n in k.inputs:
        L.append(f"  float {g.names[id(n)]}_v[{unroll}][{vec}];")
    # phase 1: issue every load of this lane
    L.append("#pragma unroll")
    L.append(f"  for (int u = 0; u < {unroll}; ++u) {{")
    L.append(f"    const {idx_t} vi = vbase + u * {POINTWISE_THREADS}u;")
    if guard:
        L.append(f"    if (vi >= {nvec}u) break;")
    L.append(f"    const {idx_t} e = vi * {vec}u;")
    for n in k.inputs:
        st = in_st[id(n)]
        nm = g.names[id(n)]
        L += ["    " + s for s in _load_lines(nm, CTYPE[n.dtype], offset_expr("e", iter_shape, st),
                                             inner_stride(iter_shape, st), vec, f"{nm}_v[u]",
                                             nt and id(n) in streamed)]
    L.append("  }")
    # phase 2: compute and store
    L.append("#pragma unroll")
    L.append(f"  for (int u = 0; u < {unroll}; ++u) {{")
    L.append(f"    const {idx_t} vi = vbase + u * {POINTWISE_THREADS}u;")
    if guard:
        L.append(f"    if (vi >= {nvec}u) break;")
    L.append(f"    const {idx_t} e = vi * {vec}u;")
    for j, o in enumerate(k.outputs):
        L.append(f"    float o{j}_v[{vec}];")
    L.append("#pragma unroll")
    L.append(f"    for (int j = 0; j < {vec}; ++j) {{")
    local = {id(n): f"{g.names[id(n)]}_v[u][j]" for n in k.inputs}
    for n in nodes:
        if n.op in ("transpose", "broadcast_to"):
            expr = local[id(n.inputs[0])]
        else:
            expr = emit_expr(n, local)
        L.append(f"      const float {g.names[id(n)]} = {expr};")
        local[id(n)] = g.names[id(n)]
    for j, o in enumerate(k.outputs):
        if id(o) not in inside:
            raise AssertionError(f"output {o.name} not computed by {g.fname}")
        L.append(f"      o{j}_v[j] = {g.names[id(o)]};")
    L.append("    }")
    for j, o in enumerate(k.outputs):
        if vec == 1:
            L.append(f"    tj_st(out{j}_p + e, o{j}_v[0]);")
        else:
            L.append(f"    tj_stv(out{j}_p + e, o{j}_v);")
    L.append("  }")
    L.append("}")
    meta = {"family": "pointwise", "vec": vec, "unroll": unroll, "numel": numel}
    return "\n".join(L), Launch(g.fname, (grid, 1, 1), (POINTWISE_THREADS, 1, 1), 0, meta)


def gen_elementwise(g: KernelGen) -> tuple[str, Launch]:
    return gen_pointwise(g, g.k.nodes, tuple(g.k.iter_shape))


TT = 64          # tiled transpose: tile edge in elements


def _tiled_transpose_plan(shape, st, itemsize):
    """For a transpose whose output's innermost dim is strided in the source: the merged
    dim groups as (E0, s0) -- the output's innermost (source stride s0) --, (Er, Ir) --
    the group that is contiguous in the source (output stride Ir) -- and the rest as
    batch groups [(extent, output stride, source stride)], or None when the plain copy
    applies (vectorisable, broadcast, or 16-byte alignment not given)."""
    groups = merged_dims(shape, st)
    if len(groups) < 2 or groups[0][2] in (0, 1):
        return None
    vec = 16 // itemsize
    rg = [i for i, g in enumerate(groups) if g[2] == 1]
    if len(rg) != 1:
        return None
    E0, _, s0 = groups[0]
    Er, Ir, _ = groups[rg[0]]
    batch = [g for i, g in enumerate(groups) if i not in (0, rg[0])]
    # 16-byte vectors along the source's contiguous group (reads) and the output's
    # innermost group (writes): every row start of either must be 16-byte aligned
    if E0 % vec or Er % vec or s0 % vec or any(g[2] % vec or g[1] % vec for g in batch) or Ir % vec:
        return None
    return E0, s0, Er, Ir, batch


def gen_copy_tiled(g: KernelGen, plan) -> tuple[str, Launch]:
    """Transpose whose output's innermost dim is strided in the source, through LDS:
    a workgroup moves a TT x TT tile -- 16-byte loads along the source's contiguous
    dim into LDS rows, then 16-byte stores along the output's innermost dim gathered
    from LDS columns -- so both HBM streams are coalesced (the plain copy gathers
    single elements at the source stride)."""
    k = g.k
    node = k.anchor
    (src,) = k.inputs if k.inputs else (node.inputs[0],)
    E0, s0, Er, Ir, batch = plan
    ct = CTYPE[node.dtype]
    isz = node.dtype.itemsize
    vec = 16 // isz
    numel = math.prod(node.shape)
    idx_t = _index_type(numel)
    tc, tr = -(-E0 // TT), -(-Er // TT)
    nb = math.prod(e for e, _, _ in batch) if batch else 1
    vpr = TT // vec                        # 16-byte vectors per tile row
    per = TT * vpr // THREADS              # vectors per lane per phase
    pitch = TT + vec                       # LDS row pitch: 16 bytes of padding keep rows 16-byte aligned
    sname = g.names[id(src)]
    L = [f'extern "C" __global__ __launch_bounds__({THREADS}) void {g.fname}({g.params()}) {{',
         f"  __shared__ __attribute__((aligned(16))) {ct} T_[{TT}][{pitch}];",
         f"  const unsigned int tid = threadIdx.x, c0 = (blockIdx.x % {tc}u) * {TT}u,"
         f" r0 = ((blockIdx.x / {tc}u) % {tr}u) * {TT}u;",
         f"  {idx_t} bi = blockIdx.x / {tc * tr}u, so = 0, oo = 0;"]
    for j, (e, ostride, sstride) in enumerate(batch):
        L.append(f"  {{ const {idx_t} x_ = bi % {e}u; bi /= {e}u; so += x_ * {sstride}u; oo += x_ * {ostride}u; }}")
    # load: tile row = output-inner index c (source stride s0), 16 bytes along r
    L += ["#pragma unroll", f"  for (int u = 0; u < {per}; ++u) {{",
          f"    const unsigned int v = u * {THREADS}u + tid, c = v / {vpr}u, r = (v % {vpr}u) * {vec}u;",
          f"    if (c0 + c < {E0}u && r0 + r < {Er}u)",
          f"      *(tj_u32x4*)&T_[c][r] = *(const tj_u32x4*)&{sname}_p[so + ({idx_t})(c0 + c) * {s0}u + r0 + r];",
          "  }", "  __syncthreads();",
          # store: output row = r, 16 bytes along c, gathered from the LDS column
          "#pragma unroll", f"  for (int u = 0; u < {per}; ++u) {{",
          f"    const unsigned int v = u * {THREADS}u + tid, r = v / {vpr}u, c = (v % {vpr}u) * {vec}u;",
          f"    if (c0 + c < {E0}u && r0 + r < {Er}u) {{",
          f"      {ct} t_[{vec}];",
          "#pragma unroll",
          f"      for (int j = 0; j < {vec}; ++j) t_[j] = T_[c + j][r];",
          f"      tj_st16(out0_p + oo + ({idx_t})(r0 + r) * {Ir}u + c0 + c, *(const tj_u32x4*)t_);",
          "    }", "  }", "}"]
    meta = {"family": "copy", "vec": vec, "tiled": TT, "numel": numel}
    return "\n".join(L), Launch(g.fname, (tc * tr * nb, 1, 1), (THREADS, 1, 1), 0, meta)


def gen_copy(g: KernelGen) -> tuple[str, Launch]:
    """Materialised transpose / broadcast_to: a bit-exact move of storage elements."""
    k = g.k
    node = k.anchor
    (src,) = k.inputs if k.inputs else (node.inputs[0],)
    shape = tuple(node.shape)
    numel = math.prod(shape) if shape else 1
    ct = CTYPE[node.dtype]
    st = access_strides(src, node, shape)
    inner = inner_stride(shape, st)
    if node.op == "transpose" and len(k.outputs) == 1 and k.outputs[0] is node and node.dtype == src.dtype:
        plan = _tiled_transpose_plan(shape, st, node.dtype.itemsize)
        if plan is not None:
            return gen_copy_tiled(g, plan)
    row_len = shape[-1] if shape else 1
    vec = _vec_for(row_len, numel, node.dtype)
    nvec = numel // vec
    unroll = POINTWISE_UNROLL
    per_block = THREADS * unroll
    grid = max(1, -(-nvec // per_block))
    idx_t = _index_type(numel)
    sname = g.names[id(src)]
    off = offset_expr("e", shape, st)
    L = [f'extern "C" __global__ __launch_bounds__({THREADS}) void {g.fname}({g.params()}) {{',
         f"  const {idx_t} vbase = ({idx_t})blockIdx.x * {per_block}u + threadIdx.x;",
         "#pragma unroll",
         f"  for (int u = 0; u < {unroll}; ++u) {{",
         f"    const {idx_t} vi = vbase + u * {THREADS}u;"]
    if nvec % per_block:
        L.append(f"    if (vi >= {nvec}u) break;")
    L.append(f"    const {idx_t} e = vi * {vec}u;")
    if vec > 1 and inner == 1:
        L.append(f"    tj_st16(out0_p + e, *(const tj_u32x4*)({sname}_p + ({off})));")
    elif vec > 1 and inner == 0:
        L.append(f"    const {ct} s_ = {sname}_p[{off}];")
        L.append(f"    for (int j = 0; j < {vec}; ++j) out0_p[e + j] = s_;")
    elif vec > 1:
        L.append(f"    {ct} t_[{vec}];")
        L.append(f"    for (int j = 0; j < {vec}; ++j) t_[j] = {sname}_p[({off}) + j * {inner}u];")
        L.append("    tj_st16(out0_p + e, *(const tj_u32x4*)t_);")
    else:
        L.append(f"    out0_p[e] = {sname}_p[{off}];")
    L += ["  }", "}"]
    if len(k.outputs) != 1 or k.outputs[0] is not node:
        raise AssertionError("copy kernels have exactly one output, the moved value")
    if node.dtype != src.dtype:
        raise AssertionError("copy kernels do not convert dtypes")
    meta = {"family": "copy", "vec": vec, "unroll": unroll, "numel": numel}
    return "\n".join(L), Launch(g.fname, (grid, 1, 1), (THREADS, 1, 1), 0, meta)


# ---------------------------------------------------------------------------
# family 2: row kernels
# ---------------------------------------------------------------------------


# Rows past 256 lanes x 16 chunks: a single-stage reduction streams through a rolled
# loop; a row with several stages keeps every stage's values in VGPRs, so it takes up to
# 1024 lanes (16 waves: 128 VGPRs each) holding at most ROW_MAX_FLOATS floats per lane
# per row array.  That covers every row of up to 32768 elements at any vector width.
ROW_MAX_FLOATS = 32


def row_geometry(N: int, vec: int, streaming_ok: bool) -> tuple[int, int, bool]:
    """(threads T, chunks per lane NCH, streaming).  Up to 256 lanes x 16 chunks of
    ``vec`` elements (rows with several stages: 512 lanes from 12 chunks at 256); then a
    rolled loop over 1024 lanes (single-stage reductions) or up to 1024 lanes x
    ROW_MAX_FLOATS // vec chunks (rows with several stages)."""
    nv = -(-N // vec)
    nch = max(1, -(-nv // 256))
    t = 64 * -(-(-(-nv // nch)) // 64)
    if nch <= 16:
        if nch >= 12 and not streaming_ok and -(-nv // 512) * vec <= ROW_MAX_FLOATS:
            # rows with several stages that would hold 12-16 chunks per lane take 512 lanes:
            # same box, generator, 256 x 16 -> 512 x 8 for fp32 [8192, 16384] LayerNorm
            # 179.7 -> 169.9 us, softmax 181.0 -> 172.1, RMSNorm 181.0 -> 183.8; 256 x 12 ->
            # 512 x 6 for fp32 [8192, 12288] 131.8 / 132.8 / 131.1 -> 130.0 / 130.3 / 127.0
            # (bf16 rows of 8 chunks keep 256 lanes: 512 lanes lost 0-3%; past 256 lanes a lane
            # holds at most ROW_MAX_FLOATS values per row array, as below)
            nch = -(-nv // 512)
            return 64 * -(-(-(-nv // nch)) // 64), nch, False
        return t, nch, False
    if streaming_ok:
        return 1024, -(-nv // 1024), True
    nch = -(-nv // 1024)
    if nch * vec > ROW_MAX_FLOATS:
        raise NotImplementedError(f"row length {N} needs {nch} chunks of {vec} per lane at 1024 lanes")
    return 64 * -(-(-(-nv // nch)) // 64), nch, False


# Row layouts, chosen by row size in 16-byte chunks (nv), measured on MI355X against a
# flat copy of the same bytes (165 us for bf16 [65536, 4096] on the same box):
# * nv <= 256 (rows up to 4 KiB): one 64-lane wave per row, WAVE_ROWS_PER_BLOCK rows per
#   workgroup; reductions never leave the wave (no LDS, no barrier).  Config 5's bf16
#   softmax [262144, 2048]: 360 us against 395 us for one 256-lane workgroup per row.
# * nv <= 1024 (up to 16 KiB): one workgroup per row, one chunk per lane (nv lanes rounded
#   up to a whole wave).  Streaming copies run fastest with a single 16-byte load per lane
#   (two or more per lane lose 6-12%): RMSNorm bf16 [65536, 4096] 167 us against 173 us
#   with 256 lanes x 2 chunks.
# * longer rows: row_geometry (256 lanes x up to 16 chunks, then 1024 lanes).
WAVE_ROW_MAX_CHUNKS = 4
WAVE_ROWS_PER_BLOCK = 4
ONE_CHUNK_MAX_LANES = 1024
# Rows of 257-1024 chunks with two or more reductions take this many lanes and several
# chunks per lane instead, when the rows are longer than 512 chunks (8 KiB) or every input
# the row kernel reads per element is a whole [rows, N] tensor: every reduction is a
# barrier across the row's waves, and fewer waves per row wait less.  Measured on one box
# through the generator (us, 512 or 1024 lanes x 1 chunk -> 256 lanes x 2-4 chunks):
# softmax fp32 [65536, 2048] 171.6 -> 161.6, bf16 [65536, 4096] 192.8 -> 169.4, fp16
# 200.8 -> 180.2, bf16 [32768, 8192] 197.0 -> 165.8, fp32 [32768, 4096] 172.1 -> 167.9;
# LayerNorm (with a gain broadcast over rows) bf16 [32768, 8192] 186.3 -> 173.4, fp32
# [32768, 4096] 186.3 -> 172.7, but over 8 KiB rows it loses: bf16 [65536, 4096] 169.0 ->
# 173.0, fp16 171.2 -> 173.4, fp32 [65536, 2048] 164.4 -> 172.1.  128 lanes was slower
# than 256 on 10 of those 12 cases.  A plain copy of 8 KiB rows runs 163.0 us at 512 x 1
# and 178.1 at 256 x 2, so single-reduction and reduction-free rows keep one chunk.
MULTI_REDUCTION_LANES = 256


@dataclass(frozen=True)
class RowShape:
    lanes: int          # lanes per row
    chunks: int         # 16-byte chunks per lane
    streaming: bool     # rolled chunk loop, inputs loaded per stage
    rows_per_block: int


def row_shape(N: int, vec: int, streaming_ok: bool, reductions: int = 1, whole_row_inputs: bool = False) -> RowShape:
    """Lanes and chunks of a row kernel over rows of ``N`` elements in ``vec``-element
    chunks; ``reductions``: reduction stages in the row kernel; ``whole_row_inputs``: every
    input read per element is a whole [rows, N] tensor (none is broadcast over rows)."""
    nv = -(-N // vec)
    if nv <= 64 * WAVE_ROW_MAX_CHUNKS:
        return RowShape(64, -(-nv // 64), False, WAVE_ROWS_PER_BLOCK)
    if nv <= ONE_CHUNK_MAX_LANES:
        if reductions >= 2 and nv > MULTI_REDUCTION_LANES and (nv > 512 or whole_row_inputs):
            return RowShape(MULTI_REDUCTION_LANES, -(-nv // MULTI_REDUCTION_LANES), False, 1)
        return RowShape(64 * -(-nv // 64), 1, False, 1)
    t, nch, streaming = row_geometry(N, vec, streaming_ok)
    return RowShape(t, nch, streaming, 1)


# A reduction over few long rows splits each row over workgroups.  With one workgroup
# per row, a [1, 2^26] fp32 sum ran on one CU at 62 GB/s (4.3 ms).  Here a row is cut
# into segments of SPLIT_CHUNKS chunks of SPLIT_THREADS x 16 bytes.  Each of ``S``
# workgroups per row loops over every S-th segment.  It preloads the segment's chunks,
# folds them into its partial, and writes the partial to the workspace.  A second
# launch, one workgroup per row, combines the partials.  It then divides a mean by N
# and runs the reduction's epilogue.  Measured on MI355X, fp32 sum (max alike), one
# workgroup per row -> split: [1, 2^26] 4330 -> 39.5 us (6.8 TB/s; torch 47.5),
# [8, 2^23] 524 -> 39.7, [64, 2^20] 78.9 -> 42.5, [1, 2^20] 29.4 -> 4.2, [8, 2^18]
# 8.7 -> 4.5; the combine launch costs 2.0 us, so 256 KiB rows lose ([1, 2^16]
# 3.2 -> 4.4) and [200, 2^16] gains nothing (10.9 -> 10.6).  One workgroup per CU in all:
# against 2 / 4 / 8 per CU (same box, main + combine launch, us) [1, 2^26] 38.8 against
# 39.7 / 39.7 / 39.7, [64, 2^20] 39.1 against 39.3 / 41.1 / 40.2, [1, 2^27] 75.5 against
# 77.0 / 76.4 / 77.3, [1, 2^25] 21.2 against 21.4 / 21.3 / 21.5.  TENSORJIT_HIP_ROW_SPLIT=0 / 1
# forces the split off / on.
SPLIT_THREADS = 256
SPLIT_CHUNKS = 8
SPLIT_MIN_ROW_BYTES = 512 << 10


@dataclass(frozen=True)
class RowSplit:
    chunks: int         # chunks per lane per segment
    segments: int       # segments per row
    splits: int         # workgroups per row


def row_split(nrows: int, N: int, vec: int, itemsize: int) -> RowSplit | None:
    """Split of a single-stage reduction over ``nrows`` rows of ``N`` elements, or None
    when one workgroup per row already fills the chip or a row is short.  About
    CU_COUNT workgroups in all; segments shrink, down to one chunk per lane, until
    the row count times the segments per row reaches that."""
    forced = os.environ.get("TENSORJIT_HIP_ROW_SPLIT")
    if forced == "0" or (forced != "1" and (nrows >= CU_COUNT or N * itemsize < SPLIT_MIN_ROW_BYTES)):
        return None
    target = CU_COUNT
    per_row = -(-N // (SPLIT_THREADS * vec))
    nch = max(1, min(SPLIT_CHUNKS, per_row * nrows // target))
    segs = -(-per_row // nch)
    splits = min(segs, -(-target // nrows))
    return RowSplit(nch, segs, splits) if splits > 1 else None


def gen_row(g: KernelGen, stages: list[Kernel], rows: tuple, N: int) -> tuple[str, Launch]:
    k = g.k
    nrows = math.prod(rows) if rows else 1
    vec_shape = tuple(rows) + (N,)
    has_reduce = any(st.kind == "reduce" for st in stages)
    if not has_reduce and all(tuple(st.iter_shape) == vec_shape for st in stages):
        return gen_pointwise(g, k.nodes, vec_shape)

    dt = _kernel_dtype(k)
    vec = _vec_for(N, N, dt)
    inside = {id(n) for n in k.nodes}
    escaping = {id(o): j for j, o in enumerate(k.outputs)}
    stage_of = {id(n): si for si, st in enumerate(stages) for n in st.nodes}
    # per-row scalars: reduction results, their epilogues and scalar stages (classified by
    # position, not shape: with N == 1 a keepdim reduction has the row shape too)
    scalar_ids = set()
    for st in stages:
        if st.kind == "reduce":
            scalar_ids |= {id(n) for n in st.nodes[st.nodes.index(st.anchor):]}
        elif tuple(st.iter_shape) != vec_shape:
            scalar_ids |= {id(n) for n in st.nodes}
    is_vec = lambda n: id(n) not in scalar_ids  # noqa: E731
    # vec values read by a later stage stay in registers, and so do those a per-row node
    # reads (possible only with N == 1, where the row is one element)
    anchors = {id(st.anchor) for st in stages if st.kind == "reduce"}   # read their input in the row loop
    kept = [n for si, st in enumerate(stages) for n in st.nodes
            if is_vec(n) and any(stage_of.get(id(u), si) != si or not (is_vec(u) or id(u) in anchors)
                                 for u in n.users if id(u) in inside)]
    kept_ids = {id(n) for n in kept}
    scalars = [n for n in k.nodes if not is_vec(n)]
    nred = sum(st.kind == "reduce" for st in stages)
    idx_t = _index_type(nrows * N)

    # external inputs read per element (vec context) and per row (scalar context)
    vec_ext: dict[int, tuple[Node, tuple[int, ...]]] = {}
    for st in stages:
        if st.kind == "reduce":
            red = st.anchor
            pos = st.nodes.index(red)
            elem_nodes = st.nodes[:pos + 1]
        elif tuple(st.iter_shape) == vec_shape:
            elem_nodes = st.nodes
        else:
            continue
        for n in st.inputs:
            if id(n) in inside or id(n) in vec_ext:
                continue
            if not any(n in m.inputs for m in elem_nodes):
                continue
            strides = access_strides(n, g.consumer(n, [m for m in elem_nodes if n in m.inputs] or elem_nodes),
                                     vec_shape)
            vec_ext[id(n)] = (n, strides)
    ext_streamed = {i for i, (n, st_) in vec_ext.items() if _streamed(vec_shape, st_)}
    nt = _nt_loads(sum(math.prod(n.shape) * n.dtype.itemsize for i, (n, _) in vec_ext.items() if i in ext_streamed))

    split = row_split(nrows, N, vec, dt.itemsize) if len(stages) == 1 and stages[0].kind == "reduce" else None
    if split:
        T, NCH, streaming, R = SPLIT_THREADS, split.chunks, False, 1
    else:
        shape = row_shape(N, vec, streaming_ok=len(stages) == 1, reductions=nred,
                          whole_row_inputs=len(ext_streamed) == len(vec_ext))
        T, NCH, streaming, R = shape.lanes, shape.chunks, shape.streaming, shape.rows_per_block
    if R > 1 and nrows < R * 256:
        # too few rows to fill the chip with R-row workgroups: one row per workgroup
        R = 1
    nwaves = T // 64
    # every chunk in bounds: whole rows of chunks, and with a split whole segments
    full = N % (T * vec * (NCH if split else 1)) == 0

    ws_param = ", float* __restrict__ ws_p" if split else ""
    L = [f'extern "C" __global__ __launch_bounds__({T * R}) void {g.fname}({g.params()}{ws_param}) {{']
    if nred and nwaves > 1:
        L.append(f"  __shared__ float tj_red[{nred}][{nwaves}];")
    if split:
        # workgroup (r, sb): segments sb, sb + S, ... of row r
        L.append(f"  const {idx_t} r = blockIdx.x / {split.splits}u;")
        L.append(f"  const unsigned int sb = blockIdx.x % {split.splits}u;")
        L.append("  const unsigned int tid = threadIdx.x;")
    elif R == 1:
        L.append(f"  const {idx_t} r = blockIdx.x;")
        L.append("  const unsigned int tid = threadIdx.x;")
    else:
        # one wave per row: reductions never leave the wave, so a wave past the last
        # row simply returns
        L.append(f"  const {idx_t} r = ({idx_t})blockIdx.x * {R}u + (threadIdx.x >> 6);")
        L.append("  const unsigned int tid = threadIdx.x & 63u;")
        if nrows % R:
            L.append(f"  if (r >= {nrows}u) return;")
    if scalars:
        L.append("  float " + ", ".join(g.names[id(n)] for n in scalars) + ";")

    def chunk_open(c: str, body_indent: str = "    ") -> list[str]:
        c = f"(seg * {NCH}u + {c})" if split else c
        out = [f"  {{ const unsigned int n0 = ({c} * {T}u + tid) * {vec}u;"]
        if not full:
            out.append(f"  if (n0 < {N}u) {{")
        return out

    def chunk_close() -> list[str]:
        return ["  }"] + ([] if full else ["  }"])

    def ext_load(n: Node, strides, dst: str) -> list[str]:
        off = offset_expr(f"(r * {N}u + n0)", vec_shape, strides)
        return _load_lines(g.names[id(n)], CTYPE[n.dtype], off, inner_stride(vec_shape, strides), vec, dst,
                           nt and id(n) in ext_streamed)

    # register arrays: preloaded external inputs and kept values
    preload = not streaming
    if preload:
        for n, strides in vec_ext.values():
            nm = g.names[id(n)]
            L.append(f"  float {nm}_r[{NCH}][{vec}];")
        for n in kept:
            # lanes past the row's end never write theirs: start them at zero
            L.append(f"  float {g.names[id(n)]}_r[{NCH}][{vec}]{'' if full else ' = {}'};")
    preload_lines = []
    if preload and vec_ext:
        preload_lines.append("#pragma unroll")
        preload_lines.append(f"  for (int c = 0; c < {NCH}; ++c) {{")
        preload_lines += ["  " + s for s in chunk_open("c")]
        for n, strides in vec_ext.values():
            preload_lines += ["      " + s for s in ext_load(n, strides, f"{g.names[id(n)]}_r[c]")]
        preload_lines += ["  " + s for s in chunk_close()]
        preload_lines.append("  }")
    if not split:
        L += preload_lines

    def elem_value(n: Node) -> str:
        """fp32 value of input/earlier-stage node ``n`` at (chunk c, lane element j)."""
        if id(n) in vec_ext:
            return f"{g.names[id(n)]}_r[c][j]" if preload else f"{g.names[id(n)]}_l[j]"
        if id(n) in kept_ids:
            return f"{g.names[id(n)]}_r[c][j]"
        if id(n) in inside and not is_vec(n):
            return g.names[id(n)]
        raise AssertionError(f"row kernel {g.fname}: no value for {n.name}")

    def elem_block(nodes: list[Node], inputs: list[Node], extra: list[str]) -> list[str]:
        """Per-element body for chunk c: loads (streaming), compute, stores, keeps."""
        out = []
        if not preload:
            for n in inputs:
                if id(n) in vec_ext:
                    out.append(f"float {g.names[id(n)]}_l[{vec}];")
                    out += ext_load(n, vec_ext[id(n)][1], f"{g.names[id(n)]}_l")
        stores = [n for n in nodes if id(n) in escaping and is_vec(n)]
        for n in stores:
            out.append(f"float {g.names[id(n)]}_o[{vec}];")
        out.append("#pragma unroll")
        out.append(f"for (int j = 0; j < {vec}; ++j) {{")
        own = {id(m) for m in nodes}
        local = {id(n): elem_value(n) for n in inputs if id(n) not in own}
        for n in nodes:
            out.append(f"  const float {g.names[id(n)]}_e = {emit_expr(n, local)};")
            local[id(n)] = f"{g.names[id(n)]}_e"
            if id(n) in kept_ids:
                out.append(f"  {g.names[id(n)]}_r[c][j] = {g.names[id(n)]}_e;")
            if n in stores:
                out.append(f"  {g.names[id(n)]}_o[j] = {g.names[id(n)]}_e;")
        out += ["  " + s for s in extra]
        out.append("}")
        for n in stores:
            j = escaping[id(n)]
            dst = f"out{j}_p + r * {N}u + n0"
            out.append(f"tj_stv({dst}, {g.names[id(n)]}_o);" if vec > 1 else f"tj_st({dst}, {g.names[id(n)]}_o[0]);")
        return out

    def chunk_loop(body: list[str]) -> list[str]:
        out = []
        if streaming:
            out.append(f"  for (int c = 0; c < {NCH}; ++c) {{")
        else:
            out.append("#pragma unroll")
            out.append(f"  for (int c = 0; c < {NCH}; ++c) {{")
        out += ["  " + s for s in chunk_open("c")]
        out += ["      " + s for s in body]
        out += ["  " + s for s in chunk_close()]
        out.append("  }")
        return out

    def scalar_store(n: Node) -> list[str]:
        if id(n) not in escaping:
            return []
        return [f"  if (tid == 0) tj_st(out{escaping[id(n)]}_p + r, {g.names[id(n)]});"]

    def scalar_lines(nodes: list[Node], st: Kernel, shape: tuple, idx_vars_expr: str,
                     anchor: Node | None = None) -> list[str]:
        """Per-row scalar nodes (uniform across the workgroup)."""
        out = []
        local: dict[int, str] = {id(anchor): g.names[id(anchor)]} if anchor is not None else {}
        for n in st.inputs + [i for nd in nodes for i in nd.inputs if id(i) in inside and is_vec(i)]:
            if id(n) in local or not any(n in m.inputs for m in nodes):
                continue
            if id(n) in inside and is_vec(n):
                # a row value read per row: N == 1, and the row's one element is held by
                # the row's first lane; every lane takes that lane's value
                assert N == 1 and id(n) in kept_ids, (g.fname, n.name)
                local[id(n)] = (f"__builtin_bit_cast(float, __builtin_amdgcn_readfirstlane("
                                f"__builtin_bit_cast(int, {g.names[id(n)]}_r[0][0])))")
            elif id(n) in inside:
                local[id(n)] = g.names[id(n)]
            elif any(n in m.inputs for m in nodes):
                strides = access_strides(n, g.consumer(n, [m for m in nodes if n in m.inputs]), shape)
                off = offset_expr(idx_vars_expr, shape, strides)
                out.append(f"  const float {g.names[id(n)]}_s{st_i} = tj_ld({g.names[id(n)]}_p[{off}]);")
                local[id(n)] = f"{g.names[id(n)]}_s{st_i}"
        for n in nodes:
            local[id(n)] = g.names[id(n)]
            out.append(f"  {g.names[id(n)]} = {emit_expr(n, local)};")
            out += scalar_store(n)
        return out

    red_slot = 0
    for st_i, st in enumerate(stages):
        L.append(f"  // stage {st_i}: {st.kind} {[n.op for n in st.nodes]}")
        if st.kind == "reduce":
            red = st.anchor
            pos = st.nodes.index(red)
            prologue, epilogue = st.nodes[:pos], st.nodes[pos + 1:]
            x = red.inputs[0]
            is_max = red.op == "max"
            init = "(-__builtin_inff())" if is_max else "0.0f"
            xv = f"{g.names[id(x)]}_e" if x in prologue else elem_value(x)
            upd = f"acc{st_i} = fmaxf(acc{st_i}, {xv});" if is_max else f"acc{st_i} += {xv};"
            L.append(f"  float acc{st_i} = {init};")
            used = [n for n in st.inputs if any(n in m.inputs for m in prologue + [red])]
            if split:
                # this workgroup's segments of the row: preload one, fold it in, next
                L.append(f"  for (unsigned int seg = sb; seg < {split.segments}u; seg += {split.splits}u) {{")
                L += ["  " + s for s in preload_lines + chunk_loop(elem_block(prologue, used, [upd]))]
                L.append("  }")
            else:
                L += chunk_loop(elem_block(prologue, used, [upd]))
            L += _block_reduce_lines(f"acc{st_i}", is_max, nwaves, red_slot)
            red_slot += 1
            if split:
                # the partial of segments sb, sb + S, ...; the combine launch finishes the row
                L.append(f"  if (tid == 0u) ws_p[blockIdx.x] = acc{st_i};")
                break
            if red.op == "mean":
                L.append(f"  {g.names[id(red)]} = acc{st_i} / {float(N)!r}f;")
            else:
                L.append(f"  {g.names[id(red)]} = acc{st_i};")
            L += scalar_store(red)
            L += scalar_lines(epilogue, st, tuple(red.shape), "r", anchor=red)
        elif tuple(st.iter_shape) == vec_shape:
            used = [n for n in st.inputs if any(n in m.inputs for m in st.nodes)]
            L += chunk_loop(elem_block(st.nodes, used, []))
        else:
            # per-row scalar stage over [rows] or [rows, 1]: linear index r addresses both
            L += scalar_lines(st.nodes, st, tuple(st.iter_shape), "r")
    L.append("}")
    meta = {"family": "row", "vec": vec, "threads": T, "chunks": NCH, "streaming": streaming, "rows": nrows, "n": N,
            "rows_per_block": R}
    if not split:
        return "\n".join(L), Launch(g.fname, (-(-nrows // R), 1, 1), (T * R, 1, 1), 0, meta)

    # combine launch: one workgroup per row folds the row's S partials, then the
    # reduction's finish (mean: / N) and its epilogue, as the one-workgroup row does
    st = stages[0]
    red = st.anchor
    S = split.splits
    is_max = red.op == "max"
    C = [f'extern "C" __global__ __launch_bounds__({COMBINE_THREADS}) void {g.fname}_combine({g.params()}, '
         "const float* __restrict__ ws_p) {",
         f"  __shared__ float tj_red[1][{COMBINE_THREADS // 64}];",
         f"  const {idx_t} r = blockIdx.x;",
         "  const unsigned int tid = threadIdx.x;"]
    if scalars:
        C.append("  float " + ", ".join(g.names[id(n)] for n in scalars) + ";")
    C.append(f"  float acc = {'(-__builtin_inff())' if is_max else '0.0f'};")
    upd = "acc = fmaxf(acc, ws_p[r * {S}u + s]);" if is_max else "acc += ws_p[r * {S}u + s];"
    C.append(f"  for (unsigned int s = tid; s < {S}u; s += {COMBINE_THREADS}u) " + upd.format(S=S))
    C += _block_reduce_lines("acc", is_max, COMBINE_THREADS // 64, 0)
    C.append(f"  {g.names[id(red)]} = acc{' / ' + repr(float(N)) + 'f' if red.op == 'mean' else ''};")
    C += scalar_store(red)
    C += scalar_lines(st.nodes[st.nodes.index(red) + 1:], st, tuple(red.shape), "r", anchor=red)
    C.append("}")
    meta.update({"splits": S, "segments": split.segments, "workspace": nrows * S * 4, "ws_arg": True})
    cmeta = {"family": "row_combine", "splits": S, "rows": nrows, "ws_arg": True}
    return "\n".join(L) + "\n\n" + "\n".join(C), [
        Launch(g.fname, (nrows * S, 1, 1), (T, 1, 1), 0, meta),
        Launch(g.fname + "_combine", (nrows, 1, 1), (COMBINE_THREADS, 1, 1), 0, cmeta)]


COMBINE_THREADS = 256


def _block_reduce_lines(acc: str, is_max: bool, nwaves: int, slot: int) -> list[str]:
    """All-reduce of ``acc`` over the workgroup: wave64 DPP, then (several waves) one
    exchange through LDS slots ``tj_red[slot]`` behind one barrier."""
    out = [f"  {acc} = {'tj_wave_max' if is_max else 'tj_wave_sum'}({acc});"]
    if nwaves > 1:
        out.append(f"  if ((tid & 63u) == 0u) tj_red[{slot}][tid >> 6] = {acc};")
        out.append("  __syncthreads();")
        out.append(f"  {acc} = tj_red[{slot}][0];")
        for w in range(1, nwaves):
            comb = f"fmaxf({acc}, tj_red[{slot}][{w}])" if is_max else f"{acc} + tj_red[{slot}][{w}]"
            out.append(f"  {acc} = {comb};")
    return out


# ---------------------------------------------------------------------------
# column reductions (hip-backend rewrite of transpose -> reduce)
# ---------------------------------------------------------------------------

# A reduction over a non-last axis: the plan transposes the reduced axis last (a copy
# kernel) and reduces rows.  The ``colreduce`` kernel reads the source in place instead,
# viewed as [A, Rd, B] with the reduced axis Rd in the middle: the 64 lanes of a wave own
# 64 consecutive 16-byte vectors along B, so each row of Rd is a coalesced 1 KiB load per
# wave; the workgroup's 4 waves take interleaved rows of its slice of Rd and combine their
# partials through LDS.  Rd is split over S workgroups to reach a workgroup count set by
# the bytes the reduction streams (``col_workgroups_per_cu``; each workgroup walks at least
# COL_MIN_ROWS rows, at most COL_MAX_SPLITS splits); with S > 1 the partials go to the
# workspace as [S][A*B] and a combine launch adds them in a fixed order and runs the
# reduction's finish and epilogue: one lane per output, the S partials of 64 outputs
# spread over up to 16 waves and combined through LDS.
COL_WAVES = 4
COL_MIN_ROWS = 16
COL_MAX_SPLITS = 512


def col_workgroups_per_cu(streamed_bytes: int) -> int:
    """Workgroups per CU for a column reduction streaming ``streamed_bytes``.  Measured on
    MI355X (one box, back-to-back launches, main + combine launch in us at 1 / 2 / 4
    workgroups per CU): 512 MiB fp32 [32768, 4096] 85.7 / 79.6 / 85.2; 256 MiB fp32
    [16384, 4096] 39.7 / 42.4 / 46.4, [65536, 1024] 38.5 / 39.9 / 40.8, [32768, 2048]
    38.6 / 41.1 / 45.9, bf16 [16384, 8192] 40.1 / 42.4 / 47.0, [65536, 2048] 39.5 / 39.7 /
    40.8; 192 MiB fp32 [12288, 4096] 34.8 / 34.2 / 33.2, [24576, 2048] 40.9 / 31.5 / 32.9;
    128 MiB bf16 [16384, 4096] 36.3 / 35.1 / 24.9; 64 MiB fp32 [8192, 2048] 20.5 / 14.0 /
    14.6 (13.5 at 8).  So one per CU for about the MALL's size, two above, four below
    (inputs that fit the 256 MB MALL stay partly in it between launches and want more
    loads in flight); the boundaries sit between the measured sizes."""
    if streamed_bytes >= 448 * 2**20:
        return 2
    if streamed_bytes >= 224 * 2**20:
        return 1
    return 4


def col_layout(A: int, Rd: int, B: int, vec: int, streamed_bytes: int = 0) -> tuple[int, int, int]:
    """(column blocks per A-slice nb, rows per workgroup RS, splits S) of a column reduction
    whose inputs stream ``streamed_bytes``."""
    L = -(-B // vec)
    nb = -(-L // 64)
    base = A * nb
    forced = os.environ.get("TENSORJIT_HIP_COL_SPLITS")
    if forced and forced.isdigit():
        S = max(1, min(int(forced), Rd))
    else:
        wgs = col_workgroups_per_cu(streamed_bytes) * CU_COUNT
        S = max(1, min(-(-wgs // base), Rd // COL_MIN_ROWS, COL_MAX_SPLITS))
    RS = -(-Rd // S)
    return nb, RS, -(-Rd // RS)


def gen_colreduce(g: KernelGen) -> tuple[str, Launch | list[Launch]]:
    k = g.k
    X, t, red = k.src, k.tnode, k.anchor          # type: ignore[attr-defined]
    A, Rd, B = k.col                              # type: ignore[attr-defined]
    xnodes = k.xnodes                             # type: ignore[attr-defined]
    pos = k.nodes.index(red)
    tnodes = k.nodes[len(xnodes):pos]
    epilogue = k.nodes[pos + 1:]
    Sx = tuple(X.shape)
    dt = _kernel_dtype(k)
    vec = _vec_for(Sx[-1], A * Rd * B, dt)
    # inputs read per element of X: the folded elementwise kernel's inputs, or X itself
    xin = [n for n in k.inputs if n is X or any(n in m.inputs for m in xnodes)]
    xstr = {id(n): broadcast_strides(n.shape, Sx) for n in xin}
    streamed = sum(math.prod(n.shape) * n.dtype.itemsize for n in xin if _streamed(Sx, xstr[id(n)]))
    nt = _nt_loads(streamed)
    nb, RS, S = col_layout(A, Rd, B, vec, streamed)
    L = -(-B // vec)
    AB = A * B
    idx_t = _index_type(A * Rd * B)
    is_max = red.op == "max"
    init = "(-__builtin_inff())" if is_max else "0.0f"
    escaping = {id(o): j for j, o in enumerate(k.outputs)}
    nm = lambda n: g.names[id(n)]  # noqa: E731

    def fold(acc: str, v: str) -> str:
        return f"{acc} = fmaxf({acc}, {v});" if is_max else f"{acc} += {v};"

    def finish_lines(r: str, acc: str, ind: str) -> list[str]:
        """The reduction's value at output ``r`` from ``acc``, its epilogue, the stores."""
        out, local = [], {}
        val = f"{acc} / {float(Rd)!r}f" if red.op == "mean" else acc
        out.append(f"{ind}const float {nm(red)}_v = {val};")
        local[id(red)] = f"{nm(red)}_v"
        loaded = set()
        for n in [red] + epilogue:
            if n is not red:
                for i in n.inputs:
                    if id(i) in local or (i.op == "const" and i.shape == ()) or id(i) in loaded:
                        continue
                    off = offset_expr(r, tuple(red.shape), access_strides(i, n, tuple(red.shape)))
                    out.append(f"{ind}const float {nm(i)}_s = tj_ld({nm(i)}_p[{off}]);")
                    local[id(i)] = f"{nm(i)}_s"
                    loaded.add(id(i))
                out.append(f"{ind}const float {nm(n)}_v = {emit_expr(n, local)};")
                local[id(n)] = f"{nm(n)}_v"
            if id(n) in escaping:
                out.append(f"{ind}tj_st(out{escaping[id(n)]}_p + {r}, {nm(n)}_v);")
        return out

    ws_param = ", float* __restrict__ ws_p" if S > 1 else ""
    C = [f'extern "C" __global__ __launch_bounds__({64 * COL_WAVES}) void {g.fname}({g.params()}{ws_param}) {{',
         f"  __shared__ float tj_col[{COL_WAVES}][{64 * vec}];",
         "  const unsigned int blk = blockIdx.x, lane = threadIdx.x & 63u, w = threadIdx.x >> 6;",
         f"  const unsigned int bb = blk % {nb}u, ai = (blk / {nb}u) % {A}u, s = blk / {nb * A}u;",
         "  const unsigned int lv = bb * 64u + lane;",
         f"  const unsigned int j0 = s * {RS}u, j1 = j0 + {RS}u < {Rd}u ? j0 + {RS}u : {Rd}u;",
         f"  float acc[{vec}];",
         "#pragma unroll",
         f"  for (int q = 0; q < {vec}; ++q) acc[q] = {init};",
         f"  if (lv < {L}u) {{",
         "#pragma unroll 4",
         f"    for (unsigned int j = j0 + w; j < j1; j += {COL_WAVES}u) {{",
         f"      const {idx_t} e = (({idx_t})ai * {Rd}u + j) * {B}u + lv * {vec}u;"]
    for n in xin:
        C.append(f"      float {nm(n)}_l[{vec}];")
        C += ["      " + s for s in _load_lines(nm(n), CTYPE[n.dtype], offset_expr("e", Sx, xstr[id(n)]),
                                                inner_stride(Sx, xstr[id(n)]), vec, f"{nm(n)}_l",
                                                nt and _streamed(Sx, xstr[id(n)]))]
    C += ["#pragma unroll", f"      for (int q = 0; q < {vec}; ++q) {{"]
    local = {id(n): f"{nm(n)}_l[q]" for n in xin}
    for n in xnodes + tnodes:
        C.append(f"        const float {nm(n)}_e = {emit_expr(n, local)};")
        local[id(n)] = f"{nm(n)}_e"
        if n is X:
            local[id(t)] = local[id(X)]
    if id(t) not in local:
        local[id(t)] = local[id(X)]
    C.append("        " + fold("acc[q]", local[id(red.inputs[0])]))
    C += ["      }", "    }", "  }"]
    # the 4 waves' partials through LDS, combined by wave 0 in a fixed order
    C += ["#pragma unroll", f"  for (int q = 0; q < {vec}; ++q) tj_col[w][lane * {vec}u + q] = acc[q];",
          "  __syncthreads();", f"  if (w != 0u || lv >= {L}u) return;",
          "#pragma unroll", f"  for (int q = 0; q < {vec}; ++q) {{", "    float a = tj_col[0][lane * %du + q];" % vec]
    for w in range(1, COL_WAVES):
        C.append("    " + fold("a", f"tj_col[{w}][lane * {vec}u + q]"))
    C.append(f"    const {idx_t} r = ({idx_t})ai * {B}u + lv * {vec}u + q;")
    if S == 1:
        C += finish_lines("r", "a", "    ")
    else:
        C.append(f"    ws_p[({idx_t})s * {AB}u + r] = a;")
    C += ["  }", "}"]
    meta = {"family": "colreduce", "vec": vec, "A": A, "Rd": Rd, "B": B, "splits": S, "rows_per_wg": RS}
    main = Launch(g.fname, (nb * A * S, 1, 1), (64 * COL_WAVES, 1, 1), 0, meta)
    if S == 1:
        return "\n".join(C), main
    meta.update({"workspace": S * AB * 4, "ws_arg": True})
    CW = min(16, S)
    D = [f'extern "C" __global__ __launch_bounds__({64 * CW}) void {g.fname}_combine({g.params()}, '
         "const float* __restrict__ ws_p) {",
         f"  __shared__ float tj_cmb[{CW}][64];",
         "  const unsigned int lane = threadIdx.x & 63u, w = threadIdx.x >> 6;",
         f"  const {idx_t} r = ({idx_t})blockIdx.x * 64u + lane;",
         f"  float a = {init};",
         f"  if (r < {AB}u) {{",
         "#pragma unroll 4",
         f"    for (unsigned int s = w; s < {S}u; s += {CW}u) " + fold("a", f"ws_p[({idx_t})s * {AB}u + r]"),
         "  }",
         "  tj_cmb[w][lane] = a;",
         "  __syncthreads();",
         f"  if (w != 0u || r >= {AB}u) return;",
         "  a = tj_cmb[0][lane];"]
    D += ["  " + fold("a", f"tj_cmb[{w}][lane]") for w in range(1, CW)]
    D += finish_lines("r", "a", "  ")
    D.append("}")
    comb = Launch(g.fname + "_combine", (-(-AB // 64), 1, 1), (64 * CW, 1, 1), 0,
                  {"family": "colreduce_combine", "splits": S, "ws_arg": True, "outputs": AB})
    return "\n".join(C) + "\n\n" + "\n".join(D), [main, comb]
