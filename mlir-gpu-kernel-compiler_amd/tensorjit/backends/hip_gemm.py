"""Kernel family 3 of the hip backend: tiled MFMA GEMM with a fused epilogue.

``out = epilogue(A @ op(B))`` where ``op(B) = B^T`` when the fusion passes
folded a transpose into the matmul (``trans_b``; the ``nn.Linear`` layout),
with broadcast batch dims.  Reference template:
``tensorjit/backends/cuda_backend.py:296-429`` (64x64x16 SIMT / WMMA tiles,
single-buffered, epilogue in the store loop).

gfx950 design:

* Matrix cores: bf16 / fp16 use ``v_mfma_f32_32x32x16_{bf16,f16}`` (MI=32) or
  ``v_mfma_f32_16x16x32_{bf16,f16}`` (MI=16); fp32 uses
  ``v_mfma_f32_32x32x2f32`` / ``v_mfma_f32_16x16x4f32``.  fp32 accumulate.
* Workgroup = ``WM x WN`` waves of 64 lanes; each wave owns a
  ``(TM/WM) x (TN/WN)`` sub-tile as a grid of MI x MI accumulator blocks.
* LDS holds A as ``[TM][TK+pad]`` and B as ``[TN][TK+pad]`` (both K
  contiguous, 16-byte row padding so the 16-byte fragment reads of a wave hit
  distinct banks), double buffered: while the waves run the MFMAs of K step
  ``t`` from one buffer, the global loads of step ``t+1`` are already in
  flight into registers (issued a whole MFMA phase before they are written
  to the other buffer); one barrier per K step.
* ``trans_b`` (NT): both operands are K contiguous and load as 16-byte
  vectors straight into the LDS layout.  Plain B (NN, ``[K][N]``) loads 16
  bytes along N and is transposed on its way into LDS.
* The epilogue runs on the accumulator registers: every fused pointwise op
  (bias, gelu, residual, scale ...) is applied in fp32 and each escaping value
  is stored once, with its extra inputs read at their broadcast strides.
* Bounds checks are generated only for the edges the shape actually has.
"""
from __future__ import annotations

import math
import os

from ..ir import DType, Node
from ..runtime.autotune import MatmulConfig
from .common import access_strides, contiguous_strides, emit_expr
from .hip_kernels import KernelGen, Launch
from .hip_prelude import CTYPE

# (dtype, MI) -> (builtin, KI = K per instruction, KPL = K elements per lane, acc regs, operand vector type)
MFMA = {
    (DType.bf16, 32): ("__builtin_amdgcn_mfma_f32_32x32x16_bf16", 16, 8, 16, "tj_bf16x8"),
    (DType.bf16, 16): ("__builtin_amdgcn_mfma_f32_16x16x32_bf16", 32, 8, 4, "tj_bf16x8"),
    (DType.f16, 32): ("__builtin_amdgcn_mfma_f32_32x32x16_f16", 16, 8, 16, "tj_f16x8"),
    (DType.f16, 16): ("__builtin_amdgcn_mfma_f32_16x16x32_f16", 32, 8, 4, "tj_f16x8"),
    (DType.f32, 32): ("__builtin_amdgcn_mfma_f32_32x32x2f32", 2, 1, 16, "float"),
    (DType.f32, 16): ("__builtin_amdgcn_mfma_f32_16x16x4f32", 4, 1, 4, "float"),
}


def matmul_dims(mm: Node) -> tuple[int, int, int, bool]:
    a, b = mm.inputs
    tb = bool(mm.attrs.get("trans_b"))
    M, K = a.shape[-2], a.shape[-1]
    N = b.shape[-2] if tb else b.shape[-1]
    return M, N, K, tb


def compute_dtype(mm: Node) -> DType:
    """Operand type of the MFMA path: bf16/fp16 when both operands share it, else fp32."""
    a, b = mm.inputs
    if a.dtype == b.dtype and a.dtype in (DType.bf16, DType.f16):
        return a.dtype
    return DType.f32


def epilogue_inputs(k, epilogue: list[Node]) -> list[Node]:
    """The kernel inputs the epilogue reads, in kernel-input order.  An operand of the
    product can be one of them (``x + linear(x, w)``)."""
    used = {id(i) for n in epilogue for i in n.inputs}
    return [i for i in k.inputs if id(i) in used]


def batch_folds_into_m(mm: Node) -> bool:
    """Is ``mm`` one 2-D GEMM over (batch x M) rows: A contiguous across its batch dims
    and B shared by every batch entry (a projection of a [B, S, D] activation)?"""
    batch_shape = tuple(mm.shape[:-2])
    if not batch_shape:
        return True
    a, b = mm.inputs
    M, _, K, _ = matmul_dims(mm)
    want = tuple(s * M * K for s in contiguous_strides(batch_shape))
    return (tuple(a.shape[:-2]) == batch_shape and _batch_strides(a, batch_shape) == want
            and all(s == 0 for s in _batch_strides(b, batch_shape)))


def _folded_strides(st: tuple[int, ...], batch_shape: tuple, M: int) -> tuple[int, int] | None:
    """An epilogue input's (row, column) strides over the folded (batch x M, N) output,
    given its strides over (batch..., i, j); None when it does not fold."""
    *sb, si, sj = st
    inner = M
    for d in range(len(batch_shape) - 1, -1, -1):
        if sb[d] != si * inner:
            return None
        inner *= batch_shape[d]
    return si, sj


def config_ok(cfg: MatmulConfig, dt: DType, mm: Node | None = None) -> bool:
    """Is ``cfg`` a valid tiling for operand type ``dt`` (and for matmul ``mm`` if given)?"""
    if (dt, cfg.MI) not in MFMA:
        return False
    _, ki, _, _, _ = MFMA[(dt, cfg.MI)]
    if cfg.PERSIST and (not cfg.DIRECT or cfg.KSPLIT > 1):
        return False
    if cfg.KSPLIT > 1:
        # K split over workgroups: the plain double-buffered schedule or the skinny
        # kernel, every split an equal whole number of K steps (no K edge inside a split)
        if cfg.PINGPONG or cfg.INTERLEAVE or cfg.DIRECT or cfg.KSPLIT > 16:
            return False
        if mm is not None:
            K = matmul_dims(mm)[2]
            step = cfg.KSPLIT * (cfg.SPLIT_K * ki if cfg.SPLIT_K > 1 else cfg.TK)
            if K % step:
                return False
    if cfg.SPLIT_K > 1:
        # skinny kernel: one MI x MI tile per workgroup, K split over its waves (NT, bf16/fp16)
        ok = (dt in (DType.bf16, DType.f16) and cfg.TM == cfg.MI and cfg.TN % cfg.MI == 0
              and cfg.TN // cfg.MI <= 4 and cfg.num_warps == cfg.SPLIT_K and cfg.TK % ki == 0 and cfg.TK > 0)
        if ok and mm is not None:
            M, N, K, tb = matmul_dims(mm)
            a, b = mm.inputs
            # buffer descriptors: byte offsets and ranges in 31 bits (out-of-range marker 2^31)
            ok = (tb and M <= cfg.TM and K % 8 == 0 and a.dtype == b.dtype == dt
                  and (N + cfg.TN) * K * 2 < 2**31 and M * K * 2 < 2**31)
        return ok
    if cfg.INTERLEAVE and (cfg.PINGPONG or (cfg.TK // ki) % 2):
        return False
    if cfg.DIRECT:
        # direct-to-LDS tiles: 128-byte K rows -- 16-bit operands with TK 64 and 32x32x16
        # or 16x16x32 MFMAs, or fp32 with TK 32 and 16x16x4 MFMAs -- wave tiles whose row
        # bases are multiples of 32 (the LDS swizzle's period), 8-row DMA blocks per wave
        # and no other schedule.  fp32 tiles stop at 128x256: at 256x256 each wave's 4
        # passes of 64 MFMAs per sub-step need ~500 VGPRs, spill in the persistent form
        # and take ~80 s to compile.
        ok = (((dt in (DType.bf16, DType.f16) and cfg.TK == 64 and cfg.MI in (16, 32))
               or (dt == DType.f32 and cfg.TK == 32 and cfg.MI == 16 and cfg.TM * cfg.TN <= 128 * 256))
              and not cfg.PINGPONG
              and not cfg.INTERLEAVE and cfg.SPLIT_K == 1 and cfg.WM * cfg.WN == cfg.num_warps
              and cfg.TM % (cfg.WM * 32) == 0 and cfg.TN % (cfg.WN * 32) == 0
              and cfg.TM % (8 * cfg.num_warps) == 0 and cfg.TN % (8 * cfg.num_warps) == 0
              and 2 * (cfg.TM + cfg.TN) * 128 <= 160 * 1024
              # one K tile's DMA loads per wave fit the 6-bit vmcnt of the stage waits
              and (cfg.TM + cfg.TN) // (8 * cfg.num_warps) < 64)
        if ok and mm is not None:
            M, N, K, tb = matmul_dims(mm)
            a, b = mm.inputs
            # buffer descriptors: byte offsets (rows padded to the tile) and ranges in int32
            ok = (tb and K % cfg.TK == 0 and a.dtype == b.dtype == dt
                  and (M + cfg.TM) * K * dt.itemsize < 2**31 and (N + cfg.TN) * K * dt.itemsize < 2**31)
        if ok and cfg.PERSIST:
            # persistent tile loop: 16x16 MFMAs, 4 waves, a multiple of 8 workgroups
            # (XCD order), an epilogue staging array of its own beside the two stages,
            # wave columns a power of two (a staged output row splits evenly over the 64
            # lanes), whole tiles (no edges), an even number of at least 4 K tiles, and a
            # batch only where it folds into M
            cols = cfg.TN // cfg.WN
            ok = (cfg.MI == 16 and cfg.num_warps == 4 and cfg.PERSIST % XCDS == 0 and cols >= 64
                  and cols & (cols - 1) == 0
                  and 2 * (cfg.TM + cfg.TN) * 128 + 4 * 16 * cols * 4 <= 160 * 1024)
            if ok and mm is not None:
                M, N, K, _ = matmul_dims(mm)
                M *= math.prod(mm.shape[:-2])
                ok = (batch_folds_into_m(mm) and M % cfg.TM == 0 and N % cfg.TN == 0 and K % (2 * cfg.TK) == 0
                      and K >= 4 * cfg.TK and M * N < 2**31 and M * K * dt.itemsize < 2**31)
        return ok
    if cfg.PINGPONG:
        ks = cfg.TK // ki
        if cfg.num_warps % 2 or cfg.PINGPONG > 3 or (cfg.PINGPONG == 3 and ks % 2):
            return False
        # ping-pong holds accumulators, one step's fragments and its staging registers at
        # once; past ~216 of the 256 VGPRs (addresses need the rest) it spills
        tmw, tnw = cfg.TM // (cfg.WM * cfg.MI), cfg.TN // (cfg.WN * cfg.MI)
        acc = tmw * tnw * cfg.MI * cfg.MI // 64
        frag = (ks // 2 if cfg.PINGPONG == 3 else ks) * (tmw + tnw) * 4
        sets = 2 if cfg.PINGPONG == 2 else 1
        stage = sets * (cfg.TM + cfg.TN) * cfg.TK * dt.itemsize // (cfg.num_warps * 64 * 4)
        if acc + frag + stage > 216:
            return False
    return (cfg.WM * cfg.WN == cfg.num_warps and cfg.TM % (cfg.WM * cfg.MI) == 0
            and cfg.TN % (cfg.WN * cfg.MI) == 0 and cfg.TK % ki == 0 and cfg.TK > 0)


SKINNY_A_CHUNK = 256   # K elements of A per LDS chunk of the decode GEMM (128-1024; 16 rows x 2*chunk bytes)


def gen_skinny_matmul(g: KernelGen, cfg: MatmulConfig) -> tuple[str, Launch]:
    """Decode-shaped GEMM (M <= MI, NT layout): HBM-bound on streaming B.

    A workgroup owns TN = NT * MI output columns; its ``SPLIT_K`` waves each take a
    contiguous K slice.  The MFMA operands need no LDS: with K-contiguous A and B,
    lane ``l``'s 16-byte load of row ``l % MI`` at k-chunk ``l / MI`` is exactly its
    operand register, so each wave streams B straight from HBM into the matrix core
    and reuses each A fragment for its NT column tiles.  The loads of ``D = TK / KI``
    K-steps are in flight ahead of the MFMAs (a ring of D register sets, the whole
    slice unrolled).  Partial tiles are summed through LDS (one barrier), then the
    epilogue runs per element.

    A, which every workgroup reads whole (from L2), goes through LDS when the slices
    allow it (16x16x32 MFMAs, whole 256-deep chunks, one workgroup along K): a fragment
    load touches 16 rows x 64 bytes, and those scattered A loads on top of B's cost
    16 x 8192 x 8192 3.5 us (23.5 vs 20.0 us with A's loads replaced by 1 KiB runs).
    Each wave copies its slice of A 256 k at a time with ``buffer_load ... lds`` as
    2 rows x 512 bytes per instruction into its own two chunk buffers, and reads the
    fragments back with ``ds_read_b128``; 16-byte chunk q of row r is stored at slot
    q ^ r, so the 16 rows a fragment read touches sit in 16 different bank groups."""
    k = g.k
    mm = k.anchor
    a, b = mm.inputs
    M, N, K, tb = matmul_dims(mm)
    dt = compute_dtype(mm)
    builtin, KI, KPL, NACC, opvec = MFMA[(dt, cfg.MI)]
    MI, SK = cfg.MI, cfg.SPLIT_K
    NT = cfg.TN // MI
    TN = cfg.TN
    THREADS = 64 * SK
    U = cfg.TK // KI                                 # MFMA steps per unrolled iteration
    out_shape = tuple(mm.shape)
    batch_shape = out_shape[:-2]
    batch = math.prod(batch_shape) if batch_shape else 1
    S = cfg.KSPLIT                                   # workgroups along K (partials summed by a 2nd launch)
    Kw = K // S                                      # this workgroup's K range
    steps_total = -(-Kw // KI)
    steps_per_wave = -(-steps_total // SK)
    k_guard = steps_per_wave * SK * KI != Kw          # some slice runs past the workgroup's K range
    A, B = g.names[id(a)], g.names[id(b)]
    epilogue = [n for n in k.nodes if n is not mm]
    fname = g.fname
    ws_param = ", float* __restrict__ ws_p" if S > 1 else ""
    L = [f'extern "C" __global__ __launch_bounds__({THREADS}) void {fname}({g.params()}{ws_param}) {{']
    L.append(f"  __shared__ float red[{SK}][{MI}][{TN + 1}];")
    L.append("  const unsigned int tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;")
    L.append(f"  const unsigned int n0 = blockIdx.x * {TN}u;")
    bidx: list[str] = []
    if batch_shape:
        L.append("  const unsigned int bi = blockIdx.z;")
        rem = "bi"
        for d, cst in enumerate(contiguous_strides(batch_shape)):
            v = f"b{d}"
            if d == len(batch_shape) - 1:
                L.append(f"  const unsigned int {v} = {rem};")
            else:
                L.append(f"  const unsigned int {v} = {rem} / {cst}u, br{d} = {rem} % {cst}u;")
                rem = f"br{d}"
            bidx.append(v)

        def boff(t: Node) -> str:
            terms = [f"{v} * {s}u" for v, s in zip(bidx, _batch_strides(t, batch_shape)) if s]
            return " + ".join(terms) if terms else "0u"

        L.append(f"  const {CTYPE[a.dtype]}* __restrict__ Ab = {A}_p + ({boff(a)});")
        L.append(f"  const {CTYPE[b.dtype]}* __restrict__ Bb = {B}_p + ({boff(b)});")
    else:
        L.append(f"  const {CTYPE[a.dtype]}* __restrict__ Ab = {A}_p;")
        L.append(f"  const {CTYPE[b.dtype]}* __restrict__ Bb = {B}_p;")
    # Operands come through buffer descriptors: a lane whose row is past M or N, or
    # whose K position is past its slice, gets an offset beyond the descriptor's range
    # and reads zeros -- no branch around any load, so the loads of D K-steps stay in
    # flight ahead of the MFMAs (a ring of D register sets, fully unrolled).
    OOB = 0x80000000
    L.append(f"  const unsigned int row = lane % {MI}u, kofs = (lane / {MI}u) * {KPL}u;")
    L.append(f"  const __amdgpu_buffer_rsrc_t rsA = __builtin_amdgcn_make_buffer_rsrc((void*)Ab, (short)0, {M * K * 2}, 0x00020000);")
    L.append(f"  const __amdgpu_buffer_rsrc_t rsB = __builtin_amdgcn_make_buffer_rsrc((void*)Bb, (short)0, {N * K * 2}, 0x00020000);")
    # the K slice of wave w in workgroup b is (w + b) mod SK: at any moment the
    # workgroups read different parts of A (which every workgroup reads whole) instead
    # of all requesting the same lines (27.7 vs 30.5 us for 16 x 8192 x 8192, TN 32)
    L.append(f"  const unsigned int kw = {'blockIdx.y * ' + str(Kw) + 'u + ' if S > 1 else ''}"
             f"((wave + blockIdx.x) % {SK}u) * {steps_per_wave * KI}u;")
    kmax = f"{Kw}u" if S == 1 else f"(blockIdx.y + 1u) * {Kw}u"
    L.append(f"  const unsigned int kend = {kmax} < kw + {steps_per_wave * KI}u ? {kmax} : kw + {steps_per_wave * KI}u;")
    L.append(f"  const unsigned int offA = row < {M}u ? (row * {K}u + kw + kofs) * 2u : {OOB}u;")
    L.append(f"  unsigned int offB[{NT}];")
    L.append("#pragma unroll")
    L.append(f"  for (int t = 0; t < {NT}; ++t) {{")
    L.append(f"    const unsigned int col = n0 + t * {MI}u + row;")
    L.append(f"    offB[t] = col < {N}u ? (col * {K}u + kw + kofs) * 2u : {OOB}u;")
    L.append("  }")
    acc_t = "tj_f32x16" if NACC == 16 else "tj_f32x4"
    L.append(f"  {acc_t} acc[{NT}];")
    L.append("#pragma unroll")
    L.append(f"  for (int t = 0; t < {NT}; ++t) acc[t] = ({acc_t})(0.0f);")
    D = max(1, min(U, steps_per_wave))
    L.append(f"  tj_u32x4 ra[{D}], rb[{D}][{NT}];")
    CH = SKINNY_A_CHUNK // KI                     # MFMA steps per A chunk
    cb = MI * SKINNY_A_CHUNK * 2                  # bytes of one chunk buffer (16 rows x 512 B)
    lds_a = (MI == 16 and S == 1 and not k_guard and steps_per_wave % CH == 0 and dt.itemsize == 2
             and 2 * SK * cb + SK * MI * (TN + 1) * 4 <= 160 * 1024)
    n_chunks = steps_per_wave // CH
    row_b = SKINNY_A_CHUNK * 2                    # bytes of one row of a chunk
    n_dma = cb // 1024                            # 1 KiB copy instructions per chunk
    if lds_a:
        L.append(f"  __shared__ __attribute__((aligned(1024))) char Ach0[{SK * cb}];")
        L.append(f"  __shared__ __attribute__((aligned(1024))) char Ach1[{SK * cb}];")
        L.append("  const unsigned int wv = __builtin_amdgcn_readfirstlane(wave);")
        # DMA lane offsets: instruction gq fills chunk bytes [1024 gq, 1024 gq + 1024),
        # lane slot j of row r fetching 16-byte chunk j ^ r; rows past M read zeros
        L.append(f"  unsigned int voA[{n_dma}];")
        L.append("#pragma unroll")
        L.append(f"  for (int gq = 0; gq < {n_dma}; ++gq) {{")
        L.append(f"    const unsigned int byte = gq * 1024u + lane * 16u, r = byte / {row_b}u, j = (byte % {row_b}u) / 16u;")
        L.append(f"    voA[gq] = r < {M}u ? (r * {K}u + kw + ((j ^ r) * 8u)) * 2u : {OOB}u;")
        L.append("  }")
        # fragment read: row lane % 16, logical chunk 4 s + lane / 16 at slot chunk ^ row
        L.append("  const unsigned int fr = lane & 15u, fc = lane >> 4;")

    def a_dma(chunk: int) -> list[str]:
        buf = f"Ach{chunk % 2}"
        return [f"  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsA, (__attribute__((address_space(3))) void*)"
                f"({buf} + wv * {cb}u + {gq * 1024}u), 16, voA[{gq}], {chunk * row_b}, 0, 0);"
                for gq in range(n_dma)]

    def load(step: int) -> list[str]:
        slot, byte = step % D, step * KI * 2
        # a lane whose 16-byte chunk starts at or past the end of the slice reads zeros
        # (slices are whole multiples of the chunk, so no chunk straddles the end)
        kin = f"kw + {step * KI}u + kofs < kend" if k_guard else None
        out = []
        if lds_a:
            chunk, sc = divmod(step, CH)
            if sc == 0 and chunk + 1 < n_chunks:
                # the next chunk goes into the buffer the chunk before this one used:
                # its fragment reads are done once no LDS read is outstanding
                out.append(f"  __builtin_amdgcn_s_waitcnt({_lgkmcnt_only(0)});")
                out += a_dma(chunk + 1)
            out.append(f"  ra[{slot}] = *(const tj_u32x4*)(Ach{chunk % 2} + wv * {cb}u + fr * {row_b}u"
                       f" + (({4 * sc}u + fc) ^ fr) * 16u);")
        else:
            va = f"offA + {byte}u" if not kin else f"({kin}) ? offA + {byte}u : {OOB}u"
            out.append(f"  ra[{slot}] = __builtin_bit_cast(tj_u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsA, {va}, 0, 0));")
        for t in range(NT):
            vb = f"offB[{t}] + {byte}u" if not kin else f"({kin}) ? offB[{t}] + {byte}u : {OOB}u"
            out.append(f"  rb[{slot}][{t}] = __builtin_bit_cast(tj_u32x4, "
                       f"__builtin_amdgcn_raw_buffer_load_b128(rsB, {vb}, 0, 0));")
        return out

    # The written order is kept (sched_barrier between steps): left alone, the scheduler
    # sinks every load next to its MFMA to save registers, leaving ~2 K-steps in flight.
    if lds_a:
        L += a_dma(0)
    for step in range(min(D, steps_per_wave)):
        L += load(step)
    L.append("  __builtin_amdgcn_sched_barrier(0);")
    for step in range(steps_per_wave):
        slot = step % D
        for t in range(NT):
            L.append(f"  acc[{t}] = {builtin}(__builtin_bit_cast({opvec}, ra[{slot}]), "
                     f"__builtin_bit_cast({opvec}, rb[{slot}][{t}]), acc[{t}], 0, 0, 0);")
        if step + D < steps_per_wave:
            L += load(step + D)
        L.append("  __builtin_amdgcn_sched_barrier(0);")
    if MI == 32:
        row_of, col_of = "(r / 4) * 8 + (lane / 32u) * 4 + (r % 4)", "lane % 32u"
    else:
        row_of, col_of = "(lane / 16u) * 4 + r", "lane % 16u"
    L.append("#pragma unroll")
    L.append(f"  for (int t = 0; t < {NT}; ++t)")
    L.append("#pragma unroll")
    L.append(f"    for (int r = 0; r < {NACC}; ++r) red[wave][{row_of}][t * {MI}u + {col_of}] = acc[t][r];")
    L.append("  __syncthreads();")
    L.append(f"  for (unsigned int e = tid; e < {MI * TN}u; e += {THREADS}u) {{")
    L.append(f"    const unsigned int i = e / {TN}u, jj = e % {TN}u, j = n0 + jj;")
    L.append(f"    if (i >= {M}u || j >= {N}u) continue;")
    L.append("    float s = 0.0f;")
    L.append("#pragma unroll")
    L.append(f"    for (int w = 0; w < {SK}; ++w) s += red[w][i][jj];")
    if S > 1:
        # this workgroup's K-range partial; the second launch sums and applies the epilogue
        bi = "bi" if batch_shape else "0u"
        L += [f"    ws_p[(({bi} * {S}u + blockIdx.y) * {M}u + i) * {N}u + j] = s;", "  }", "}"]
        grid = (-(-N // TN), S, batch)
        meta = {"family": "matmul_skinny", "config": cfg.as_dict(), "dtype": dt.value, "M": M, "N": N, "K": K,
                "batch": batch, "trans_b": tb, "lds_bytes": SK * MI * (TN + 1) * 4, "flops": 2.0 * M * N * K * batch,
                "workspace": batch * S * M * N * 4, "ws_arg": True}
        epi_inputs = epilogue_inputs(k, epilogue)
        src2, sum_launch = gen_ksplit_sum(g, k, mm, epilogue, epi_inputs, out_shape, batch_shape, M, N, S, fname)
        return "\n".join(L) + "\n\n" + src2, [Launch(fname, grid, (THREADS, 1, 1), 0, meta), sum_launch]
    L.append(f"    const float {g.names[id(mm)]} = s;")
    local = {id(mm): g.names[id(mm)]}
    full_idx = list(bidx) + ["i", "j"]
    for n in epilogue_inputs(k, epilogue):
        consumer = next((c for c in epilogue if n in c.inputs), epilogue[0] if epilogue else mm)
        st = access_strides(n, consumer, out_shape)
        terms = [v if s_ == 1 else f"{v} * {s_}u" for v, s_ in zip(full_idx, st) if s_]
        L.append(f"    const float {g.names[id(n)]}_e = tj_ld({g.names[id(n)]}_p[{' + '.join(terms) if terms else '0u'}]);")
        local[id(n)] = f"{g.names[id(n)]}_e"
    for n in epilogue:
        L.append(f"    const float {g.names[id(n)]} = {emit_expr(n, local)};")
        local[id(n)] = g.names[id(n)]
    obase = f"bi * {M * N}u + " if batch_shape else ""
    for jj, o in enumerate(k.outputs):
        L.append(f"    tj_st(out{jj}_p + {obase}i * {N}u + j, {local[id(o)]});")
    L.append("  }")
    L.append("}")
    grid = (-(-N // TN), 1, batch)
    meta = {"family": "matmul_skinny", "config": cfg.as_dict(), "dtype": dt.value, "M": M, "N": N, "K": K,
            "batch": batch, "trans_b": tb, "lds_bytes": SK * MI * (TN + 1) * 4 + (2 * SK * cb if lds_a else 0), "flops": 2.0 * M * N * K * batch}
    return "\n".join(L), Launch(fname, grid, (THREADS, 1, 1), 0, meta)


def _batch_strides(t: Node, batch_shape: tuple) -> tuple[int, ...]:
    """Strides of t's leading (batch) dims over the output's batch shape (0 = broadcast)."""
    cs = contiguous_strides(t.shape)
    lead = len(batch_shape) - (len(t.shape) - 2)
    st = [0] * lead
    for d in range(len(t.shape) - 2):
        st.append(0 if t.shape[d] == 1 and batch_shape[lead + d] != 1 else cs[d])
    return tuple(st)


def _run_lines(g, k, mm, epilogue, epi_inputs, out_shape, bidx, batch_shape, M, N, ve, cs,
               pre: dict | None = None, strides: dict | None = None) -> list[str]:
    """Epilogue of one run of ``ve`` consecutive outputs at (i, j) (both defined by the
    caller), the accumulators being ``cs`` with ``q`` the position in the run: extra
    inputs loaded as vectors where contiguous (or taken from the caller's preloaded
    arrays ``pre[id(input)]``), outputs stored as vectors.  ``strides[id(input)]``
    overrides an input's strides over (batch..., i, j)."""
    L = []
    full_idx = list(bidx) + ["i", "j"]
    L.append(f"    float acc_v[{ve}];")
    L.append("#pragma unroll")
    L.append(f"    for (int q = 0; q < {ve}; ++q) acc_v[q] = {cs};")
    local = {id(mm): "acc_v[q]"}
    for n in epi_inputs:
        if pre and id(n) in pre:
            local[id(n)] = f"{pre[id(n)]}[q]"
            continue
        consumer = next((c for c in epilogue if n in c.inputs), epilogue[0] if epilogue else mm)
        st = strides[id(n)] if strides else access_strides(n, consumer, out_shape)
        terms = [v if s_ == 1 else f"{v} * {s_}u" for v, s_ in zip(full_idx, st) if s_]
        off = " + ".join(terms) if terms else "0u"
        nm = g.names[id(n)]
        L.append(f"    float {nm}_v[{ve}];")
        inner = st[-1]
        if ve > 1 and inner == 1 and 16 // n.dtype.itemsize == ve:
            L.append(f"    tj_ldv({nm}_p + ({off}), {nm}_v);")
        elif inner == 0:
            L.append(f"    {{ const float s_ = tj_ld({nm}_p[{off}]); for (int q = 0; q < {ve}; ++q) {nm}_v[q] = s_; }}")
        else:
            L.append(f"    for (int q = 0; q < {ve}; ++q) {nm}_v[q] = tj_ld({nm}_p[({off}) + q * {inner}u]);")
        local[id(n)] = f"{nm}_v[q]"
    for jj in range(len(k.outputs)):
        L.append(f"    float o{jj}_v[{ve}];")
    L.append("#pragma unroll")
    L.append(f"    for (int q = 0; q < {ve}; ++q) {{")
    for n in epilogue:
        L.append(f"      const float {g.names[id(n)]} = {emit_expr(n, local)};")
        local[id(n)] = g.names[id(n)]
    for jj, o in enumerate(k.outputs):
        L.append(f"      o{jj}_v[q] = {local[id(o)]};")
    L.append("    }")
    obase = f"bi * {M * N}u + " if batch_shape else ""
    for jj in range(len(k.outputs)):
        dst = f"out{jj}_p + {obase}i * {N}u + j"
        L.append(f"    tj_stv({dst}, o{jj}_v);" if ve > 1 else f"    tj_st({dst}, o{jj}_v[0]);")
    return L


def staged_epilogue_lines(g, k, mm, epilogue, epi_inputs, out_shape, bidx, batch_shape, M, N, BM, BN, WM, WN, MI,
                          TMW, TNW, NACC, THREADS, lds_bytes, guard_m, guard_n, idx_t):
    """Epilogue through LDS: the accumulators are written to LDS in row-major order
    (``P`` passes of BM/P rows when the tile does not fit at once), then every lane
    processes 16-byte runs of a row, so the epilogue's extra inputs (bias, residual)
    are read and its outputs written as coalesced vectors instead of one element per
    lane per accumulator register.  Returns None when no pass size fits in LDS."""
    out_dt = k.outputs[0].dtype
    if any(o.dtype != out_dt for o in k.outputs):
        return None
    ve = 16 // out_dt.itemsize if N % (16 // out_dt.itemsize) == 0 else 1
    ldc = BN + 4
    P = None
    for cand in range(1, TMW + 1):
        if TMW % cand == 0 and (BM // cand) * ldc * 4 <= lds_bytes:
            P = cand
            break
    if P is None:
        return None
    XP = TMW // P
    rows = BM // P
    if MI == 32:
        row_of, col_of = "(r / 4) * 8 + (lane / 32u) * 4 + (r % 4)", "lane % 32u"
    else:
        row_of, col_of = "(lane / 16u) * 4 + r", "lane % 16u"
    chunks = rows * (BN // ve)
    L = ["  float* Cs = (float*)tj_lds;"]
    full_idx = list(bidx) + ["i", "j"]
    for p in range(P):
        L.append("  __syncthreads();")
        L.append("#pragma unroll")
        L.append(f"  for (int x = {p * XP}; x < {(p + 1) * XP}; ++x)")
        L.append("#pragma unroll")
        L.append(f"  for (int y = 0; y < {TNW}; ++y)")
        L.append("#pragma unroll")
        L.append(f"  for (int r = 0; r < {NACC}; ++r)")
        L.append(f"    Cs[(wm * {XP * MI}u + (x - {p * XP}) * {MI}u + {row_of}) * {ldc}u + wn * {BN // WN}u + y * {MI}u + "
                 f"{col_of}] = acc[x][y][r];")
        L.append("  __syncthreads();")
        L.append("#pragma unroll")
        L.append(f"  for (unsigned int c = tid; c < {chunks}u; c += {THREADS}u) {{")
        L.append(f"    const unsigned int lr = c / {BN // ve}u, cc = (c % {BN // ve}u) * {ve}u;")
        L.append(f"    const {idx_t} i = m0 + (lr / {XP * MI}u) * {BM // WM}u + {p * XP * MI}u + lr % {XP * MI}u;")
        L.append(f"    const {idx_t} j = n0 + cc;")
        conds = ([f"i < {M}u"] if guard_m else []) + ([f"j < {N}u"] if guard_n else [])
        if conds:
            L.append(f"    if (!({' && '.join(conds)})) continue;")
        L += _run_lines(g, k, mm, epilogue, epi_inputs, out_shape, bidx, batch_shape, M, N, ve,
                        f"Cs[lr * {ldc}u + cc + q]")
        L.append("  }")
    return L


def direct_staged_epilogue_lines(g, k, mm, epilogue, epi_inputs, out_shape, bidx, batch_shape, M, N, BM, BN, WM, WN,
                                 TMW, TNW, NACC, guard_m, guard_n, idx_t, cfg) -> list[str] | None:
    """Staged epilogue of the direct-to-LDS schedule.  The four K-stage arrays are free
    once every wave has finished its last fragment reads (one barrier); wave w then
    owns array w and stages its sub-tile through it 32 rows (one 32x32 or two 16x16
    MFMA row blocks) at a time, with no further workgroup barriers: a wave's LDS
    accesses complete in order.  Each pass turns the MFMA layout into 16-byte runs of
    output rows, as in the shared staged epilogue.  Returns None where the arrays do
    not fit a pass."""
    out_dt = k.outputs[0].dtype
    if cfg.num_warps != 4 or any(o.dtype != out_dt for o in k.outputs):
        return None
    MI = cfg.MI
    ve = 16 // out_dt.itemsize if N % (16 // out_dt.itemsize) == 0 else 1
    cols = TNW * MI
    ldc = cols + 4
    if 32 * ldc * 4 > min(BM, BN) * 128 or cols % ve or (TMW * MI) % 32:
        return None
    per_row = cols // ve
    L = ["  __syncthreads();",
         "  float* Cw = (float*)(wave == 0u ? As0 : wave == 1u ? As1 : wave == 2u ? Bs0 : Bs1);"]
    tiles = 32 // MI                      # MFMA row blocks per 32-row pass
    for p_ in range(TMW // tiles):
        for xl in range(tiles):
            x = p_ * tiles + xl
            row = ("(r / 4) * 8 + (lane / 32u) * 4 + (r % 4)" if MI == 32
                   else f"{xl * 16}u + (lane / 16u) * 4 + r")
            L.append("#pragma unroll")
            L.append(f"  for (int y = 0; y < {TNW}; ++y)")
            L.append("#pragma unroll")
            L.append(f"  for (int r = 0; r < {NACC}; ++r)")
            L.append(f"    Cw[({row}) * {ldc}u + y * {MI}u + lane % {MI}u] = acc[{x}][y][r];")
        L.append("#pragma unroll")
        L.append(f"  for (unsigned int c = lane; c < {32 * per_row}u; c += 64u) {{")
        L.append(f"    const unsigned int lr = c / {per_row}u, cc = (c % {per_row}u) * {ve}u;")
        L.append(f"    const {idx_t} i = m0 + wm * {BM // WM}u + {p_ * 32}u + lr;")
        L.append(f"    const {idx_t} j = n0 + wn * {BN // WN}u + cc;")
        conds = ([f"i < {M}u"] if guard_m else []) + ([f"j < {N}u"] if guard_n else [])
        if conds:
            L.append(f"    if (!({' && '.join(conds)})) continue;")
        L += _run_lines(g, k, mm, epilogue, epi_inputs, out_shape, bidx, batch_shape, M, N, ve,
                        f"Cw[lr * {ldc}u + cc + q]")
        L.append("  }")
    return L


XCDS = 8   # MI355X: workgroups are dispatched round-robin over 8 XCDs, each with its own L2


def tile_order_lines(ntm: int, ntn: int, group_m: int, BM: int, BN: int, vid: str | None = None,
                     names: tuple[str, str] = ("m0", "n0"), sfx: str = "") -> list[str]:
    """(m0, n0) of this workgroup's output tile.

    The grid is launched as (ntn, ntm).  Workgroup ``w`` (x-fastest linear id) runs on XCD
    ``w % 8``; re-numbering tiles so that XCD ``x`` owns the contiguous range
    ``[x*T/8, (x+1)*T/8)`` of a grouped order (``group_m`` tile rows walked column by
    column) makes the workgroups that share an L2 work on a compact block of tiles, so
    they share A row panels and B column panels in that L2 instead of each XCD streaming
    every panel from HBM / MALL.  ``vid``: the linear id as an expression instead (a
    persistent workgroup's virtual id, ``blockIdx.x + i * G`` with G a multiple of 8, so
    it stays on its XCD); ``names`` / ``sfx`` name the results and temporaries."""
    T = ntm * ntn
    m, n = names
    if group_m <= 0 or T < 2 * XCDS or T % XCDS:
        if vid is None:
            return [f"  const unsigned int {m} = blockIdx.y * {BM}u, {n} = blockIdx.x * {BN}u;"]
        return [f"  const unsigned int {m} = ({vid}) / {ntn}u * {BM}u, {n} = ({vid}) % {ntn}u * {BN}u;"]
    gm = min(group_m, ntm)
    per_group = gm * ntn
    w, t, g, first, gsz, r = (f"{v}{sfx}_" for v in ("w", "t", "g", "first", "gsz", "r"))
    wid = f"blockIdx.y * {ntn}u + blockIdx.x" if vid is None else vid
    return [
        f"  const unsigned int {w} = {wid};",
        f"  const unsigned int {t} = ({w} % {XCDS}u) * {T // XCDS}u + {w} / {XCDS}u;",
        f"  const unsigned int {g} = {t} / {per_group}u, {first} = {g} * {gm}u;",
        f"  const unsigned int {gsz} = ({ntm}u - {first}) < {gm}u ? ({ntm}u - {first}) : {gm}u;",
        f"  const unsigned int {r} = {t} % {per_group}u;",
        f"  const unsigned int {m} = ({first} + {r} % {gsz}) * {BM}u, {n} = ({r} / {gsz}) * {BN}u;",
    ]


def gen_matmul(g: KernelGen, cfg: MatmulConfig, suffix: str = "") -> tuple[str, Launch]:
    """GEMM kernel for ``g``'s matmul-anchored kernel under tile config ``cfg``.  When every
    output is 16-bit, the epilogue's gelu is ``tj_gelu16`` (erf by A&S 7.1.25, error far
    below the output's rounding): in an MFMA-bound kernel the epilogue's VALU work shows
    (bf16 [8192, 11008] up-projection + gelu 536 -> 522 us, 8192^3 + bias + gelu 691 -> 683)."""
    src, launches = _gen_matmul(g, cfg, suffix)
    if all(o.dtype in (DType.bf16, DType.f16) for o in g.k.outputs):
        src = src.replace("tj_gelu(", "tj_gelu16(")
    return src, launches


def _gen_matmul(g: KernelGen, cfg: MatmulConfig, suffix: str = "") -> tuple[str, Launch]:
    k = g.k
    mm = k.anchor
    a, b = mm.inputs
    M, N, K, tb = matmul_dims(mm)
    out_shape = tuple(mm.shape)
    batch_shape = out_shape[:-2]
    batch = math.prod(batch_shape) if batch_shape else 1
    dt = compute_dtype(mm)
    if not config_ok(cfg, dt, mm):
        raise ValueError(f"matmul config {cfg} is not valid for {dt.value} {M}x{N}x{K}")
    if cfg.SPLIT_K > 1:
        return gen_skinny_matmul(g, cfg)
    builtin, KI, KPL, NACC, opvec = MFMA[(dt, cfg.MI)]
    BM, BN, BK, MI = cfg.TM, cfg.TN, cfg.TK, cfg.MI
    WM, WN = cfg.WM, cfg.WN
    THREADS = 64 * cfg.num_warps
    TMW, TNW = BM // WM // MI, BN // WN // MI
    lds_t = CTYPE[dt] if dt != DType.f32 else "float"
    esz = dt.itemsize
    dvec = "tj_f32x4" if dt == DType.f32 else opvec      # a direct-to-LDS fragment read: 16 bytes
    VK = 16 // esz                 # elements per 16-byte global load
    PAD = VK                       # 16 bytes of row padding
    LDK = BK + PAD
    fname = g.fname + suffix

    a_vec = a.dtype == dt and K % VK == 0
    if tb:
        b_vec = b.dtype == dt and K % VK == 0
    else:
        b_vec = b.dtype == dt and N % VK == 0
    guard_m, guard_n, guard_k = M % BM != 0, N % BN != 0, K % BK != 0
    KT = -(-K // BK)

    A, B = g.names[id(a)], g.names[id(b)]
    epilogue = [n for n in k.nodes if n is not mm]
    idx_t = "unsigned long" if batch * M * N >= 2**31 or batch * max(M, N) * K >= 2**31 else "unsigned int"

    epi_st = None
    epi_inputs = epilogue_inputs(k, epilogue)
    if cfg.PERSIST:
        # one 2-D GEMM over (batch x M) rows; an epilogue input that does not fold the same
        # way (or outputs of mixed dtypes) keeps the one-tile-per-workgroup kernel
        epi_st = {}
        for n in epi_inputs:
            consumer = next((c for c in epilogue if n in c.inputs), epilogue[0] if epilogue else mm)
            epi_st[id(n)] = _folded_strides(access_strides(n, consumer, out_shape), batch_shape, M)
        if any(v is None for v in epi_st.values()) or any(o.dtype != k.outputs[0].dtype for o in k.outputs):
            epi_st = None

    S = cfg.KSPLIT
    ws_param = ", float* __restrict__ ws_p" if S > 1 else ""
    L = [f'extern "C" __global__ __launch_bounds__({THREADS}) void {fname}({g.params()}{ws_param}) {{']
    a_bytes = 2 * BM * LDK * esz
    lds_bytes = a_bytes + 2 * BN * LDK * esz
    if not cfg.DIRECT:
        L.append(f"  __shared__ __attribute__((aligned(16))) char tj_lds[{lds_bytes}];")
        L.append(f"  {lds_t} (*As)[{BM}][{LDK}] = ({lds_t} (*)[{BM}][{LDK}])tj_lds;")
        L.append(f"  {lds_t} (*Bs)[{BN}][{LDK}] = ({lds_t} (*)[{BN}][{LDK}])(tj_lds + {a_bytes});")
    L.append("  const unsigned int tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;")
    L.append(f"  const unsigned int wm = wave / {WN}u, wn = wave % {WN}u;")
    ntm, ntn = -(-M // BM), -(-N // BN)
    if epi_st is None:
        L += tile_order_lines(ntm, ntn, cfg.GROUP_M, BM, BN)
    # batch offsets (none when the batch folds into the rows of a persistent kernel)
    if batch_shape and epi_st is None:
        L.append(f"  const {idx_t} bi = blockIdx.z / {S}u;" if S > 1 else f"  const {idx_t} bi = blockIdx.z;")
        bst = contiguous_strides(batch_shape)
        bidx = []
        rem = "bi"
        for d, (s, cst) in enumerate(zip(batch_shape, bst)):
            v = f"b{d}"
            if d == len(batch_shape) - 1:
                L.append(f"  const {idx_t} {v} = {rem};")
            else:
                L.append(f"  const {idx_t} {v} = {rem} / {cst}u;")
                L.append(f"  const {idx_t} br{d} = {rem} % {cst}u;")
                rem = f"br{d}"
            bidx.append(v)

        def boff(t: Node) -> str:
            st = _batch_strides(t, batch_shape)
            terms = [f"{v} * {s}u" for v, s in zip(bidx, st) if s]
            return " + ".join(terms) if terms else "0u"

        L.append(f"  const {CTYPE[a.dtype]}* __restrict__ Ab = {A}_p + ({boff(a)});")
        L.append(f"  const {CTYPE[b.dtype]}* __restrict__ Bb = {B}_p + ({boff(b)});")
    else:
        bidx = []
        L.append(f"  const {CTYPE[a.dtype]}* __restrict__ Ab = {A}_p;")
        L.append(f"  const {CTYPE[b.dtype]}* __restrict__ Bb = {B}_p;")

    if epi_st is not None:
        M *= batch
        ntm = M // BM
        pre, body, stores, early = persistent_epilogue_lines(g, k, mm, epilogue, epi_inputs, out_shape, M, N, BM,
                                                             BN, WM, WN, TMW, TNW, epi_st)
        T = ntm * ntn
        G = min(cfg.PERSIST, T)
        persist = {"G": G, "T": T, "K": K, "BM": BM, "BN": BN, "ntm": ntm, "ntn": ntn, "group_m": cfg.GROUP_M,
                   "pre": pre, "epi": body, "stores": stores, "k1_early": early}
        L += direct_loop_lines(cfg, M, N, K, BM, BN, TMW, TNW, KT, dvec, builtin, persist, esz)
        L.append("}")
        lds = 2 * (BM + BN) * 128 + cfg.num_warps * 16 * TNW * MI * 4
        meta = {"family": "matmul", "config": cfg.as_dict(), "dtype": dt.value, "M": M // batch, "N": N, "K": K,
                "batch": batch, "trans_b": tb, "lds_bytes": lds, "flops": 2.0 * M * N * K,
                "epilogue": "lds-staged", "persistent": G}
        return "\n".join(L), Launch(fname, (G, 1, 1), (THREADS, 1, 1), 0, meta)
    if cfg.DIRECT:
        L += direct_loop_lines(cfg, M, N, K, BM, BN, TMW, TNW, KT, dvec, builtin, esz=esz)
        return _finish_matmul(L, g, k, mm, epilogue, out_shape, bidx, batch_shape, M, N, K, BM, BN, WM, WN, MI, TMW,
                              TNW, NACC, THREADS, 0, guard_m, guard_n, idx_t, cfg, dt, tb, batch, fname)

    # K split over workgroups: this workgroup's K steps are [ksp * KTs, (ksp + 1) * KTs)
    KTs = KT // S
    if S > 1:
        L.append(f"  const unsigned int ksp = blockIdx.z % {S}u, kbase = ksp * {KTs * BK}u;")
    kb = "kbase + " if S > 1 else ""

    # ---- global -> register staging ------------------------------------------------
    def plan_k_major(rows: int, vec: bool):
        """Chunks of a [rows][BK] tile read along K: (per-lane count, elems per chunk)."""
        ve = VK if vec else 1
        total = rows * BK // ve
        return -(-total // THREADS), ve, total

    a_cnt, a_ve, a_tot = plan_k_major(BM, a_vec)
    if tb:
        b_cnt, b_ve, b_tot = plan_k_major(BN, b_vec)
    else:
        b_ve = VK if b_vec else 1
        b_tot = BK * BN // b_ve
        b_cnt = -(-b_tot // THREADS)

    def stage_type(ve: int, src_dt: DType) -> str:
        if ve > 1:
            return "tj_u32x4"
        return lds_t

    a_st_t, b_st_t = stage_type(a_ve, a.dtype), stage_type(b_ve, b.dtype)
    L.append(f"  {a_st_t} ra[{a_cnt}];")
    L.append(f"  {b_st_t} rb[{b_cnt}];")
    if cfg.PINGPONG == 2:
        L.append(f"  {a_st_t} ra2[{a_cnt}];")
        L.append(f"  {b_st_t} rb2[{b_cnt}];")

    def conv(src_dt: DType, expr: str) -> str:
        """Scalar global element -> LDS element type."""
        if src_dt == dt:
            return expr
        return f"tj_ld({expr})"   # fp32 LDS path for mixed / integer operands

    def load_lines(sa: str = "ra", sb: str = "rb", parts: str = "ab") -> list[str]:
        out = []
        if "a" in parts:
            out += a_load_lines(sa)
        if "b" in parts:
            out += b_load_lines(sb)
        return out

    def a_load_lines(sa: str) -> list[str]:
        out = ["#pragma unroll", f"  for (int i = 0; i < {a_cnt}; ++i) {{",
               f"    const unsigned int c = i * {THREADS}u + tid;"]
        if a_tot % THREADS:
            out.append(f"    if (c >= {a_tot}u) break;")
        per_row = BK // a_ve
        out.append(f"    const unsigned int row = c / {per_row}u, kk = (c % {per_row}u) * {a_ve}u;")
        out.append(f"    const {idx_t} gm = m0 + row, gk = k0 + kk;")
        conds = []
        if guard_m:
            conds.append(f"gm < {M}u")
        if guard_k:
            conds.append(f"gk < {K}u")
        cond = " && ".join(conds)
        src = f"Ab[gm * {K}u + gk]"
        if a_ve > 1:
            ld = f"*(const tj_u32x4*)&{src}"
            zero = "(tj_u32x4){0u, 0u, 0u, 0u}"
        else:
            ld = conv(a.dtype, src)
            zero = f"({lds_t})0"
        out.append(f"    {sa}[i] = ({cond}) ? {ld} : {zero};" if cond else f"    {sa}[i] = {ld};")
        out.append("  }")
        return out

    def b_load_lines(sb: str) -> list[str]:
        out = ["#pragma unroll", f"  for (int i = 0; i < {b_cnt}; ++i) {{",
               f"    const unsigned int c = i * {THREADS}u + tid;"]
        if b_tot % THREADS:
            out.append(f"    if (c >= {b_tot}u) break;")
        if tb:
            per_row = BK // b_ve
            out.append(f"    const unsigned int row = c / {per_row}u, kk = (c % {per_row}u) * {b_ve}u;")
            out.append(f"    const {idx_t} gn = n0 + row, gk = k0 + kk;")
            conds = ([f"gn < {N}u"] if guard_n else []) + ([f"gk < {K}u"] if guard_k else [])
            src = f"Bb[gn * {K}u + gk]"
        else:
            # consecutive lanes take consecutive k rows of one 16-byte column chunk, so the
            # transposing 2-byte LDS stores below hit consecutive addresses (no bank conflicts)
            out.append(f"    const unsigned int krow = c % {BK}u, nn = (c / {BK}u) * {b_ve}u;")
            out.append(f"    const {idx_t} gn = n0 + nn, gk = k0 + krow;")
            conds = ([f"gn < {N}u"] if guard_n else []) + ([f"gk < {K}u"] if guard_k else [])
            src = f"Bb[gk * {N}u + gn]"
        cond = " && ".join(conds)
        if b_ve > 1:
            ld = f"*(const tj_u32x4*)&{src}"
            zero = "(tj_u32x4){0u, 0u, 0u, 0u}"
        else:
            ld = conv(b.dtype, src)
            zero = f"({lds_t})0"
        out.append(f"    {sb}[i] = ({cond}) ? {ld} : {zero};" if cond else f"    {sb}[i] = {ld};")
        out.append("  }")
        return out

    def store_lines(buf: str, sa: str = "ra", sb: str = "rb", parts: str = "ab") -> list[str]:
        out = []
        if "a" in parts:
            out += a_store_lines(buf, sa)
        if "b" in parts:
            out += b_store_lines(buf, sb)
        return out

    def a_store_lines(buf: str, sa: str) -> list[str]:
        out = ["#pragma unroll", f"  for (int i = 0; i < {a_cnt}; ++i) {{",
               f"    const unsigned int c = i * {THREADS}u + tid;"]
        if a_tot % THREADS:
            out.append(f"    if (c >= {a_tot}u) break;")
        per_row = BK // a_ve
        out.append(f"    const unsigned int row = c / {per_row}u, kk = (c % {per_row}u) * {a_ve}u;")
        if a_ve > 1:
            out.append(f"    *(tj_u32x4*)&As[{buf}][row][kk] = {sa}[i];")
        else:
            out.append(f"    As[{buf}][row][kk] = {sa}[i];")
        out.append("  }")
        return out

    def b_store_lines(buf: str, sb: str) -> list[str]:
        out = ["#pragma unroll", f"  for (int i = 0; i < {b_cnt}; ++i) {{",
               f"    const unsigned int c = i * {THREADS}u + tid;"]
        if b_tot % THREADS:
            out.append(f"    if (c >= {b_tot}u) break;")
        if tb:
            per_row = BK // b_ve
            out.append(f"    const unsigned int row = c / {per_row}u, kk = (c % {per_row}u) * {b_ve}u;")
            if b_ve > 1:
                out.append(f"    *(tj_u32x4*)&Bs[{buf}][row][kk] = {sb}[i];")
            else:
                out.append(f"    Bs[{buf}][row][kk] = {sb}[i];")
        else:
            out.append(f"    const unsigned int krow = c % {BK}u, nn = (c / {BK}u) * {b_ve}u;")
            if b_ve > 1:
                out.append("#pragma unroll")
                out.append("    for (int w = 0; w < 4; ++w) {")
                out.append(f"      const unsigned int x_ = {sb}[i][w];")
                if esz == 4:
                    out.append(f"      Bs[{buf}][nn + w][krow] = __builtin_bit_cast(float, x_);")
                else:
                    lo, hi = "(unsigned short)(x_ & 0xffffu)", "(unsigned short)(x_ >> 16)"
                    if dt == DType.f16:
                        lo, hi = f"__builtin_bit_cast(_Float16, {lo})", f"__builtin_bit_cast(_Float16, {hi})"
                    out.append(f"      Bs[{buf}][nn + 2 * w][krow] = {lo};")
                    out.append(f"      Bs[{buf}][nn + 2 * w + 1][krow] = {hi};")
                out.append("    }")
            else:
                out.append(f"    Bs[{buf}][nn][krow] = {sb}[i];")
        out.append("  }")
        return out

    # ---- MFMA compute on one LDS buffer ----------------------------------------------
    groups = 64 // MI
    acc_t = "tj_f32x16" if NACC == 16 else "tj_f32x4"
    L.append(f"  {acc_t} acc[{TMW}][{TNW}];")
    L.append("#pragma unroll")
    L.append(f"  for (int x = 0; x < {TMW}; ++x)")
    L.append("#pragma unroll")
    L.append(f"    for (int y = 0; y < {TNW}; ++y) acc[x][y] = ({acc_t})(0.0f);")
    L.append(f"  const unsigned int arow = wm * {BM // WM}u + (lane % {MI}u);")
    L.append(f"  const unsigned int brow = wn * {BN // WN}u + (lane % {MI}u);")
    L.append(f"  const unsigned int kofs = (lane / {MI}u) * {KPL}u;")
    if dt == DType.f32:
        L.append(f"  const unsigned int kofs4 = (lane / {MI}u) * 4u;")

    KS = BK // KI

    def compute_lines_f32(buf: str) -> list[str]:
        """fp32 MFMAs of one K step.  An fp32 MFMA takes one k per lane group (16x16x4:
        lanes l and l + 16 hold k and k + 1), so reading its operands one 4-byte LDS read
        per MFMA leaves the wave waiting on LDS latency.  Instead lane group g reads 4
        consecutive k (one 16-byte read) and the 4 MFMAs of a group take element j of
        them: MFMA j sums A[i][g*4 + j] * B[n][g*4 + j] over the groups g, so the 4 of
        them together cover every k of the group exactly once (A and B share the
        mapping; only the order of the fp32 additions changes).  Reads of the next
        group are issued before the MFMAs of this one."""
        KG = 4 * KI                                 # k per 16-byte read group: 16 (16x16x4) or 8 (32x32x2)
        NG = BK // KG
        def frag_loads(slot: str, gi: str) -> list[str]:
            return ["#pragma unroll",
                    f"    for (int x = 0; x < {TMW}; ++x) fa[{slot}][x] = *(const tj_f32x4*)&As[{buf}][arow + x * {MI}u][{gi} * {KG} + kofs4];",
                    "#pragma unroll",
                    f"    for (int y = 0; y < {TNW}; ++y) fb[{slot}][y] = *(const tj_f32x4*)&Bs[{buf}][brow + y * {MI}u][{gi} * {KG} + kofs4];"]
        out = ["  {", f"    tj_f32x4 fa[2][{TMW}], fb[2][{TNW}];"]
        out += frag_loads("0", "0")
        out += ["#pragma unroll", f"  for (int gi = 0; gi < {NG}; ++gi) {{"]
        if NG > 1:
            out.append(f"    if (gi + 1 < {NG}) {{")
            out += ["  " + x for x in frag_loads("(gi + 1) & 1", "(gi + 1)")]
            out.append("    }")
        out.append("    __builtin_amdgcn_sched_barrier(0);")
        out += ["#pragma unroll", "    for (int j = 0; j < 4; ++j)", "#pragma unroll",
                f"      for (int x = 0; x < {TMW}; ++x)", "#pragma unroll",
                f"        for (int y = 0; y < {TNW}; ++y) acc[x][y] = {builtin}(fa[gi & 1][x][j], fb[gi & 1][y][j], acc[x][y], 0, 0, 0);",
                "    __builtin_amdgcn_sched_barrier(0);", "  }", "  }"]
        return out

    def compute_lines(buf: str) -> list[str]:
        """MFMAs of one K step.  Fragment registers are double buffered: the LDS reads
        of sub-step ks+1 are issued before the MFMAs of ks, so LDS latency overlaps
        the matrix cores instead of stalling them."""
        if dt == DType.f32 and BK % (4 * KI) == 0:
            return compute_lines_f32(buf)
        def frag_loads(slot: str, ks: str) -> list[str]:
            return ["#pragma unroll",
                    f"    for (int x = 0; x < {TMW}; ++x) fa[{slot}][x] = *(const {opvec}*)&As[{buf}][arow + x * {MI}u][{ks} * {KI} + kofs];",
                    "#pragma unroll",
                    f"    for (int y = 0; y < {TNW}; ++y) fb[{slot}][y] = *(const {opvec}*)&Bs[{buf}][brow + y * {MI}u][{ks} * {KI} + kofs];"]
        out = ["  {", f"    {opvec} fa[2][{TMW}], fb[2][{TNW}];"]
        out += frag_loads("0", "0")
        out += ["#pragma unroll", f"  for (int ks = 0; ks < {KS}; ++ks) {{"]
        if KS > 1:
            out.append(f"    if (ks + 1 < {KS}) {{")
            out += ["  " + x for x in frag_loads("(ks + 1) & 1", "(ks + 1)")]
            out.append("    }")
        # keep the compiler's scheduler from sinking the next fragments' LDS reads
        # below this sub-step's MFMAs (it otherwise serialises read -> wait -> MFMA)
        out.append("    __builtin_amdgcn_sched_barrier(0);")
        out.append("#pragma unroll")
        out.append(f"    for (int x = 0; x < {TMW}; ++x)")
        out.append("#pragma unroll")
        out.append(f"      for (int y = 0; y < {TNW}; ++y) acc[x][y] = {builtin}(fa[ks & 1][x], fb[ks & 1][y], acc[x][y], 0, 0, 0);")
        out.append("    __builtin_amdgcn_sched_barrier(0);")
        out.append("  }")
        out.append("  }")
        return out

    if cfg.INTERLEAVE:
        L += interleaved_loop_lines(cfg, KT, KS, BK, TMW, TNW, MI, KI, opvec, builtin, load_lines, store_lines,
                                    a_cnt, b_cnt)
        return _finish_matmul(L, g, k, mm, epilogue, out_shape, bidx, batch_shape, M, N, K, BM, BN, WM, WN, MI, TMW,
                              TNW, NACC, THREADS, lds_bytes, guard_m, guard_n, idx_t, cfg, dt, tb, batch, fname)
    if cfg.PINGPONG:
        L += pingpong_loop_lines(cfg, KT, KS, BK, TMW, TNW, MI, KI, opvec, builtin, load_lines, store_lines)
        return _finish_matmul(L, g, k, mm, epilogue, out_shape, bidx, batch_shape, M, N, K, BM, BN, WM, WN, MI, TMW,
                              TNW, NACC, THREADS, lds_bytes, guard_m, guard_n, idx_t, cfg, dt, tb, batch, fname)
    # Pipeline: registers always hold the tile one K step ahead of LDS.  Step kt runs
    # the MFMAs on LDS[kt & 1], then writes the registers (tile kt+1, loaded one full
    # MFMA phase earlier) to LDS[(kt+1) & 1], then issues the global loads of tile kt+2
    # so their latency hides behind the next step's MFMAs; one barrier per step.
    L.append(f"  unsigned int k0 = {kb}0u;")
    L += load_lines()
    L += store_lines("0")
    if KTs > 1:
        L.append(f"  k0 = {kb}{BK}u;")
        L += load_lines()
    L.append("  __syncthreads();")
    L.append(f"  for (int kt = 0; kt < {KTs}; ++kt) {{")
    L.append("    const int cur = kt & 1;")
    L += ["  " + s for s in compute_lines("cur")]
    L.append(f"    if (kt + 1 < {KTs}) {{")
    L += ["    " + s for s in store_lines("cur ^ 1")]
    L.append("    }")
    L.append(f"    if (kt + 2 < {KTs}) {{")
    L.append(f"      k0 = {kb}(kt + 2) * {BK}u;")
    L += ["    " + s for s in load_lines()]
    L.append("    }")
    L.append("    __syncthreads();")
    L.append("  }")

    return _finish_matmul(L, g, k, mm, epilogue, out_shape, bidx, batch_shape, M, N, K, BM, BN, WM, WN, MI, TMW, TNW,
                          NACC, THREADS, lds_bytes, guard_m, guard_n, idx_t, cfg, dt, tb, batch, fname)


def pingpong_loop_lines(cfg, KT, KS, BK, TMW, TNW, MI, KI, opvec, builtin, load_lines, store_lines) -> list[str]:
    """Main loop with two wave groups a phase apart ("ping-pong").

    Waves ``[0, W/2)`` and ``[W/2, W)`` form two groups; each SIMD runs one wave of
    each.  Every step is a memory phase (read the step's fragments from LDS stage
    ``kt & 1``, write staged data of tile kt+1 to the other stage, issue global loads)
    and a compute phase (the step's MFMA burst at raised priority), separated by
    barriers.  Group 1 starts one barrier late, so on every SIMD one wave computes
    while the other moves data.  Ordering: tile kt+1 is written in the memory phases
    of tile kt and first read after the barrier that ends them; the stage it overwrites
    was last read before the barrier that starts them.  Every wave executes the same
    number of barriers plus one (at the start for group 1, at the end for group 0).

    ``PINGPONG`` 1 and 2: one step per tile; tile t's global loads are issued at step
    t-PF (PF = PINGPONG + 1) into staging register set ``t % (PF-1)`` and written to LDS
    at step t-1.  ``PINGPONG`` 3: tiles are twice as wide in K as a step (BK = 64 bf16
    = a full 128-byte line per row, half the L2 requests of BK = 32) and each tile is
    computed in two half steps; the first half step moves the A part of the staged
    tile, the second the B part, so PF = 2 with one register set.  The loop body holds
    two tiles (even and odd), which makes every LDS stage and register set a
    compile-time choice; the last tiles, which have no tile left to load, are peeled."""
    split = cfg.PINGPONG == 3
    pf = 2 if split else cfg.PINGPONG + 1
    nsets = pf - 1
    sets = [("ra", "rb"), ("ra2", "rb2")][:nsets]
    ksh = KS // 2 if split else KS
    halves = [(0, ksh, "a"), (ksh, KS, "b")] if split else [(0, KS, "ab")]

    def step(kt: str, stage: int, ks0: int, ks1: int, parts: str, do_store: bool, do_load: bool,
             ind: str) -> list[str]:
        out = ["#pragma unroll", f"for (int ks = {ks0}; ks < {ks1}; ++ks) {{", "#pragma unroll",
               f"  for (int x = 0; x < {TMW}; ++x) fa[ks - {ks0}][x] = *(const {opvec}*)&As[{stage}][arow + x * {MI}u][ks * {KI} + kofs];",
               "#pragma unroll",
               f"  for (int y = 0; y < {TNW}; ++y) fb[ks - {ks0}][y] = *(const {opvec}*)&Bs[{stage}][brow + y * {MI}u][ks * {KI} + kofs];",
               "}"]
        if do_store or do_load:
            # tile kt+1 lives in set (kt+1) % nsets; kt+PF maps to the same set
            sel = f"(({kt}) + 1) % {nsets}" if nsets > 1 else "0"
            for j, (sa, sb) in enumerate(sets):
                body = []
                if do_store:
                    body += store_lines(str(1 - stage), sa, sb, parts)
                if do_store and do_load:
                    # loads after the stores: hoisted above the fragment reads they slow the phase
                    body.append("__builtin_amdgcn_sched_barrier(0);")
                if do_load:
                    body.append(f"k0 = (({kt}) + {pf}) * {BK}u;")
                    body += load_lines(sa, sb, parts)
                if nsets > 1:
                    out.append(f"if ({sel} == {j}) {{")
                    out += ["  " + x.strip() for x in body]
                    out.append("}")
                else:
                    out += [x.strip() for x in body]
        out += ["__builtin_amdgcn_sched_barrier(0);", "__syncthreads();", "__builtin_amdgcn_sched_barrier(0);",
                "__builtin_amdgcn_s_setprio(1);", "#pragma unroll", f"for (int ks = 0; ks < {ks1 - ks0}; ++ks)",
                "#pragma unroll", f"  for (int x = 0; x < {TMW}; ++x)", "#pragma unroll",
                f"    for (int y = 0; y < {TNW}; ++y) acc[x][y] = {builtin}(fa[ks][x], fb[ks][y], acc[x][y], 0, 0, 0);",
                "__builtin_amdgcn_s_setprio(0);", "__builtin_amdgcn_sched_barrier(0);", "__syncthreads();",
                "__builtin_amdgcn_sched_barrier(0);"]
        return [ind + x for x in out]

    def tile(kt: str, stage: int, do_store: bool, do_load: bool, ind: str) -> list[str]:
        out = []
        for ks0, ks1, parts in halves:
            out += step(kt, stage, ks0, ks1, parts, do_store, do_load, ind)
        return out

    L = ["  unsigned int k0 = 0;"]
    L += load_lines(*sets[0])
    L += store_lines("0", *sets[0])
    for t in range(1, pf):
        if t < KT:
            # keep the tiles' loads in issue order: the loop's vmcnt waits assume it
            L.append("  __builtin_amdgcn_sched_barrier(0);")
            L.append(f"  k0 = {t * BK}u;")
            L += load_lines(*sets[t % nsets])
    L.append("  __syncthreads();")
    L.append(f"  const bool grp1 = wave >= {cfg.num_warps // 2}u;")
    L.append("  if (grp1) __syncthreads();")
    L.append(f"  {opvec} fa[{ksh}][{TMW}], fb[{ksh}][{TNW}];")
    # tiles 0 .. KT-PF-1 load tile kt+PF; run them in even/odd pairs, then peel the rest
    nload = max(0, KT - pf)
    npair = nload // 2
    if npair:
        L.append(f"  for (int kt = 0; kt < {2 * npair}; kt += 2) {{")
        L += tile("kt", 0, True, True, "    ")
        L += tile("kt + 1", 1, True, True, "    ")
        L.append("  }")
    for kt in range(2 * npair, KT):
        L.append(f"  {{  // K tile {kt}")
        L += tile(str(kt), kt % 2, kt + 1 < KT, kt + pf < KT, "    ")
        L.append("  }")
    L.append("  if (!grp1) __syncthreads();")
    return L


# __builtin_amdgcn_sched_group_barrier instruction classes
SG_MFMA, SG_VMEM_READ, SG_DS_READ, SG_DS_WRITE = 0x008, 0x020, 0x100, 0x200


def interleaved_loop_lines(cfg, KT, KS, BK, TMW, TNW, MI, KI, opvec, builtin, load_lines, store_lines,
                           a_cnt, b_cnt) -> list[str]:
    """Main loop for one wave per SIMD (``INTERLEAVE``): the wave's own memory traffic
    is threaded between its MFMAs instead of being given to a second wave.

    Each wave owns a large output tile (128x128 of a 256x256 block: accumulators in
    the 256 AGPRs), so every 16-byte fragment read feeds twice as many MFMAs as in the
    8-wave layouts.  Tile kt (LDS stage ``kt & 1``) is computed in KS sub-steps with
    fragments double-buffered in registers.  The first KS-1 sub-steps form one
    scheduling region holding their MFMAs, the fragment reads of the next sub-steps,
    the LDS stores of the staged tile kt+1 (into the other stage) and the global loads
    of tile kt+2 (into the staging registers just stored); ``sched_group_barrier``
    places one memory instruction after each MFMA.  One barrier per tile follows (the
    stores are complete and the other stage is no longer read), then the last
    sub-step's MFMAs run with the reads of tile kt+1's first fragments."""
    nmm = TMW * TNW                      # MFMAs per sub-step

    def frag_reads(buf: str, stage: int, ks: str) -> list[str]:
        return ["#pragma unroll",
                f"for (int x = 0; x < {TMW}; ++x) fa[{buf}][x] = *(const {opvec}*)&As[{stage}][arow + x * {MI}u][({ks}) * {KI} + kofs];",
                "#pragma unroll",
                f"for (int y = 0; y < {TNW}; ++y) fb[{buf}][y] = *(const {opvec}*)&Bs[{stage}][brow + y * {MI}u][({ks}) * {KI} + kofs];"]

    def mfmas(buf: str) -> list[str]:
        return ["#pragma unroll", f"for (int x = 0; x < {TMW}; ++x)", "#pragma unroll",
                f"  for (int y = 0; y < {TNW}; ++y) acc[x][y] = {builtin}(fa[{buf}][x], fb[{buf}][y], acc[x][y], 0, 0, 0);"]

    def pattern(n_mfma: int, n_read: int, n_write: int, n_vmem: int) -> list[str]:
        """One MFMA, then at most one memory instruction, repeated: reads first, then
        stores, then global loads, spread evenly over the MFMAs."""
        out = []
        mem = [SG_DS_READ] * n_read + [SG_DS_WRITE] * n_write + [SG_VMEM_READ] * n_vmem
        per = max(1, -(-len(mem) // max(n_mfma, 1)))
        for i in range(n_mfma):
            out.append(f"__builtin_amdgcn_sched_group_barrier({SG_MFMA}, 1, 0);")
            for m in mem[i * per:(i + 1) * per]:
                out.append(f"__builtin_amdgcn_sched_group_barrier({m}, 1, 0);")
        return out

    def tile(kt: str, stage: int, do_store: bool, do_load: bool, next_reads: bool, ind: str) -> list[str]:
        out = []
        # region A: sub-steps 0 .. KS-2
        for ks in range(KS - 1):
            out += mfmas(str(ks % 2))
            out += frag_reads(str((ks + 1) % 2), stage, str(ks + 1))
        if do_store:
            out += [x.strip() for x in store_lines(str(1 - stage))]
        if do_load:
            out.append(f"k0 = (({kt}) + 2) * {BK}u;")
            out += [x.strip() for x in load_lines()]
        nreads = (KS - 1) * (TMW + TNW)
        out += pattern((KS - 1) * nmm, nreads, (a_cnt + b_cnt) if do_store else 0, (a_cnt + b_cnt) if do_load else 0)
        out += ["__builtin_amdgcn_sched_barrier(0);", "__syncthreads();", "__builtin_amdgcn_sched_barrier(0);"]
        # region B: last sub-step, with the next tile's first fragments
        out += mfmas(str((KS - 1) % 2))
        if next_reads:
            out += frag_reads(str(KS % 2), 1 - stage, "0")
        out += pattern(nmm, (TMW + TNW) if next_reads else 0, 0, 0)
        out.append("__builtin_amdgcn_sched_barrier(0);")
        return [ind + x for x in out]

    assert KS % 2 == 0, "interleaved schedule needs an even number of sub-steps per tile"
    L = ["  unsigned int k0 = 0;"]
    L += load_lines()
    L += store_lines("0")
    if KT > 1:
        L.append("  __builtin_amdgcn_sched_barrier(0);")
        L.append(f"  k0 = {BK}u;")
        L += load_lines()
    L.append("  __syncthreads();")
    L.append(f"  {opvec} fa[2][{TMW}], fb[2][{TNW}];")
    L += ["  " + x for x in frag_reads("0", 0, "0")]
    nload = max(0, KT - 2)
    npair = nload // 2
    if npair:
        L.append(f"  for (int kt = 0; kt < {2 * npair}; kt += 2) {{")
        L += tile("kt", 0, True, True, True, "    ")
        L += tile("kt + 1", 1, True, True, True, "    ")
        L.append("  }")
    for kt in range(2 * npair, KT):
        L.append(f"  {{  // K tile {kt}")
        L += tile(str(kt), kt % 2, kt + 1 < KT, kt + 2 < KT, kt + 1 < KT, "    ")
        L.append("  }")
    return L


# direct-to-LDS load split per MFMA size: (loads of tile kt+2 issued in tile kt's
# region B, region-A sub-steps of tile kt+1 over which the rest are spread)
DIRECT_SPLIT = {32: (8, 1), 16: (12, 1)}


def _vmcnt_only(n: int) -> str:
    """s_waitcnt immediate for gfx9 that waits until at most ``n`` vector-memory
    operations are outstanding (vmcnt split over bits 3:0 and 15:14; expcnt and
    lgkmcnt at their maxima, i.e. not waited on)."""
    assert 0 <= n < 64
    return hex((n & 15) | ((n >> 4) << 14) | 0x0F70)


def _lgkmcnt_only(n: int) -> str:
    """s_waitcnt immediate for gfx9 that waits until at most ``n`` LDS / scalar-memory
    operations are outstanding (lgkmcnt in bits 11:8; vmcnt and expcnt at their maxima)."""
    assert 0 <= n < 16
    return hex(0xC07F | (n << 8))


def direct_loop_lines(cfg, M, N, K, BM, BN, TMW, TNW, KT, opvec, builtin, persist: dict | None = None,
                      esz: int = 2) -> list[str]:
    """Main loop for one wave per SIMD with tiles loaded straight into LDS (``DIRECT``).

    ``buffer_load_dwordx4 ... lds`` moves 16 bytes per lane from HBM/L2 into LDS
    without passing through registers: no staging VGPRs and no LDS store
    instructions, so each wave can hold a 128x128 accumulator tile (256 AGPRs) and its
    issue slots go to MFMAs and fragment reads.  One instruction writes 1 KiB of LDS
    contiguously (lane i at byte 16 i), i.e. eight 128-byte K rows of a 64-deep tile.
    Rows are not padded; instead the 16-byte chunk ``c`` of tile row ``r`` is stored at
    position ``c ^ f(r)`` with ``f(r) = (r & 7) ^ ((r >> 3) & 3)``, applied by choosing
    which chunk each lane fetches (the 8 lanes of a row still cover one whole 128-byte
    line).  The LDS serves a 16-byte read 32 lanes at a time over 512 bytes of banks;
    the 32 lanes of a fragment read (32 rows, or 16 rows x 2 k-groups) then land on 32
    distinct 16-byte bank groups.

    Two LDS stages, each operand and stage its own ``__shared__`` array so the
    compiler can tell the stage being filled from the stage being read and does not
    wait for the loads in flight before each fragment read.  Tile kt (stage kt & 1):
    region A runs the MFMAs of sub-steps 0 .. KS-2 with the fragment reads of the next
    sub-steps placed between them, plus the second part of tile kt+1's loads; a
    barrier (after each wave's wait for its own loads) publishes tile kt+1 and frees
    stage kt & 1; region B runs the last sub-step's MFMAs with the reads of tile
    kt+1's first fragments and the first part of tile kt+2's loads into the freed
    stage.  Every load so gets at least a sub-step of MFMAs to land.

    MFMA shapes: 32x32x16 (four 16-deep sub-steps per tile, 16 MFMAs each, both
    fragment sets double-buffered) or 16x16x32 (two 32-deep sub-steps, 64 MFMAs each;
    the A fragment of row tile x is re-read for the next sub-step right after the
    sub-step's last MFMA on that row, so only B is double-buffered: 96 fragment VGPRs
    instead of 128).  Each memory instruction has a fixed slot after one MFMA: DMA
    loads one per 64 MFMA cycles of a wave (about what the texture unit passes for
    four waves at ~16 cycles per 1 KiB load), fragment reads in the slots between.

    ``persist`` (``cfg.PERSIST`` workgroups, one per CU, looping over the output tiles;
    emitted by ``persistent_direct_lines``): the operand descriptors move with the
    tile, the next tile's first K tile is loaded into stage 0 from tile KT-2's region B
    on (stage 0 is free from that tile's barrier, as for any tile kt+2), its second
    into stage 1 once the last tile's reads are done, and the epilogue stages through
    an LDS array of its own, so the next tile's MFMAs start without a load wait and the
    output stores drain under them.

    fp32 (``esz`` 4, 16x16x4 MFMAs, 32-deep K tiles: the same 128-byte rows): a
    fragment read brings each lane 4 consecutive k, which feed 4 MFMAs (element j of A
    and B each; the lane groups' k interleave as in the bf16 layout, for A and B alike),
    so a sub-step runs 4 passes over the accumulators, j outermost (no two consecutive
    MFMAs share an accumulator); A fragments are re-read after their last pass."""
    nw = cfg.num_warps
    MI = cfg.MI
    f32 = esz == 4
    KI = 16 if MI == 32 else 32               # bf16 / fp16 K per MFMA
    KS = 64 // KI                             # sub-steps (64 bytes of K per row for 16x16) per tile
    NACC = MI * MI // 64
    # MFMAs per 64 cycles: 32x32x16 takes 32 cycles, 16x16x32 16, 16x16x4 f32 32
    dsp = 2 if f32 else 64 // MI
    passes = 4 if f32 else 1                  # MFMAs per fragment pair and sub-step
    # Barrier that publishes a stage filled by DMA: each wave first waits for its own
    # DMA loads (vmcnt 0; expcnt and lgkmcnt left at their maxima).  A workgroup-scope
    # fence does not cover loads that write LDS, and the compiler's own vmcnt wait is
    # placed after the barrier (it only orders this wave's reads), so without this
    # wait another wave can read a block whose DMA is still landing.
    publish = ["__builtin_amdgcn_s_waitcnt(0x0F70);", "__syncthreads();"]
    a_cnt, b_cnt = BM // (8 * nw), BN // (8 * nw)
    nmm = TMW * TNW
    L = [f"  __shared__ __attribute__((aligned(1024))) char As0[{BM * 128}];",
         f"  __shared__ __attribute__((aligned(1024))) char As1[{BM * 128}];",
         f"  __shared__ __attribute__((aligned(1024))) char Bs0[{BN * 128}];",
         f"  __shared__ __attribute__((aligned(1024))) char Bs1[{BN * 128}];"]
    if persist:
        L.append(f"  __shared__ __attribute__((aligned(16))) float Cs[{nw}][{16 * TNW * MI}];")
    L += [
         "  const unsigned int wv = __builtin_amdgcn_readfirstlane(wave);",
         "  const unsigned int drow = lane >> 3;",
         f"  tj_f32x{NACC} acc[{TMW}][{TNW}];",
         "#pragma unroll",
         f"  for (int x = 0; x < {TMW}; ++x)",
         "#pragma unroll",
         f"    for (int y = 0; y < {TNW}; ++y) acc[x][y] = (tj_f32x{NACC})(0.0f);",
         # fragment addresses: row (wave base + MI x + lane % MI), logical chunk
         # (KI / 8) ks + lane / MI of the 64-deep tile
         f"  const unsigned int fr = lane & {MI - 1}u, fh = lane >> {MI.bit_length() - 1};",
         "  const unsigned int fsw = (fr & 7u) ^ ((fr >> 3) & 3u);",
         f"  const unsigned int arow = (wm * {BM // cfg.WM}u + fr) * 128u;",
         f"  const unsigned int brow = (wn * {BN // cfg.WN}u + fr) * 128u;"]
    if MI == 32:
        # row tiles start at multiples of 32: f(r) is that of the row within the tile
        nofs = KS
        L.append(f"  unsigned int fofs[{nofs}];")
        L += [f"  fofs[{ks}] = (({2 * ks}u + fh) ^ fsw) * 16u;" for ks in range(KS)]
        fofs = lambda ks, t: ks                                          # noqa: E731
    else:
        # a 16-row tile at an odd multiple of 16 has bit 1 of (r >> 3) & 3 set.  K-group
        # g of a sub-step reads chunk 4 ks + sigma(g), sigma swapping g's two bits (A and
        # B alike, so each MFMA still pairs equal k): the LDS serves a 16-byte read 32
        # lanes at a time over 512 bytes of banks, and lanes 0-15 / 16-31 hold k-groups 0
        # and 1 of the same 16 rows; in chunks c and c+1 rows r and r ^ 8 would share a
        # bank group (every read 2-way conflicted, measured), in chunks c and c+2 none do
        nofs = 2 * KS
        L.append(f"  unsigned int fofs[{nofs}];")
        L.append("  const unsigned int fg = ((fh & 1u) << 1) | (fh >> 1);")
        L += [f"  fofs[{2 * ks + par}] = (({4 * ks}u + fg) ^ fsw ^ {2 * par}u) * 16u;"
              for ks in range(KS) for par in range(2)]
        fofs = lambda ks, t: 2 * ks + (t & 1)                            # noqa: E731

    # Loads go through buffer resources (buffer_load_dwordx4 ... lds): a 32-bit lane
    # offset that does not change over K (row and swizzled chunk), the tile's K position
    # in a scalar offset, and the descriptor's range check, which returns zeros for rows
    # past M or N (no clamping).  The global_load_lds form would also work, but the
    # compiler treats it as a flat access that may touch LDS and then waits for every
    # outstanding LDS read (lgkmcnt 0) wherever one fragment is needed.
    if not persist:
        L.append(f"  const __amdgpu_buffer_rsrc_t rsA = __builtin_amdgcn_make_buffer_rsrc((void*)Ab, (short)0, {M * K * esz}, 0x00020000);")
        L.append(f"  const __amdgpu_buffer_rsrc_t rsB = __builtin_amdgcn_make_buffer_rsrc((void*)Bb, (short)0, {N * K * esz}, 0x00020000);")
    # persistent: each tile's descriptors start at its first row, so the lane offsets
    # are the same for every tile
    for op, cnt, rows in (("A", a_cnt, "m0"), ("B", b_cnt, "n0")):
        L.append(f"  unsigned int vo{op}[{cnt}];")
        base = "" if persist else f"{rows} + "
        for i in range(cnt):
            q = f"({i * nw}u + wv)"
            L.append(f"  vo{op}[{i}] = (({base}{q} * 8u + drow) * {K}u + ((lane & 7u) ^ drow ^ ({q} & 3u)) * {16 // esz}u)"
                     f" * {esz}u;")

    def dma(kt: str, stage: int, nxt: bool = False) -> list[str]:
        """The DMA loads of tile ``kt`` into ``stage``, one statement per load (``nxt``:
        K tile ``kt`` of the next output tile, through its descriptors)."""
        out = []
        for op, cnt in (("A", a_cnt), ("B", b_cnt)):
            rs = f"rs{op}n" if nxt else f"rs{op}"
            for i in range(cnt):
                q = f"({i * nw}u + wv)"
                out.append(f"__builtin_amdgcn_raw_ptr_buffer_load_lds({rs}, (__attribute__((address_space(3))) void*)"
                           f"({op}s{stage} + {q} * 1024u), 16, vo{op}[{i}], (int)(({kt}) * 128u), 0, 0);")
        return out

    def fa_ref(buf: int, x: int) -> str:
        return f"fa[{buf}][{x}]" if MI == 32 else f"fa[{x}]"

    def frag_reads(buf: int, stage: int, ks: int) -> list[tuple[int, str]]:
        """(slot, statement) of the fragment reads of sub-step ``ks`` from ``stage``
        into set ``buf``.  32x32: in consumption order (fa[0], fb[0..], fa[1], ...),
        one per slot from ``rd0`` on.  16x16: B fragments early (every 4th MFMA of the
        first half), A fragment of row tile x right after the last MFMA of row x."""
        a_rd = [f"{fa_ref(buf, x)} = *(const {opvec}*)(As{stage} + arow + fofs[{fofs(ks, x)}] + {x * MI * 128}u);"
                for x in range(TMW)]
        b_rd = [f"fb[{buf}][{y}] = *(const {opvec}*)(Bs{stage} + brow + fofs[{fofs(ks, y)}] + {y * MI * 128}u);"
                for y in range(TNW)]
        if MI == 32:
            return list(enumerate([a_rd[0]] + b_rd + a_rd[1:]))
        last = (passes - 1) * nmm
        return [(4 * y + 2, r) for y, r in enumerate(b_rd)] + [(last + x * TNW + TNW - 1, r) for x, r in enumerate(a_rd)]

    def mfmas(buf: int) -> list[str]:
        if f32:
            return [f"acc[{x}][{y}] = {builtin}({fa_ref(buf, x)}[{j}], fb[{buf}][{y}][{j}], acc[{x}][{y}], 0, 0, 0);"
                    for j in range(passes) for x in range(TMW) for y in range(TNW)]
        return [f"acc[{x}][{y}] = {builtin}({fa_ref(buf, x)}, fb[{buf}][{y}], acc[{x}][{y}], 0, 0, 0);"
                for x in range(TMW) for y in range(TNW)]

    def region(buf: int, reads: list[tuple[int, str]], loads: list[str]) -> list[str]:
        """One sub-step: its MFMAs with the memory statements placed after their
        slots (DMA loads from slot 0, one per ``dsp`` MFMAs; reads as given; with
        loads present the 32x32 reads move to the odd slots), then the matching
        sched_group_barrier sequence."""
        slots: dict[int, list[tuple[int, str]]] = {}
        nm_all = passes * nmm
        for i, ld in enumerate(loads):
            slots.setdefault(min(i * dsp, nm_all - 1), []).append((SG_VMEM_READ, ld))
        for s, rd in reads:
            if MI == 32 and loads:
                s = 2 * s + 1
            slots.setdefault(min(s, nm_all - 1), []).append((SG_DS_READ, rd))
        code, sched = [], []
        for i, mf in enumerate(mfmas(buf)):
            code.append(mf)
            sched.append(f"__builtin_amdgcn_sched_group_barrier({SG_MFMA}, 1, 0);")
            for mask, stmt in slots.get(i, []):
                code.append(stmt)
                sched.append(f"__builtin_amdgcn_sched_group_barrier({mask}, 1, 0);")
        return code + sched + ["__builtin_amdgcn_sched_barrier(0);"]

    n_batch = a_cnt + b_cnt
    split = DIRECT_SPLIT[MI]
    n_b = min(split[0], n_batch)                  # loads issued in region B
    a_steps = max(1, min(split[1], KS - 1))      # region-A sub-steps taking the rest

    def tile(kt: str, stage: int, carry: bool, do_load: bool, last: bool, ind: str, next0: str = "",
             pub: list[str] | None = None) -> list[str]:
        """Tile kt from LDS stage ``stage``.  The loads of tile kt+2 (into this stage,
        released by this tile's barrier) start in region B; ``carry``: the rest of tile
        kt+1's loads (begun in the previous tile's region B) go into region A here,
        still ahead of the barrier that publishes tile kt+1.  ``last``: no tile follows.
        ``next0`` (persistent): "load" puts the first loads of the next output tile's K
        tile 0 into region B (in place of tile kt+2's), "carry" the rest into region A.
        ``pub``: the publishing wait and barrier, if not the default."""
        out = []
        if carry:
            rest = dma(f"({kt}) + 1", 1 - stage)[n_b:]
        elif next0 == "carry":
            rest = dma("0", 1 - stage, nxt=True)[n_b:]
        else:
            rest = []
        # region A: sub-steps 0 .. KS-2 with the fragment reads of the next sub-steps
        for ks in range(KS - 1):
            mine = rest[len(rest) * ks // a_steps:len(rest) * (ks + 1) // a_steps] if ks < a_steps else []
            out += region(ks % 2, frag_reads((ks + 1) % 2, stage, ks + 1), mine)
        if not last:
            out += (pub or publish) + ["__builtin_amdgcn_sched_barrier(0);"]
        # region B: last sub-step, with the first fragments of tile kt+1 and the first
        # loads of tile kt+2
        reads = frag_reads(0, 1 - stage, 0) if not last else []
        if do_load:
            loads = dma(f"({kt}) + 2", stage)[:n_b]
        elif next0 == "load":
            loads = dma("0", stage, nxt=True)[:n_b]
        else:
            loads = []
        out += region((KS - 1) % 2, reads, loads)
        return [ind + x for x in out]

    if persist:
        return L + persistent_direct_lines(persist, KT, n_batch, dma, frag_reads, tile, opvec, MI, TMW, TNW, esz)
    # prologue: tiles 0 and 1 in flight, wait for tile 0 only (the 2nd batch may
    # stay outstanding: vmcnt <= its load count)
    L += ["  " + x for x in dma("0", 0)]
    if KT > 1:
        L += ["  " + x for x in dma("1", 1)]
        L.append(f"  __builtin_amdgcn_s_waitcnt({_vmcnt_only(n_batch)});")
        L.append("  __syncthreads();")
    else:
        L += ["  " + x for x in publish]
    L.append(f"  {opvec} fa[2][{TMW}], fb[2][{TNW}];" if MI == 32 else f"  {opvec} fa[{TMW}], fb[2][{TNW}];")
    L += ["  " + r for _, r in frag_reads(0, 0, 0)]
    # tile 0 (nothing to carry: the prologue loaded tile 1 whole), then (odd, even)
    # pairs of tiles that all carry and load, then the tail
    L.append("  {  // K tile 0")
    L += tile("0", 0, False, 2 < KT, KT == 1, "    ")
    L.append("  }")
    npair = max(0, KT - 3) // 2
    if npair:
        L.append(f"  for (unsigned int kt = 1; kt < {1 + 2 * npair}u; kt += 2) {{")
        L += tile("kt", 1, True, True, False, "    ")
        L += tile("kt + 1u", 0, True, True, False, "    ")
        L.append("  }")
    for kt in range(1 + 2 * npair, KT):
        L.append(f"  {{  // K tile {kt}")
        L += tile(str(kt), kt % 2, kt + 1 < KT, kt + 2 < KT, kt + 1 == KT, "    ")
        L.append("  }")
    return L


def persistent_direct_lines(p: dict, KT: int, n_batch: int, dma, frag_reads, tile, opvec: str, MI: int, TMW: int,
                            TNW: int, esz: int = 2) -> list[str]:
    """Tile loop of the persistent direct-to-LDS kernel (after the shared set-up of
    ``direct_loop_lines``).

    Workgroup b runs virtual tiles b, b + G, b + 2G, ... (G a multiple of 8, so every
    one of them stays on b's XCD in the XCD-aware order).  Per tile: the descriptors of
    this tile and of the next one (the same tile again after the last, so the
    prefetches stay in bounds), the K loop -- whose tile KT-2 starts, and KT-1 finishes,
    the loads of the next tile's K tile 0 into stage 0 -- a barrier (the last K tile's
    reads are done), the next tile's K tile 1 into stage 1, and the epilogue through
    the ``Cs`` array.  vmcnt counts a wave's vector-memory instructions and completes
    them in issue order, so the waits name how many of the youngest may stay
    outstanding: before the next tile's first fragment reads, its K tile 1 and at
    least ``p["stores"]`` epilogue stores (issued after K tile 0); at its first
    barrier, the epilogue stores only (issued after K tile 1; when the epilogue still
    loads inputs, K tile 1 is issued after it and that barrier waits for everything).
    ``p["pre"]`` loads the epilogue's row-invariant inputs before K tile 1 is issued,
    so the epilogue itself waits on no load behind it."""
    G, T, K, BM, BN = p["G"], p["T"], p["K"], p["BM"], p["BN"]
    early = p["k1_early"]
    x0 = min(63, n_batch + p["stores"])
    x1 = min(63, p["stores"]) if early else 0
    ntm, ntn, gm = p["ntm"], p["ntn"], p["group_m"]

    def rsrc(name: str, base: str, row0: str, rows: int) -> str:
        return (f"const __amdgpu_buffer_rsrc_t {name} = __builtin_amdgcn_make_buffer_rsrc("
                f"(void*)({base} + (unsigned long)({row0}) * {K}u), (short)0, {rows * K * esz}, 0x00020000);")

    L = tile_order_lines(ntm, ntn, gm, BM, BN, vid="blockIdx.x", names=("m0i", "n0i"), sfx="i")
    L += ["  unsigned int v = blockIdx.x, m0 = m0i, n0 = n0i;",
          "  {",
          "    " + rsrc("rsA", "Ab", "m0", BM),
          "    " + rsrc("rsB", "Bb", "n0", BN)]
    L += ["    " + x for x in dma("0", 0) + dma("1", 1)]
    L += [f"    __builtin_amdgcn_s_waitcnt({_vmcnt_only(n_batch)});", "    __syncthreads();", "  }"]
    L.append(f"  {opvec} fa[{TMW}], fb[2][{TNW}];")
    L.append("  for (unsigned int it = 0u;; ++it) {")
    ind = "    "
    L.append(f"{ind}const unsigned int vn = v + {G}u < {T}u ? v + {G}u : v;")
    L += [ind + x.strip() for x in tile_order_lines(ntm, ntn, gm, BM, BN, vid="vn", names=("mn", "nn"), sfx="n")]
    L += [ind + rsrc("rsA", "Ab", "m0", BM), ind + rsrc("rsB", "Bb", "n0", BN),
          ind + rsrc("rsAn", "Ab", "mn", BM), ind + rsrc("rsBn", "Bb", "nn", BN)]
    L += [f"{ind}#pragma unroll", f"{ind}for (int x = 0; x < {TMW}; ++x)", f"{ind}#pragma unroll",
          f"{ind}  for (int y = 0; y < {TNW}; ++y) acc[x][y] = (tj_f32x{MI * MI // 64})(0.0f);"]
    L += [ind + r for _, r in frag_reads(0, 0, 0)]
    pub0 = [f"if (it == 0u) __builtin_amdgcn_s_waitcnt({_vmcnt_only(0)}); "
            f"else __builtin_amdgcn_s_waitcnt({_vmcnt_only(x1)});", "__syncthreads();"]
    L.append(f"{ind}{{  // K tile 0")
    L += tile("0", 0, False, 2 < KT, False, ind + "  ", pub=pub0)
    L.append(f"{ind}}}")
    npair = max(0, KT - 3) // 2
    if npair:
        L.append(f"{ind}for (unsigned int kt = 1; kt < {1 + 2 * npair}u; kt += 2) {{")
        L += tile("kt", 1, True, True, False, ind + "  ")
        L += tile("kt + 1u", 0, True, True, False, ind + "  ")
        L.append(f"{ind}}}")
    for kt in range(1 + 2 * npair, KT):
        nxt = "load" if kt == KT - 2 else "carry" if kt == KT - 1 else ""
        L.append(f"{ind}{{  // K tile {kt}")
        L += tile(str(kt), kt % 2, kt + 1 < KT, kt + 2 < KT, kt + 1 == KT, ind + "  ", next0=nxt)
        L.append(f"{ind}}}")
    # every wave's reads of the last K tile (stage 1) are done; a plain barrier, since the
    # workgroup fence of __syncthreads would also wait for the next tile's K tile 0
    L += [f"{ind}__builtin_amdgcn_sched_barrier(0);", f"{ind}__builtin_amdgcn_s_waitcnt({_lgkmcnt_only(0)});",
          f"{ind}__builtin_amdgcn_s_barrier();", f"{ind}__builtin_amdgcn_sched_barrier(0);"]
    k1 = [ind + x for x in dma("1", 1, nxt=True)] + [f"{ind}__builtin_amdgcn_sched_barrier(0);"]
    L += [ind + x.strip() for x in p["pre"]]
    if p["pre"]:
        L.append(f"{ind}__builtin_amdgcn_sched_barrier(0);")
    if early:
        L += k1
    L += p["epi"]
    if not early:
        L += k1
    L += [f"{ind}if (vn == v) break;",
          f"{ind}v = vn; m0 = mn; n0 = nn;",
          f"{ind}__builtin_amdgcn_s_waitcnt({_vmcnt_only(x0)});",
          f"{ind}__syncthreads();",
          "  }",
          # the last tile's prefetches (of itself again) land before the workgroup's LDS is released
          f"  __builtin_amdgcn_s_waitcnt({_vmcnt_only(0)});"]
    return L


def persistent_epilogue_lines(g, k, mm, epilogue, epi_inputs, out_shape, M, N, BM, BN, WM, WN, TMW, TNW,
                              epi_st: dict) -> tuple[list[str], list[str], int, bool]:
    """Epilogue of the persistent direct kernel: (loads of row-invariant inputs, body,
    minimum number of store instructions per wave, whether every input is preloaded).

    Wave w stages its sub-tile through ``Cs[w]`` one 16-row MFMA block at a time (a
    wave's LDS accesses complete in order: no barrier).  The rows of a block are
    ``cols`` floats apart, a multiple of the 64 banks, so float ``c`` of row ``r`` sits
    at column ``c ^ ((r >> 2) << 4)``: the four row groups a lane writes from land on
    four different 16-bank ranges, and the 16-byte runs read back stay contiguous."""
    MI = 16
    out_dt = k.outputs[0].dtype
    ve = 16 // out_dt.itemsize
    cols, rows_w = TNW * MI, TMW * MI
    per_row = cols // ve
    assert 64 % per_row == 0 and cols >= 64
    jcol = f"n0 + wn * {BN // WN}u + (lane % {per_row}u) * {ve}u"
    # the row-invariant inputs are loaded raw here and converted in the body, after the
    # next tile's K tile 1 is issued: a conversion waits for its load, and vmcnt would
    # make that wait cover every older load as well
    pre_lines, conv, pre = [], [], {}
    for n in epi_inputs:
        si, sj = epi_st[id(n)]
        if si != 0:
            continue
        nm = g.names[id(n)]
        conv.append(f"float {nm}_pre[{ve}];")
        if sj == 1 and 16 // n.dtype.itemsize == ve:
            pre_lines.append(f"const tj_u32x4 {nm}_raw = *(const tj_u32x4*)({nm}_p + ({jcol}));")
            conv.append(f"tj_unpackv({nm}_raw, {nm}_p, {nm}_pre);")
        else:
            pre_lines.append(f"{CTYPE[n.dtype]} {nm}_raw[{ve}];")
            pre_lines.append(f"for (int q = 0; q < {ve}; ++q) {nm}_raw[q] = {nm}_p[({jcol}) * {sj}u + q * {sj}u];")
            conv.append(f"for (int q = 0; q < {ve}; ++q) {nm}_pre[q] = tj_ld({nm}_raw[q]);")
        pre[id(n)] = f"{nm}_pre"
    ind = "    "
    L = [ind + x for x in conv] + [f"{ind}float* __restrict__ Cw = Cs[wave];"]
    for x in range(TMW):
        L += [f"{ind}#pragma unroll", f"{ind}for (int y = 0; y < {TNW}; ++y)", f"{ind}#pragma unroll",
              f"{ind}  for (int r = 0; r < 4; ++r)",
              f"{ind}    Cw[((lane / 16u) * 4u + r) * {cols}u + ((y * 16u + lane % 16u) ^ ((lane / 16u) << 4))] = "
              f"acc[{x}][y][r];"]
        L.append(f"{ind}#pragma unroll")
        L.append(f"{ind}for (unsigned int c = lane; c < {16 * per_row}u; c += 64u) {{")
        L.append(f"{ind}  const unsigned int lr = c / {per_row}u, cc = (c % {per_row}u) * {ve}u;")
        L.append(f"{ind}  const unsigned int i = m0 + wm * {BM // WM}u + {x * 16}u + lr;")
        L.append(f"{ind}  const unsigned int j = n0 + wn * {BN // WN}u + cc;")
        L += [ind + x_ for x_ in _run_lines(g, k, mm, epilogue, epi_inputs, out_shape, [], (), M, N, ve,
                                            f"Cw[lr * {cols}u + ((cc ^ ((lr >> 2) << 4)) + q)]", pre, epi_st)]
        L.append(f"{ind}}}")
    stores = len(k.outputs) * rows_w * cols * out_dt.itemsize // 1024
    return pre_lines, L, stores, len(pre) == len(epi_inputs)


def ksplit_fused_enabled() -> bool:
    return os.environ.get("TENSORJIT_HIP_KSPLIT_FUSED", "1") != "0"


def _ksplit_sum_lines(g, k, mm, epilogue, epi_inputs, out_shape, bidx, batch_shape, M, N, S, bi, i_expr, j_expr,
                      ve, idx_t, coherent: bool = False) -> list[str]:
    """out = epilogue(sum of the S partials) for the run of ``ve`` outputs at (i, j): the
    partials added in split order, as ``gen_ksplit_sum`` and the fused last-workgroup sum
    both do, so the two forms give the same bits.  ``coherent``: the partials are read
    through the buffer descriptor ``rsW`` with sc1 (agent-coherent: past this XCD's L2,
    which may hold no line of them yet but is not kept coherent with the other XCDs)."""
    L = [f"    const {idx_t} i = {i_expr}, j = {j_expr};",
         f"    float sm[{ve}];", "#pragma unroll", f"    for (int q = 0; q < {ve}; ++q) sm[q] = 0.0f;",
         "#pragma unroll", f"    for (int s = 0; s < {S}; ++s) {{"]
    if coherent:
        L.append(f"      const unsigned int src = (unsigned int)((({bi} * {S}u + s) * {M}u + i) * {N}u + j) * 4u;")
        ld4 = "__builtin_bit_cast(tj_f32x4, __builtin_amdgcn_raw_buffer_load_b128(rsW, (int)(src + q4 * 16u), 0, 16))"
        ld1 = "__builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsW, (int)(src + q * 4u), 0, 16))"
    else:
        L.append(f"      const float* src = ws_p + (({bi} * {S}u + s) * {M}u + i) * {N}u + j;")
        ld4, ld1 = "*(const tj_f32x4*)(src + q4 * 4)", "src[q]"
    if ve % 4 == 0:
        L += ["#pragma unroll", f"      for (int q4 = 0; q4 < {ve // 4}; ++q4) {{",
              f"        const tj_f32x4 x = {ld4};",
              "        sm[q4 * 4] += x[0]; sm[q4 * 4 + 1] += x[1]; sm[q4 * 4 + 2] += x[2]; sm[q4 * 4 + 3] += x[3];",
              "      }"]
    else:
        L.append(f"      for (int q = 0; q < {ve}; ++q) sm[q] += {ld1};")
    L.append("    }")
    return L + _run_lines(g, k, mm, epilogue, epi_inputs, out_shape, bidx, batch_shape, M, N, ve, "sm[q]")


def _ksplit_ve(k, N) -> int:
    out_dt = k.outputs[0].dtype
    if any(o.dtype.itemsize != out_dt.itemsize for o in k.outputs):
        return 1
    return 16 // out_dt.itemsize if N % (16 // out_dt.itemsize) == 0 else 1


def _ksplit_finish(L, g, k, mm, epilogue, epi_inputs, out_shape, bidx, batch_shape, M, N, K, BM, BN, WM, WN, MI, TMW,
                   TNW, NACC, THREADS, lds_bytes, guard_m, guard_n, idx_t, cfg, dt, tb, batch, fname):
    """K split over workgroups: each workgroup stores its fp32 partial tile into the
    workspace ``[batch][KSPLIT][M][N]``.  Fused form (default): the last of a tile's S
    workgroups to finish sums the tile's partials and applies the epilogue.  Each
    workgroup writes its partial with agent-scope stores (sc1: through this XCD's L2),
    waits for them (vmcnt 0), and bumps the tile's counter after a workgroup barrier; the
    one that reads S - 1 reads the partials with sc1 loads, sums, and resets the counter
    to 0 for the next call.  (Agent-scope fences instead write back and invalidate the
    whole L2 of the XCD per workgroup: 112 µs instead of 26 for config 1's
    down-projection.)  The counters
    are a zero-initialised ``__device__`` array of the program's code object (zero when
    it is loaded, zero again after every complete launch), so no memset is needed and a
    captured graph replays as is; calls of one program that overlap on a GPU race on
    them as they do on its arena.  Otherwise a second launch sums the partials and
    applies the fused epilogue (``gen_ksplit_sum``)."""
    S = cfg.KSPLIT
    if MI == 32:
        row_of, col_of = "(r / 4) * 8 + (lane / 32u) * 4 + (r % 4)", "lane % 32u"
    else:
        row_of, col_of = "(lane / 16u) * 4 + r", "lane % 16u"
    bi = "bi" if batch_shape else "0u"
    L += ["#pragma unroll", f"  for (int x = 0; x < {TMW}; ++x)", "#pragma unroll", f"  for (int y = 0; y < {TNW}; ++y)",
          "#pragma unroll", f"  for (int r = 0; r < {NACC}; ++r) {{",
          f"    const {idx_t} i = m0 + wm * {BM // WM}u + x * {MI}u + {row_of};",
          f"    const {idx_t} j = n0 + wn * {BN // WN}u + y * {MI}u + {col_of};"]
    conds = ([f"i < {M}u"] if guard_m else []) + ([f"j < {N}u"] if guard_n else [])
    if conds:
        L.append(f"    if ({' && '.join(conds)})")
    grid = (-(-N // BN), -(-M // BM), batch * S)
    ws_bytes = batch * S * M * N * 4
    ve = _ksplit_ve(k, N)
    fused = ksplit_fused_enabled() and BN % ve == 0 and ws_bytes < 2**31
    dst = f"ws_p + (({bi} * {S}u + ksp) * {M}u + i) * {N}u + j"
    # fused: agent-scope stores (sc1, written through to the coherent level) so the last
    # workgroup, possibly on another XCD, reads them without an L2 write-back / invalidate
    L += [f"    __hip_atomic_store({dst}, acc[x][y][r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);" if fused else
          f"    *({dst}) = acc[x][y][r];", "  }"]
    meta = {"family": "matmul", "config": cfg.as_dict(), "dtype": dt.value, "M": M, "N": N, "K": K, "batch": batch,
            "trans_b": tb, "lds_bytes": lds_bytes, "flops": 2.0 * M * N * K * batch, "workspace": ws_bytes,
            "ws_arg": True, "epilogue": "k-split partials"}
    if fused:
        ntm, ntn = -(-M // BM), -(-N // BN)
        cnt = f"{fname}_cnt"
        runs, rpr = BM * BN // ve, BN // ve
        L += ["  __builtin_amdgcn_s_waitcnt(0x0F70);       // vmcnt(0): this lane's partial stores are done",
              "  __shared__ unsigned int tj_last_;",
              "  __syncthreads();",
              f"  const unsigned int ct_ = ({bi} * {ntm}u + m0 / {BM}u) * {ntn}u + n0 / {BN}u;",
              f"  if (tid == 0u) tj_last_ = atomicAdd(&{cnt}[ct_], 1u) == {S - 1}u ? 1u : 0u;",
              "  __syncthreads();",
              "  if (tj_last_ == 0u) return;",
              f"  const __amdgpu_buffer_rsrc_t rsW = __builtin_amdgcn_make_buffer_rsrc((void*)ws_p, (short)0, {ws_bytes}, 0x00020000);"]
        if runs % THREADS == 0:
            # a whole number of runs per lane, unrolled so every partial load is in flight at once
            L += ["#pragma unroll", f"  for (unsigned int rr = 0; rr < {runs // THREADS}u; ++rr) {{",
                  f"    const unsigned int run = tid + rr * {THREADS}u;"]
        else:
            L.append(f"  for (unsigned int run = tid; run < {runs}u; run += {THREADS}u) {{")
        conds = ([f"m0 + run / {rpr}u < {M}u"] if guard_m else []) + ([f"n0 + (run % {rpr}u) * {ve}u < {N}u"] if guard_n else [])
        if conds:
            L.append(f"    if (!({' && '.join(conds)})) continue;")
        L += _ksplit_sum_lines(g, k, mm, epilogue, epi_inputs, out_shape, bidx, batch_shape, M, N, S, bi,
                               f"m0 + run / {rpr}u", f"n0 + (run % {rpr}u) * {ve}u", ve, idx_t, coherent=True)
        L += ["  }", f"  if (tid == 0u) {cnt}[ct_] = 0u;", "}"]
        meta = dict(meta, epilogue="k-split, last workgroup sums", fused_sum=True)
        decl = f"__device__ unsigned int {cnt}[{batch * ntm * ntn}];\n"
        return decl + "\n".join(L), Launch(fname, grid, (THREADS, 1, 1), 0, meta)
    L.append("}")
    partial = Launch(fname, grid, (THREADS, 1, 1), 0, meta)
    src2, sum_launch = gen_ksplit_sum(g, k, mm, epilogue, epi_inputs, out_shape, batch_shape, M, N, S, fname)
    return "\n".join(L) + "\n\n" + src2, [partial, sum_launch]


def gen_ksplit_sum(g, k, mm, epilogue, epi_inputs, out_shape, batch_shape, M, N, S, fname) -> tuple[str, Launch]:
    """Second launch of a K-split GEMM: out = epilogue(sum over the S partials), one lane
    per run of ``ve`` outputs (16-byte output stores, 16-byte partial loads)."""
    ve = _ksplit_ve(k, N)
    batch = math.prod(batch_shape) if batch_shape else 1
    runs = batch * M * N // ve
    idx_t = "unsigned long" if batch * M * N >= 2**31 else "unsigned int"
    name = fname + "_ksum"
    L = [f'extern "C" __global__ __launch_bounds__(256) void {name}({g.params()}, const float* __restrict__ ws_p) {{',
         f"  const {idx_t} t = ({idx_t})blockIdx.x * 256u + threadIdx.x;",
         f"  if (t >= {runs}u) return;",
         f"  const {idx_t} e = t * {ve}u, bi = e / {M * N}u, rem = e % {M * N}u, i0 = rem / {N}u, j0 = rem % {N}u;"]
    bidx = []
    if batch_shape:
        rem = "bi"
        for d, cst in enumerate(contiguous_strides(batch_shape)):
            v = f"b{d}"
            if d == len(batch_shape) - 1:
                L.append(f"  const {idx_t} {v} = {rem};")
            else:
                L.append(f"  const {idx_t} {v} = {rem} / {cst}u, br{d} = {rem} % {cst}u;")
                rem = f"br{d}"
            bidx.append(v)
    L.append("  {")
    L += _ksplit_sum_lines(g, k, mm, epilogue, epi_inputs, out_shape, bidx, batch_shape, M, N, S, "bi", "i0", "j0",
                           ve, idx_t)
    L += ["  }", "}"]
    meta = {"family": "ksplit_sum", "splits": S, "ws_arg": True, "numel": batch * M * N}
    return "\n".join(L), Launch(name, (-(-runs // 256), 1, 1), (256, 1, 1), 0, meta)


def _finish_matmul(L, g, k, mm, epilogue, out_shape, bidx, batch_shape, M, N, K, BM, BN, WM, WN, MI, TMW, TNW, NACC,
                   THREADS, lds_bytes, guard_m, guard_n, idx_t, cfg, dt, tb, batch, fname):
    a, b = mm.inputs
    # ---- epilogue on accumulators ------------------------------------------------------
    epi_inputs = epilogue_inputs(k, epilogue)
    if cfg.KSPLIT > 1:
        return _ksplit_finish(L, g, k, mm, epilogue, epi_inputs, out_shape, bidx, batch_shape, M, N, K, BM, BN, WM, WN,
                              MI, TMW, TNW, NACC, THREADS, lds_bytes, guard_m, guard_n, idx_t, cfg, dt, tb, batch, fname)
    if cfg.DIRECT:
        staged = direct_staged_epilogue_lines(g, k, mm, epilogue, epi_inputs, out_shape, bidx, batch_shape, M, N, BM,
                                              BN, WM, WN, TMW, TNW, NACC, guard_m, guard_n, idx_t, cfg)
    else:
        staged = staged_epilogue_lines(g, k, mm, epilogue, epi_inputs, out_shape, bidx, batch_shape, M, N, BM, BN, WM,
                                       WN, MI, TMW, TNW, NACC, THREADS, lds_bytes, guard_m, guard_n, idx_t)
    if staged is not None:
        L += staged
        L.append("}")
        grid = (-(-N // BN), -(-M // BM), batch)
        meta = {"family": "matmul", "config": cfg.as_dict(), "dtype": dt.value, "M": M, "N": N, "K": K,
                "batch": batch, "trans_b": tb, "lds_bytes": lds_bytes, "flops": 2.0 * M * N * K * batch,
                "epilogue": "lds-staged"}
        return "\n".join(L), Launch(fname, grid, (THREADS, 1, 1), 0, meta)
    nrow_regs = NACC
    if MI == 32:
        row_of = "(r / 4) * 8 + (lane / 32u) * 4 + (r % 4)"
        col_of = "lane % 32u"
    else:
        row_of = "(lane / 16u) * 4 + r"
        col_of = "lane % 16u"
    L.append("#pragma unroll")
    L.append(f"  for (int x = 0; x < {TMW}; ++x)")
    L.append("#pragma unroll")
    L.append(f"  for (int y = 0; y < {TNW}; ++y)")
    L.append("#pragma unroll")
    L.append(f"  for (int r = 0; r < {nrow_regs}; ++r) {{")
    L.append(f"    const {idx_t} i = m0 + wm * {BM // WM}u + x * {MI}u + {row_of};")
    L.append(f"    const {idx_t} j = n0 + wn * {BN // WN}u + y * {MI}u + {col_of};")
    conds = ([f"i < {M}u"] if guard_m else []) + ([f"j < {N}u"] if guard_n else [])
    if conds:
        L.append(f"    if ({' && '.join(conds)}) {{")
    L.append(f"    const float {g.names[id(mm)]} = acc[x][y][r];")
    local = {id(mm): g.names[id(mm)]}
    full_idx = list(bidx) + ["i", "j"]
    for n in epi_inputs:
        consumer = next((c for c in epilogue if n in c.inputs), epilogue[0] if epilogue else mm)
        st = access_strides(n, consumer, out_shape)
        terms = [v if s == 1 else f"{v} * {s}u" for v, s in zip(full_idx, st) if s]
        off = " + ".join(terms) if terms else "0u"
        L.append(f"    const float {g.names[id(n)]}_e = tj_ld({g.names[id(n)]}_p[{off}]);")
        local[id(n)] = f"{g.names[id(n)]}_e"
    for n in epilogue:
        L.append(f"    const float {g.names[id(n)]} = {emit_expr(n, local)};")
        local[id(n)] = g.names[id(n)]
    obase = f"bi * {M * N}u + " if batch_shape else ""
    for jj, o in enumerate(k.outputs):
        L.append(f"    tj_st(out{jj}_p + {obase}i * {N}u + j, {local[id(o)]});")
    if conds:
        L.append("    }")
    L.append("  }")
    L.append("}")

    grid = (-(-N // BN), -(-M // BM), batch)
    meta = {"family": "matmul", "config": cfg.as_dict(), "dtype": dt.value, "M": M, "N": N, "K": K, "batch": batch,
            "trans_b": tb, "lds_bytes": lds_bytes, "flops": 2.0 * M * N * K * batch}
    return "\n".join(L), Launch(fname, grid, (THREADS, 1, 1), 0, meta)
