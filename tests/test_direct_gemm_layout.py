"""The direct-to-LDS GEMM schedule, checked on the CPU from its generated source.

The kernel writes LDS through DMA (each load instruction places lane ``l``'s 16 bytes
at byte ``16 l`` of a 1 KiB block, so the swizzle lives in *which* global chunk each
lane fetches) and reads MFMA fragments with a different set of expressions.  These
tests evaluate both sets of expressions exactly as generated, for every wave and
lane, and check that (a) the DMA fills each LDS slot of a stage exactly once, (b)
every fragment read returns the (row, k-chunk) the 32x32x16 MFMA expects in that
lane (32x32x16: row l % 32, chunk 2 ks + l / 32; 16x16x32: row l % 16, chunk
4 ks + sigma(l / 16), sigma swapping the two bits), and (c) the 32 lanes the LDS
serves in one pass hit 32 distinct 16-byte bank groups.  The model -- a 16-byte read
served 32 lanes at a time (lanes 0-31, then 32-63) over 128 four-byte banks (512
bytes) -- is the one that fits every rocprofv3 SQ_LDS_BANK_CONFLICT reading taken:
zero for the 32x32 layout, one extra pass per read for a 16x16 layout with k-groups
0 and 1 in chunks c and c+1 (rows r and r ^ 8 collide), zero once they sit in c and
c+2, and zero for the flash-attention kernel's 272-byte row pitch (32 consecutive
rows on 32 distinct groups).  Groupings of 16 consecutive lanes, or of 8 + 8 lanes,
contradict at least one of these readings as the only condition.  The 32-lane condition
is necessary, not sufficient: the flash kernel's unpadded 256-byte K rows with a swizzle
that met it but put rows 2k and 2k + 1 of each 16 consecutive lanes on one bank group
measured 1.7e7 conflict cycles per launch, and 0 once each 16 lanes also spread over 256
bytes (its own test checks both).  The GEMM layouts here meet that too: with 128-byte
rows, the rows of one parity among 16 consecutive lanes sit at distinct chunks.  The
wait-count immediate is pinned against the assembler's own decoding of a compiled kernel."""
import re
import shutil
import subprocess

import pytest

import tensorjit as tj
import tensorjit.compiler as C
from tensorjit.backends import hip_backend as hb
from tensorjit.backends import hip_gemm as hg
from tensorjit.ir import DType, TensorType
from tensorjit.runtime.autotune import MatmulConfig

DIRECT = MatmulConfig(256, 256, 64, 4, 2, 2, 32, 1, 8, 0, 0, 1)
DIRECT_N128 = MatmulConfig(256, 128, 64, 4, 2, 2, 32, 1, 8, 0, 0, 1)
DIRECT16 = MatmulConfig(256, 256, 64, 4, 2, 2, 16, 1, 8, 0, 0, 1)
DIRECT16_N128 = MatmulConfig(256, 128, 64, 4, 2, 2, 16, 1, 8, 0, 0, 1)
ALL_DIRECT = [DIRECT, DIRECT_N128, DIRECT16, DIRECT16_N128]
DIRECT_IDS = ["256x256", "256x128", "256x256_mi16", "256x128_mi16"]
# fp32 operands: 32-deep K tiles (the same 128-byte rows), 16x16x4 MFMAs
F32_DIRECT = [MatmulConfig(128, 128, 32, 4, 2, 2, 16, 1, 8, 0, 0, 1), MatmulConfig(256, 128, 32, 4, 2, 2, 16, 1, 8, 0, 0, 1),
              MatmulConfig(128, 256, 32, 4, 2, 2, 16, 1, 8, 0, 0, 1), MatmulConfig(64, 64, 32, 4, 2, 2, 16, 1, 8, 0, 0, 1)]
F32_IDS = ["f32_128x128", "f32_256x128", "f32_128x256", "f32_64x64"]


def _source(cfg, M=256, N=256, K=64, epi="plain", dt=DType.bf16):
    fns = {"plain": (lambda x, w: tj.linear(x, w), [(M, K), (N, K)]),
           "residual": (lambda x, w, r: tj.linear(x, w) + r, [(M, K), (N, K), (M, N)]),
           "bias_gelu": (lambda x, w, b: tj.gelu(tj.linear(x, w, b)), [(M, K), (N, K), (N,)])}
    fn, shapes = fns[epi]
    p = C.lower(tj.trace(fn, [TensorType(s, dt) for s in shapes]), "hip")
    return hb.generate(p, {0: cfg})


def _c_eval(expr: str, env: dict) -> int:
    """Evaluate a generated unsigned-int C expression (literals with a u suffix,
    + * ^ & >> and parentheses) in Python."""
    py = re.sub(r"(\d+)u\b", r"\1", expr)
    return int(eval(py, {}, dict(env))) & 0xFFFFFFFF


@pytest.mark.parametrize("cfg", ALL_DIRECT + F32_DIRECT, ids=DIRECT_IDS + F32_IDS)
def test_dma_placement_and_fragment_reads_agree(cfg):
    """(fp32: the same 128-byte rows hold 32 k; a lane's 16-byte chunk holds 4 consecutive k,
    element j of which feeds the group's j-th 16x16x4 MFMA, so the (row, chunk) checks are
    the bf16 16x16x32 kernel's.)"""
    f32 = cfg.TK == 32
    esz, K = (4, 32) if f32 else (2, 64)
    src, launches = _source(cfg, M=cfg.TM, N=cfg.TN, K=K, dt=DType.f32 if f32 else DType.bf16)
    nw, WM, WN, MI = cfg.num_warps, cfg.WM, cfg.WN, cfg.MI
    kc = 2 if MI == 32 else 4                     # 16-byte chunks of K per sub-step
    fofs = {int(i): e for i, e in re.findall(r"  fofs\[(\d+)\] = (.*);\n", src)}
    assert sorted(fofs) == list(range(4))
    for op, rows, wdim, rowdim in (("A", cfg.TM, WM, cfg.TM // WM), ("B", cfg.TN, WN, cfg.TN // WN)):
        vo = dict(re.findall(rf"  vo{op}\[(\d+)\] = (.*);\n", src))
        dst = re.findall(rf"raw_ptr_buffer_load_lds\(rs{op}, \(__attribute__\(\(address_space\(3\)\)\) void\*\)"
                         rf"\({op}s0 \+ (.*?)\), 16, vo{op}\[(\d+)\], \(int\)\(\(0\) \* 128u\), 0, 0\);", src)
        assert vo and dst and len({i for _, i in dst}) == len(vo), op
        slots = {}
        for wv in range(nw):
            for lane in range(64):
                env = {"m0": 0, "n0": 0, "wv": wv, "lane": lane, "drow": lane >> 3}
                for lds_expr, i in dst:
                    off = _c_eval(vo[i], env)                # global byte offset of this lane's 16 bytes
                    g_row, g_col = divmod(off // esz, K)
                    assert g_col % (16 // esz) == 0
                    slot = (_c_eval(lds_expr, env) + lane * 16) // 16
                    assert slot not in slots, (op, wv, lane, i)
                    slots[slot] = (g_row, g_col // (16 // esz))
        assert sorted(slots) == list(range(rows * K * esz // 16)), op      # every 16-byte slot filled once
        # fragment reads: lane l of wave (wm, wn), tile t, sub-step ks wants row base + MI t + l % MI,
        # 16-byte chunk kc ks + l / MI (8 bf16 of k per lane)
        fsw = re.search(r"const unsigned int fsw = (.*);", src).group(1)
        base = re.search(rf"const unsigned int {'arow' if op == 'A' else 'brow'} = (.*);", src).group(1)
        vt = "tj_f32x4" if f32 else "tj_bf16x8"
        reads = re.findall(rf"f{'a' if op == 'A' else 'b'}(?:\[\d\])?\[(\d)\] = \*\(const {vt}\*\)\({op}s0 \+ "
                           rf"{'arow' if op == 'A' else 'brow'} \+ fofs\[(\d)\] \+ (\d+)u\);", src)
        # every (tile, sub-step) pair is read, each with its own offset register
        assert len(set(reads)) == (rowdim // MI) * (64 // (8 * kc)), (op, sorted(set(reads)))
        if f32:
            # every fp32 MFMA takes element j of a fragment pair read with the same chunk offsets
            assert re.search(r"mfma_f32_16x16x4f32\(fa\[\d+\]\[3\], fb\[\d\]\[\d+\]\[3\]", src)

        def lane_env(lane, w):
            env = {"fr": lane & (MI - 1), "fh": lane // MI, "wm": w, "wn": w}
            env["fsw"] = _c_eval(fsw, env)
            if MI == 16:
                env["fg"] = _c_eval(re.search(r"const unsigned int fg = (.*);", src).group(1), env)
            return env

        def kgroup(lane):
            g = lane // MI
            return ((g & 1) << 1) | (g >> 1) if MI == 16 else g

        def sub_step(t, f):
            if MI == 32:
                return f
            assert f % 2 == t % 2, (t, f)            # odd 16-row tiles take the odd offsets
            return f // 2

        for w in range(wdim):
            for lane in range(64):
                env = lane_env(lane, w)
                for t, f, xoff in set(reads):
                    t, f = int(t), int(f)
                    addr = _c_eval(base, env) + _c_eval(fofs[f], env) + int(xoff)
                    want = (w * rowdim + t * MI + (lane & (MI - 1)), kc * sub_step(t, f) + kgroup(lane))
                    assert slots[addr // 16] == want, (op, w, lane, t, f)
        # bank groups: the 32 lanes served in one pass touch 32 distinct 16-byte groups of 512 bytes
        for w in range(wdim):
            for t, f, xoff in set(reads):
                for half in range(2):
                    grp = []
                    for lane in range(32 * half, 32 * half + 32):
                        env = lane_env(lane, w)
                        grp.append(((_c_eval(base, env) + _c_eval(fofs[int(f)], env) + int(xoff)) // 16) % 32)
                    assert len(set(grp)) == 32, (op, w, t, f, half, grp)


@pytest.mark.parametrize("epi", ["plain", "residual", "bias_gelu"])
@pytest.mark.parametrize("shape", [(256, 256, 64), (300, 520, 192), (1024, 768, 4096)])
def test_direct_kernels_compile_for_gfx950(epi, shape, tj_env):
    M, N, K = shape
    for cfg in ALL_DIRECT:
        src, launches = _source(cfg, M, N, K, epi)
        assert launches[0].meta["config"]["DIRECT"] == 1
        assert launches[0].meta.get("epilogue") == "lds-staged"
        assert "raw_ptr_buffer_load_lds" in src and "__builtin_amdgcn_s_waitcnt(0x0F70);" in src
        hb.compile_source(src, "gfx950")


def test_direct_config_rules():
    p = C.lower(tj.trace(lambda x, w: tj.linear(x, w), [TensorType((512, 200), DType.bf16),
                                                       TensorType((512, 200), DType.bf16)]), "hip")
    mm = p.kernels[0].anchor
    assert not hb.config_ok(DIRECT, DType.bf16, mm)                        # K not a multiple of 64
    p = C.lower(tj.trace(lambda x, w: tj.matmul(x, w), [TensorType((512, 256), DType.bf16),
                                                       TensorType((256, 512), DType.bf16)]), "hip")
    assert not hb.config_ok(DIRECT, DType.bf16, p.kernels[0].anchor)       # NN layout
    assert not hb.config_ok(DIRECT, DType.f32)                             # 16-bit operands only
    assert not hb.config_ok(MatmulConfig(256, 256, 32, 4, 2, 2, 32, 1, 8, 0, 0, 1), DType.bf16)   # TK must be 64


@pytest.mark.skipif(shutil.which("llvm-objdump") is None and not __import__("os").path.exists(
    "/opt/rocm/llvm/bin/llvm-objdump"), reason="llvm-objdump not available")
def test_vmcnt_immediate_decodes_as_intended(tmp_path):
    ns = [0, 5, 15, 16, 24, 63]
    # one wait per kernel: inside one kernel the compiler merges redundant waits
    src = "\n".join(f'extern "C" __global__ void probe{n}() {{ __builtin_amdgcn_s_waitcnt({hg._vmcnt_only(n)}); }}'
                    for n in ns)
    code = hb.compile_source(src, "gfx950")
    (tmp_path / "p.co").write_bytes(code)
    objdump = shutil.which("llvm-objdump") or "/opt/rocm/llvm/bin/llvm-objdump"
    dis = subprocess.run([objdump, "-d", "--mcpu=gfx950", str(tmp_path / "p.co")], capture_output=True,
                         text=True, check=True).stdout
    waits = [re.sub(r"\s*(expcnt\(7\)|lgkmcnt\(15\))", "", w).strip() for w in re.findall(r"s_waitcnt\s+([^\n/]*)", dis)]
    assert waits == [f"vmcnt({n})" for n in ns], waits      # expcnt / lgkmcnt left at their maxima
