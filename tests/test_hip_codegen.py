"""hip backend code generation, checked on the CPU: every generated program must
compile for gfx950 with hipRTC (the same compiler the runtime uses), and the
launch geometry / kernel selection must be what the design says.  Mirrors the
reference's host type-check of its generated CUDA (tests/test_cuda_backend.py:20-65),
with a real device compiler instead of a host stub."""
import pytest

import tensorjit as tj
import tensorjit.compiler as C
from tensorjit.backends import hip_backend as hb
from tensorjit.ir import DType, TensorType
from tensorjit.runtime.autotune import HIP_CANDIDATES, HIP_F32_CANDIDATES, MatmulConfig

CASES = {
    "mlp": (lambda x, g, w1, b1, w2, b2: x + tj.linear(tj.gelu(tj.linear(tj.layer_norm(x, g), w1, b1)), w2, b2),
            [(64, 128), (128,), (256, 128), (256,), (128, 256), (128,)]),
    "rows": (lambda x, w: (tj.softmax(x), tj.rms_norm(x, w), tj.sum(x * x), tj.max(x, keepdim=True)), [(8, 100), (100,)]),
    "bmm": (lambda a, b: tj.relu(tj.matmul(a, b)).sum(axis=2), [(2, 3, 8, 16), (3, 16, 8)]),
    "pointwise": (lambda a, b: tj.where(a, tj.maximum(a, b), tj.minimum(a, b)) + tj.exp(a) ** 2.0, [(4, 5, 6), (6,)]),
    "movement": (lambda t: tj.exp(tj.permute(t, 2, 0, 1)).reshape(5, 12) + 1.0, [(3, 4, 5)]),
    "gemm": (lambda x, w, b: tj.gelu(tj.linear(x, w, b)), [(64, 128), (256, 128), (256,)]),
    "eltwise_cfg2": (lambda x, a, b, c: tj.gelu(x * a + b) * tj.sigmoid(c) + x, [(64, 4096), (4096,), (4096,), (64, 4096)]),
    "long_reduce": (lambda x: tj.sum(x * x), [(3, 100000)]),
}


def _program(name, dtype):
    fn, shapes = CASES[name]
    return C.lower(tj.trace(fn, [TensorType(s, dtype) for s in shapes]), "hip")


@pytest.mark.parametrize("dtype", [DType.f32, DType.f16, DType.bf16])
@pytest.mark.parametrize("name", list(CASES))
def test_generated_hip_compiles_for_gfx950(name, dtype, tj_env):
    src, launches = hb.generate(_program(name, dtype))
    assert 'extern "C" __global__' in src and "__launch_bounds__" in src
    assert all(l.block[0] <= 1024 and l.block[0] % 64 == 0 for l in launches)
    code = hb.compile_source(src, "gfx950")
    assert code[:4] == b"\x7fELF" or len(code) > 1000


def test_source_is_hip_and_specialised():
    src, _ = hb.generate(_program("eltwise_cfg2", DType.f32))
    assert "blockIdx.x" in src and "4096" in src and "tj_gelu(" in src and "tj_sigmoid(" in src
    assert "cuda" not in src.lower() and "nvcuda" not in src


def test_mfma_selected_for_half_precision_and_fp32():
    for dt, needle in [(DType.bf16, "mfma_f32_32x32x16_bf16"), (DType.f16, "mfma_f32_32x32x16_f16")]:
        src, _ = hb.generate(_program("gemm", dt), {0: MatmulConfig(64, 64, 64, 4, 2, 2, 32)})
        assert needle in src
    src, _ = hb.generate(_program("gemm", DType.f32), {0: MatmulConfig(64, 64, 16, 4, 2, 2, 32)})
    assert "mfma_f32_32x32x2f32" in src


def test_launch_geometry():
    p = _program("mlp", DType.f32)
    assert [k.kind for k in p.kernels] == ["row", "matmul", "matmul"]
    cfg = MatmulConfig(64, 64, 32, 4, 2, 2, 16)
    _, launches = hb.generate(p, {1: cfg, 2: cfg})
    assert launches[0].grid == (64, 1, 1) and launches[0].block == (64, 1, 1)   # one workgroup per row
    assert launches[1].grid == (4, 1, 1) and launches[2].grid == (2, 1, 1)     # 256/64 and 128/64 column tiles


def test_row_kernel_geometry_for_benchmark_rows():
    from tensorjit.backends.hip_kernels import RowShape, row_geometry, row_shape

    # rows of 8-16 KiB: one workgroup per row, one 16-byte chunk per lane; with two or more
    # reductions 256 lanes and several chunks when the rows pass 8 KiB or no input is
    # broadcast over rows (softmax; a LayerNorm gain is)
    assert row_shape(4096, 8, False) == RowShape(512, 1, False, 1)     # config 3 RMS bf16
    assert row_shape(4096, 8, False, reductions=2) == RowShape(512, 1, False, 1)    # config 3 LN bf16 (gain)
    assert row_shape(2048, 4, False, reductions=2, whole_row_inputs=True) == RowShape(256, 2, False, 1)  # softmax
    assert row_shape(4096, 4, False) == RowShape(1024, 1, False, 1)    # fp32 N=4096
    assert row_shape(4096, 4, False, reductions=3) == RowShape(256, 4, False, 1)    # 16 KiB rows, gain or not
    assert row_shape(1200, 4, False, reductions=2, whole_row_inputs=True) == RowShape(256, 2, False, 1)
    assert row_shape(1200, 4, False, reductions=2) == RowShape(320, 1, False, 1)
    # rows up to 4 KiB: one wave per row, 4 rows per workgroup
    assert row_shape(2048, 8, False) == RowShape(64, 4, False, 4)      # config 5 softmax bf16
    assert row_shape(768, 4, False) == RowShape(64, 3, False, 4)       # config 1 LayerNorm fp32
    assert row_shape(70, 1, False) == RowShape(64, 2, False, 4)        # unvectorised odd rows
    # longer rows: several chunks per lane, then a rolled loop
    assert row_shape(8192, 4, False) == RowShape(256, 8, False, 1)
    assert row_shape(16384, 4, False) == RowShape(512, 8, False, 1)      # 12+ chunks at 256 lanes
    assert row_shape(16384, 4, True) == RowShape(256, 16, False, 1)      # a single reduction keeps 256
    assert row_geometry(4096, 8, False) == (256, 2, False)
    assert row_shape(100000, 4, True).streaming is True                # long stand-alone reductions stream


def test_row_kernel_launch_shapes():
    """Wave-per-row kernels put 4 rows in a workgroup when there are rows enough to fill the
    chip (a ragged last workgroup returns its extra waves), else one row per workgroup; the
    reductions are wave-only there (no LDS array), and 8 KiB rows take 512-lane workgroups with
    one reduction, 256-lane workgroups with two."""
    import tensorjit as tj
    from tensorjit.compiler import lower

    def launch(shape, dt, fn=lambda s: tj.softmax(s)):
        p = lower(tj.trace(fn, [TensorType(shape, dt)]), "hip")
        src, ls = hb.generate(p)
        return src, ls[0]

    src, l = launch((262144, 2048), DType.bf16)
    assert l.grid == (65536, 1, 1) and l.block == (256, 1, 1) and "tj_red" not in src
    assert "threadIdx.x >> 6" in src and "return;" not in src.split("tj0_")[1]
    src, l = launch((1000, 2048), DType.bf16)
    assert l.grid == (1000, 1, 1) and l.block == (64, 1, 1)        # too few rows for 4 per workgroup
    src, l = launch((4098, 1000), DType.f32)
    assert l.grid == (1025, 1, 1) and l.block == (256, 1, 1) and "if (r >= 4098u) return;" in src
    src, l = launch((65536, 2048), DType.f32)
    assert l.grid == (65536, 1, 1) and l.block == (256, 1, 1) and "tj_red" in src     # two reductions
    src, l = launch((65536, 2048), DType.f32, fn=lambda s: tj.sum(s * s, axis=-1))
    assert l.grid == (65536, 1, 1) and l.block == (512, 1, 1) and "tj_red" in src     # one


def test_every_candidate_config_generates_valid_code():
    p16 = _program("gemm", DType.bf16)
    p32 = _program("gemm", DType.f32)
    for cands, p, dt in [(HIP_CANDIDATES, p16, DType.bf16), (HIP_F32_CANDIDATES, p32, DType.f32)]:
        for cfg in cands:
            if not hb.config_ok(cfg, dt, p.kernels[0].anchor):
                continue
            src, launches = hb.generate(p, {0: cfg})
            assert launches[0].meta["lds_bytes"] <= 160 * 1024


@pytest.mark.parametrize("dtype,cands", [(DType.bf16, HIP_CANDIDATES), (DType.f32, HIP_F32_CANDIDATES)])
@pytest.mark.parametrize("shape", [(256, 512), (16, 512), (512, 4096)])
def test_epilogue_may_read_the_gemm_operand(dtype, cands, shape):
    """``x + linear(x, w)``: the epilogue's residual is the product's A operand, so the
    epilogue inputs are the kernel inputs its nodes read, operands included; every
    candidate tiling generates it and reads x in the epilogue."""
    types = [TensorType(shape, dtype), TensorType((shape[1], shape[1]), dtype)]
    p = C.lower(tj.trace(lambda x, w: x + tj.linear(x, w), types), "hip")
    plain = C.lower(tj.trace(lambda x, w: tj.linear(x, w), types), "hip")
    (k,) = p.kernels
    assert [n.op for n in k.nodes] == ["matmul", "add"]
    tried = 0
    for cfg in cands:
        if hb.config_ok(cfg, dtype, k.anchor):
            src, _ = hb.generate(p, {0: cfg})
            # x is read once more than by the plain product: by the epilogue
            assert src.count("in0_p") > hb.generate(plain, {0: cfg})[0].count("in0_p"), cfg
            tried += 1
    assert tried >= 10


def test_config2_row_group_lowers_to_vectorised_flat_loop():
    src, launches = hb.generate(_program("eltwise_cfg2", DType.f32))
    assert launches[0].meta["family"] == "pointwise" and launches[0].meta["vec"] == 4
    assert "tj_ldv(" in src and "tj_stv(" in src


def test_skinny_decode_shapes_use_the_streaming_kernel():
    for m in (1, 7, 16):
        g = tj.trace(lambda x, w, b: tj.gelu(tj.linear(x, w, b)),
                     [TensorType(s, DType.bf16) for s in [(m, 8192), (8192, 8192), (8192,)]])
        p = C.lower(g, "hip")
        cfg = hb.analytic_config(p.kernels[0])
        assert cfg.SPLIT_K > 1, cfg
        src, launches = hb.generate(p, {0: cfg})
        assert launches[0].meta["family"] == "matmul_skinny" and launches[0].grid[0] == 8192 // cfg.TN
        hb.compile_source(src, "gfx950")


def test_tile_order_is_a_bijection_when_compiled_for_the_host(tmp_path):
    """The XCD-aware tile order text is compiled with gcc on the CPU (blockIdx as
    arguments) and must visit every tile of the grid exactly once."""
    import subprocess

    from tensorjit.backends.hip_gemm import tile_order_lines

    cases = [(32, 32, 8), (64, 48, 8), (7, 9, 8), (3, 40, 4), (33, 17, 8), (1, 16, 8), (16, 1, 8)]
    fns = []
    for ci, (ntm, ntn, gm) in enumerate(cases):
        body = "\n".join(tile_order_lines(ntm, ntn, gm, 1, 1)).replace("blockIdx.x", "bx").replace("blockIdx.y", "by")
        fns.append(f"static void order{ci}(unsigned bx, unsigned by, unsigned* mo, unsigned* no) {{\n{body}\n"
                   "  *mo = m0; *no = n0; }")
    checks = []
    for ci, (ntm, ntn, gm) in enumerate(cases):
        checks.append(f"""  {{ static unsigned char seen[{ntm}][{ntn}]; unsigned m, n;
    for (unsigned by = 0; by < {ntm}u; ++by) for (unsigned bx = 0; bx < {ntn}u; ++bx) {{
      order{ci}(bx, by, &m, &n); if (m >= {ntm}u || n >= {ntn}u || seen[m][n]++) return {ci + 1}; }} }}""")
    src = "\n".join(fns) + "\nint main(void) {\n" + "\n".join(checks) + "\n  return 0;\n}\n"
    c = tmp_path / "order.c"
    c.write_text(src)
    exe = tmp_path / "order"
    subprocess.run(["gcc", "-O1", "-o", str(exe), str(c)], check=True)
    assert subprocess.run([str(exe)]).returncode == 0


def test_persistent_tile_order_visits_every_tile_once_on_its_xcd(tmp_path):
    """Persistent workgroups b < min(G, T) walk virtual ids b, b + G, ... < T through the
    same tile order (compiled with gcc on the CPU): every tile exactly once, and every
    virtual id of a workgroup on the workgroup's own XCD (id mod 8)."""
    import subprocess

    from tensorjit.backends.hip_gemm import tile_order_lines

    cases = [(32, 32, 8, 256), (4, 4, 8, 8), (3, 5, 8, 8), (43, 32, 8, 256), (2, 2, 8, 256)]
    fns, checks = [], []
    for ci, (ntm, ntn, gm, G) in enumerate(cases):
        body = "\n".join(tile_order_lines(ntm, ntn, gm, 1, 1, vid="v", names=("m0", "n0"), sfx="p"))
        fns.append(f"static void order{ci}(unsigned v, unsigned* mo, unsigned* no) {{\n{body}\n  *mo = m0; *no = n0; }}")
        T = ntm * ntn
        checks.append(f"""  {{ static unsigned char seen[{ntm}][{ntn}]; unsigned m, n, cnt = 0;
    for (unsigned b = 0; b < {min(G, T)}u; ++b) for (unsigned v = b; v < {T}u; v += {G}u) {{
      if (v % 8u != b % 8u) return 100 + {ci};
      order{ci}(v, &m, &n); if (m >= {ntm}u || n >= {ntn}u || seen[m][n]++) return {ci + 1}; ++cnt; }}
    if (cnt != {T}u) return 200 + {ci}; }}""")
    src = "\n".join(fns) + "\nint main(void) {\n" + "\n".join(checks) + "\n  return 0;\n}\n"
    c = tmp_path / "porder.c"
    c.write_text(src)
    exe = tmp_path / "porder"
    subprocess.run(["gcc", "-O1", "-o", str(exe), str(c)], check=True)
    assert subprocess.run([str(exe)]).returncode == 0


PERSIST = MatmulConfig(256, 256, 64, 4, 2, 2, 16, 1, 8, 0, 0, 1, 1, 256)


def _gemm(kind):
    """(function, operand shapes) of the persistent-kernel applicability cases."""
    lin = lambda x, w: tj.linear(x, w)                      # noqa: E731
    res = lambda x, w, r: tj.linear(x, w) + r               # noqa: E731
    return {
        "c4_bias_gelu": (lambda x, w, b: tj.gelu(tj.linear(x, w, b)), [(8192, 8192), (8192, 8192), (8192,)]),
        "c5_folded_residual": (res, [(4, 2048, 4096), (4096, 4096), (4, 2048, 4096)]),
        "c5_row_broadcast_residual": (res, [(4, 2048, 4096), (4096, 4096), (2048, 4096)]),
        "ragged_m": (lin, [(8000, 4096), (4096, 4096)]),
        "k_not_multiple_of_128": (lin, [(4096, 4160), (4096, 4160)]),
        "k_below_256": (lin, [(4096, 128), (4096, 128)]),
        "per_batch_weight": (lambda x, w: tj.matmul(x, tj.transpose(w, -1, -2)), [(4, 2048, 512), (4, 1024, 512)]),
    }[kind]


@pytest.mark.parametrize("kind,ok", [("c4_bias_gelu", True), ("c5_folded_residual", True),
                                     ("c5_row_broadcast_residual", True), ("ragged_m", False),
                                     ("k_not_multiple_of_128", False), ("k_below_256", False),
                                     ("per_batch_weight", False)])
def test_persistent_gemm_applies_to_whole_tiles_and_foldable_batches(kind, ok):
    fn, shapes = _gemm(kind)
    p = C.lower(tj.trace(fn, [TensorType(s, DType.bf16) for s in shapes]), "hip")
    assert hb.config_ok(PERSIST, DType.bf16, p.kernels[0].anchor) == ok
    # the workgroup count must keep every virtual id on its XCD, and only the direct
    # kernel has a persistent form
    assert not hb.config_ok(MatmulConfig(256, 256, 64, 4, 2, 2, 16, 1, 8, 0, 0, 1, 1, 100), DType.bf16,
                            p.kernels[0].anchor)
    assert not hb.config_ok(MatmulConfig(256, 256, 64, 4, 2, 2, 32, 1, 8, 0, 0, 1, 1, 256), DType.bf16,
                            p.kernels[0].anchor)


def test_configs_the_generators_cannot_schedule_are_rejected():
    """A direct tile whose per-wave DMA count overflows the 6-bit vmcnt (one wave over a
    256x256 tile: 64 loads), and a persistent tile whose wave columns (96) do not split a
    staged row evenly over the lanes, are invalid configs: gen_matmul raises ValueError."""
    # 3072 rows and columns: whole 192-wide tiles, so only the column split rejects cols96
    fn, shapes = (lambda x, w, b: tj.gelu(tj.linear(x, w, b))), [(3072, 4096), (3072, 4096), (3072,)]
    p = C.lower(tj.trace(fn, [TensorType(s, DType.bf16) for s in shapes]), "hip")
    anchor = p.kernels[0].anchor
    one_wave = MatmulConfig(256, 256, 64, 1, 1, 1, 16, 1, 8, 0, 0, 1)
    cols96 = MatmulConfig(192, 192, 64, 4, 2, 2, 16, 1, 8, 0, 0, 1, 1, 256)
    # their neighbours are valid: one wave over 128x128 (32 loads), 4 waves with 128 columns
    assert hb.config_ok(MatmulConfig(128, 128, 64, 1, 1, 1, 16, 1, 8, 0, 0, 1), DType.bf16, anchor)
    assert hb.config_ok(MatmulConfig(256, 256, 64, 4, 2, 2, 16, 1, 8, 0, 0, 1, 1, 256), DType.bf16, anchor)
    assert hb.config_ok(MatmulConfig(192, 192, 64, 4, 2, 2, 16, 1, 8, 0, 0, 1), DType.bf16, anchor)
    for cfg in (one_wave, cols96):
        assert not hb.config_ok(cfg, DType.bf16, anchor)
        with pytest.raises(ValueError, match="not valid"):
            hb.generate(p, {0: cfg})


def test_persistent_gemm_launch_lds_and_waits():
    """Config 4: 1024 tiles on 256 workgroups, two LDS stages plus the 32 KiB epilogue
    staging array (the whole 160 KiB); the waits before the next tile's first fragment
    reads (48: its K tile 1 and the 32 epilogue stores of each wave) and at its first
    barrier (32: the stores) leave the stores draining; a residual broadcast over the
    batch does not fold, and the direct kernel is generated instead."""
    fn, shapes = _gemm("c4_bias_gelu")
    p = C.lower(tj.trace(fn, [TensorType(s, DType.bf16) for s in shapes]), "hip")
    src, (l,) = hb.generate(p, {0: PERSIST})
    assert l.grid == (256, 1, 1) and l.block == (256, 1, 1) and l.meta["persistent"] == 256
    assert l.meta["lds_bytes"] == 160 * 1024 and l.meta["flops"] == 2.0 * 8192 ** 3
    assert "__builtin_amdgcn_s_waitcnt(0xcf70)" in src and "__builtin_amdgcn_s_waitcnt(0x8f70)" in src
    assert "_raw = *(const tj_u32x4*)" in src          # the bias is preloaded before the next K tile 1
    hb.compile_source(src, "gfx950")
    fn, shapes = _gemm("c5_folded_residual")
    p = C.lower(tj.trace(fn, [TensorType(s, DType.bf16) for s in shapes]), "hip")
    _, (l,) = hb.generate(p, {0: PERSIST})
    assert l.grid == (256, 1, 1) and l.meta["batch"] == 4 and l.meta["M"] == 2048
    assert l.meta["flops"] == 2.0 * 4 * 2048 * 4096 * 4096
    fn, shapes = _gemm("c5_row_broadcast_residual")
    p = C.lower(tj.trace(fn, [TensorType(s, DType.bf16) for s in shapes]), "hip")
    _, (l,) = hb.generate(p, {0: PERSIST})
    assert "persistent" not in l.meta and l.grid == (16, 8, 4)


def test_fp32_direct_to_lds_tiles():
    """fp32 operands take the direct-to-LDS schedule with 32-deep K tiles (the bf16 kernel's
    128-byte rows) and 16x16x4 MFMAs: NT layout, K a multiple of 32, tiles up to 128x256.
    Each 16-byte fragment read feeds 4 MFMAs (element j of A and B), j the outer pass."""
    def prog(M, N, K, tb=True):
        fn = (lambda x, w: tj.linear(x, w)) if tb else (lambda x, w: tj.matmul(x, w))
        shapes = [(M, K), (N, K) if tb else (K, N)]
        return C.lower(tj.trace(fn, [TensorType(s, DType.f32) for s in shapes]), "hip")

    d128 = MatmulConfig(128, 128, 32, 4, 2, 2, 16, 1, 8, 0, 0, 1)
    p = prog(4096, 1024, 4096)
    mm = p.kernels[0].anchor
    assert hb.config_ok(d128, DType.f32, mm)
    assert hb.config_ok(MatmulConfig(128, 256, 32, 4, 2, 2, 16, 1, 8, 0, 0, 1), DType.f32, mm)
    assert hb.config_ok(MatmulConfig(128, 128, 32, 4, 2, 2, 16, 1, 8, 0, 0, 1, 1, 256), DType.f32, mm)
    assert not hb.config_ok(MatmulConfig(256, 256, 32, 4, 2, 2, 16, 1, 8, 0, 0, 1), DType.f32, mm)
    assert not hb.config_ok(MatmulConfig(128, 128, 64, 4, 2, 2, 16, 1, 8, 0, 0, 1), DType.f32, mm)
    assert not hb.config_ok(MatmulConfig(128, 128, 32, 4, 2, 2, 32, 1, 8, 0, 0, 1), DType.f32, mm)
    assert not hb.config_ok(d128, DType.f32, prog(512, 512, 520).kernels[0].anchor)          # K % 32
    assert not hb.config_ok(d128, DType.f32, prog(512, 512, 512, tb=False).kernels[0].anchor)  # NN
    src, _ = hb.generate(p, {0: d128})
    body = src[len(hb.PRELUDE):]
    assert "*(const tj_f32x4*)(As0 + arow" in body
    assert "__builtin_amdgcn_mfma_f32_16x16x4f32(fa[0][3], fb[0][0][3]" in body
    assert "__builtin_amdgcn_raw_ptr_buffer_load_lds" in body
    hb.compile_source(src, "gfx950")


def test_k_split_gemm_sums_in_its_last_workgroup():
    """K split over workgroups, default form: one launch owning a workspace of
    batch x splits x M x N fp32 partials; the last of a tile's workgroups (a counter per
    output tile in a zero-initialised device array of the code object, reset by that
    workgroup) sums them: partials written by agent-scope stores and waited for before the
    counter moves, read back with sc1 (agent-coherent) buffer loads."""
    fn = lambda x, w, b: tj.gelu(tj.linear(x, w, b))
    p = C.lower(tj.trace(fn, [TensorType(s, DType.f32) for s in [(512, 3072), (768, 3072), (768,)]]), "hip")
    cfg = MatmulConfig(64, 64, 32, 4, 2, 2, 16, 1, 8, 0, 0, 0, 8)
    src, launches = hb.generate(p, {0: cfg})
    assert len(launches) == 1 and launches[0].grid == (12, 8, 8) and launches[0].meta["fused_sum"]
    assert launches[0].meta["workspace"] == 8 * 512 * 768 * 4 and launches[0].meta["ws_arg"]
    assert f"__device__ unsigned int {launches[0].name}_cnt[96];" in src
    assert "__hip_atomic_store(ws_p + " in src and "__builtin_amdgcn_s_waitcnt(0x0F70);" in src
    assert "== 7u ? 1u : 0u" in src and src.count("raw_buffer_load_b128(rsW") == 1 and "__threadfence" not in src
    assert f"{launches[0].name}_cnt[ct_] = 0u;" in src
    hb.compile_source(src, "gfx950")


def test_k_split_gemm_has_a_partial_and_a_sum_launch(monkeypatch):
    """K split over workgroups, two-launch form (``TENSORJIT_HIP_KSPLIT_FUSED=0``): the
    partial-product launch owns a workspace of batch x splits x M x N fp32 values (placed
    after the planned intermediates in the arena) and both launches take it as their last
    argument."""
    monkeypatch.setenv("TENSORJIT_HIP_KSPLIT_FUSED", "0")
    fn = lambda x, w, b: tj.gelu(tj.linear(x, w, b))
    p = C.lower(tj.trace(fn, [TensorType(s, DType.f32) for s in [(512, 3072), (768, 3072), (768,)]]), "hip")
    cfg = MatmulConfig(64, 64, 32, 4, 2, 2, 16, 1, 8, 0, 0, 0, 8)
    assert hb.config_ok(cfg, DType.f32, p.kernels[0].anchor)
    src, launches = hb.generate(p, {0: cfg})
    assert [l.meta["kernel"] for l in launches] == [0, 0]
    assert launches[0].grid == (12, 8, 8) and launches[0].meta["workspace"] == 8 * 512 * 768 * 4
    assert launches[1].meta["family"] == "ksplit_sum" and launches[1].grid == (384, 1, 1)
    ws, arena = hb.workspace_layout(launches, 1000)
    assert ws == {0: (1024, 8 * 512 * 768 * 4)} and arena == 1024 + 8 * 512 * 768 * 4
    refs = hb.launch_args(launches, [[("in", 0), ("in", 1), ("in", 2), ("out", 0)]], ws)
    assert all(r[-1] == (hb.rt.ARENA, 1024, 8 * 512 * 768 * 4) for r in refs)
    hb.compile_source(src, "gfx950")
    # splits must divide K into whole K steps
    assert not hb.config_ok(MatmulConfig(64, 64, 32, 4, 2, 2, 16, 1, 8, 0, 0, 0, 7), DType.f32, p.kernels[0].anchor)


@pytest.mark.parametrize("case", ["pointwise_0x4", "pointwise_3x0", "softmax_0x8", "softmax_4x0", "matmul_m0", "matmul_k0"])
def test_zero_size_tensors_are_refused_before_codegen(case):
    """Every kernel assumes a non-empty iteration space (a pointwise kernel over [0, 4] would run
    one unguarded workgroup), so zero-size tensors raise NotImplementedError -- the signal that
    sends torch.compile back to eager -- before any source is generated."""
    fn, shapes = {
        "pointwise_0x4": (lambda a: tj.exp(a) + 1.0, [(0, 4)]),
        "pointwise_3x0": (lambda a: tj.exp(a) + 1.0, [(3, 0)]),
        "softmax_0x8": (lambda a: tj.softmax(a), [(0, 8)]),
        "softmax_4x0": (lambda a: tj.softmax(a), [(4, 0)]),
        "matmul_m0": (lambda a, b: tj.matmul(a, b), [(0, 8), (8, 4)]),
        "matmul_k0": (lambda a, b: tj.matmul(a, b), [(4, 0), (0, 4)]),
    }[case]
    p = C.lower(tj.trace(fn, [TensorType(s, DType.f32) for s in shapes]), "hip")
    with pytest.raises(NotImplementedError, match="zero-size"):
        hb.generate(p)


def _loads(fn, shapes, dt):
    src, _ = hb.generate(C.lower(tj.trace(fn, [TensorType(s, dt) for s in shapes]), "hip"))
    body = src.split('extern "C"', 1)[1]
    return [ln.strip().split(" + ")[0] for ln in body.splitlines() if "tj_ldv" in ln]


def test_nontemporal_loads_for_streamed_inputs_past_the_mall(monkeypatch):
    """Inputs read once (no broadcast dim) get the nontemporal hint when together they
    exceed the 256 MiB MALL; broadcast operands never do, and kernels whose streamed
    inputs fit keep plain loads (their inputs may stay cached from the producer or the
    previous call), however much they write."""
    monkeypatch.delenv("TENSORJIT_HIP_NT_LOADS", raising=False)
    c2 = lambda x, a, b, c: tj.gelu(x * a + b) * tj.sigmoid(c) + x  # noqa: E731
    big = [(16384, 4096), (4096,), (4096,), (16384, 4096)]           # 512 MiB streamed in
    assert _loads(c2, big, DType.f32) == ["tj_ldv_nt(in0_p", "tj_ldv_nt(in1_p", "tj_ldv(in2_p", "tj_ldv(in3_p"]
    assert all(x.startswith("tj_ldv(") for x in _loads(c2, big, DType.bf16))     # exactly 256 MiB in
    small = [(4096, 4096), (4096,), (4096,), (4096, 4096)]
    assert all(x.startswith("tj_ldv(") for x in _loads(c2, small, DType.f32))
    rms = lambda x, g: tj.rms_norm(x, g)  # noqa: E731
    assert _loads(rms, [(65536, 4096), (4096,)], DType.bf16) == ["tj_ldv_nt(in0_p", "tj_ldv(in1_p"]
    assert all(x.startswith("tj_ldv(") for x in _loads(rms, [(8192, 4096), (4096,)], DType.bf16))
    # 128 MiB in, 256 MiB of traffic: plain loads
    assert all(x.startswith("tj_ldv(") for x in _loads(lambda s: tj.softmax(s), [(16384, 2048)], DType.f32))
    monkeypatch.setenv("TENSORJIT_HIP_NT_LOADS", "1")
    assert _loads(rms, [(8192, 4096), (4096,)], DType.bf16) == ["tj_ldv_nt(in0_p", "tj_ldv(in1_p"]
    monkeypatch.setenv("TENSORJIT_HIP_NT_LOADS", "0")
    assert all(x.startswith("tj_ldv(") for x in _loads(c2, big, DType.f32))


def test_tiled_transpose_plan_and_index_math():
    """The tiled transpose applies where the output's innermost dim is strided in the
    source and both 16-byte row starts are aligned; its tile index math (the loops of
    gen_copy_tiled, replayed on the CPU over every workgroup and lane) reproduces
    numpy's permute exactly, ragged edge tiles included."""
    import numpy as np
    from tensorjit.backends import hip_kernels as hk

    def plan(shape_in, perm, isz):
        cs = [int(np.prod(shape_in[i + 1:])) for i in range(len(shape_in))]
        return hk._tiled_transpose_plan(tuple(shape_in[p] for p in perm), tuple(cs[p] for p in perm), isz)

    assert plan((4, 64, 8, 32), (0, 2, 1, 3), 2) is None        # innermost dim stays contiguous: vector copy
    assert plan((100, 40), (1, 0), 2) is None                    # 100 bf16 rows: not 16-byte aligned
    assert plan((7, 64, 8), (2, 1, 0), 4) is None

    def replay(shape_in, perm, isz):
        x = np.arange(int(np.prod(shape_in)), dtype=np.int64).reshape(shape_in)
        ref = np.ascontiguousarray(np.transpose(x, perm)).reshape(-1)
        E0, s0, Er, Ir, batch = plan(shape_in, perm, isz)
        TT, vec, T = hk.TT, 16 // isz, hk.THREADS
        tc, tr = -(-E0 // TT), -(-Er // TT)
        vpr = TT // vec
        src, out = x.reshape(-1), np.full(ref.shape, -1, dtype=np.int64)
        for blk in range(tc * tr * int(np.prod([e for e, _, _ in batch]) if batch else 1)):
            c0, r0, bi, so, oo = (blk % tc) * TT, ((blk // tc) % tr) * TT, blk // (tc * tr), 0, 0
            for e, ost, sst in batch:
                so, oo, bi = so + (bi % e) * sst, oo + (bi % e) * ost, bi // e
            tile = np.zeros((TT, TT + vec), dtype=np.int64)
            for v in range(TT * vpr):
                c, r = v // vpr, (v % vpr) * vec
                if c0 + c < E0 and r0 + r < Er:
                    tile[c, r:r + vec] = src[so + (c0 + c) * s0 + r0 + r:][:vec]
            for v in range(TT * vpr):
                r, c = v // vpr, (v % vpr) * vec
                if c0 + c < E0 and r0 + r < Er:
                    o = oo + (r0 + r) * Ir + c0 + c
                    out[o:o + vec] = tile[c:c + vec, r]
        assert np.array_equal(out, ref), (shape_in, perm, isz)

    for shape_in, perm, isz in [((128, 64), (1, 0), 2), ((104, 48), (1, 0), 4), ((3, 40, 72), (2, 0, 1), 2),
                                ((5, 8, 16, 24), (3, 1, 0, 2), 4), ((2, 3, 96, 80), (0, 1, 3, 2), 2),
                                ((6, 5, 16, 8), (1, 3, 0, 2), 4)]:
        replay(shape_in, perm, isz)


def test_row_split_rule_and_index_math(monkeypatch):
    """Reductions over fewer rows than CUs, each row at least 512 KiB, split each row over
    workgroups.  The segment and chunk index math of the split kernel (replayed on the
    CPU over every workgroup, segment, chunk and lane) reads every element of every row
    exactly once, and every workgroup writes its own workspace slot."""
    import numpy as np
    from tensorjit.backends import hip_kernels as hk
    from tensorjit.runtime.autotune import CU_COUNT

    assert hk.row_split(CU_COUNT, 1 << 20, 4, 4) is None          # one workgroup per row fills the chip
    assert hk.row_split(8, 32768, 4, 4) is None                  # 128 KiB rows: one workgroup each
    assert hk.row_split(1, 1 << 26, 4, 4) == hk.RowSplit(8, 8192, CU_COUNT)
    assert hk.row_split(1, 65536, 4, 4) is None                  # 256 KiB: the combine launch costs more
    assert hk.row_split(1, 131072, 4, 4) == hk.RowSplit(1, 128, 128)   # short enough for one chunk a segment
    monkeypatch.setenv("TENSORJIT_HIP_ROW_SPLIT", "0")
    assert hk.row_split(1, 1 << 26, 4, 4) is None
    monkeypatch.setenv("TENSORJIT_HIP_ROW_SPLIT", "1")
    assert hk.row_split(37, 5000, 4, 4) == hk.RowSplit(1, 5, 5)

    def replay(nrows, N, vec, sp):
        T, NCH, S, SEGS = hk.SPLIT_THREADS, sp.chunks, sp.splits, sp.segments
        seen = np.zeros(nrows * N, dtype=np.int64)
        slots = np.zeros(nrows * S, dtype=np.int64)
        for blk in range(nrows * S):
            r, sb = blk // S, blk % S
            for seg in range(sb, SEGS, S):
                for c in range(NCH):
                    n0 = (np.arange(T) + (seg * NCH + c) * T) * vec
                    for n in n0[n0 < N]:
                        seen[r * N + n:r * N + n + vec] += 1
            slots[blk] += 1
        assert (seen == 1).all() and (slots == 1).all(), (nrows, N, vec, sp)

    for nrows, N, vec in [(1, 300000, 4), (3, 5000, 4), (2, 300001, 1), (5, 40000, 8), (1, 1 << 20, 4)]:
        replay(nrows, N, vec, hk.row_split(nrows, N, vec, 4))


@pytest.mark.parametrize("case", ["sum", "mse", "rms_bf16", "max_keepdim", "odd"])
def test_split_reductions_generate_and_compile(case, tj_env):
    cases = {
        "sum": (lambda x: tj.sum(x), [(1 << 23,)], DType.f32, "sum"),
        "mse": (lambda x, y: tj.mean((x - y) * (x - y), axis=-1), [(3, 300000)] * 2, DType.f32, "mean"),
        "rms_bf16": (lambda x: tj.sqrt(tj.mean(x * x, axis=-1) + 1e-5), [(8, 262144)], DType.bf16, "mean"),
        "max_keepdim": (lambda x: tj.max(x, axis=-1, keepdim=True) * 2.0, [(4, 262144)], DType.f32, "max"),
        "odd": (lambda x: tj.sum(tj.abs(x), axis=-1), [(2, 300001)], DType.f32, "sum"),
    }
    fn, shapes, dt, red = cases[case]
    p = C.lower(tj.trace(fn, [TensorType(s, dt) for s in shapes]), "hip")
    src, launches = hb.generate(p)
    part, comb = launches
    nrows = part.meta["rows"]
    assert comb.meta["family"] == "row_combine" and comb.grid == (nrows, 1, 1)
    assert part.grid == (nrows * part.meta["splits"], 1, 1) and part.meta["workspace"] == nrows * part.meta["splits"] * 4
    assert part.meta["ws_arg"] and comb.meta["ws_arg"]
    if red == "mean":
        assert f"acc / {float(shapes[0][-1])!r}f" in src
    hb.compile_source(src, "gfx950")


def test_long_rows_with_several_stages_fit_one_workgroup(tj_env):
    """Rows with several stages up to the hip row-fusion limit (32768) get one row kernel:
    256 lanes x up to 11 chunks (512 lanes from 12), then up to 1024 lanes x 32 values per
    lane per row array (odd lengths load one element per chunk), and the kernels compile
    for gfx950."""
    from tensorjit.backends import hip_kernels as hk

    assert hk.row_geometry(16384, 4, False) == (512, 8, False)
    assert hk.row_geometry(16384, 4, True) == (256, 16, False)
    assert hk.row_geometry(11264, 4, False) == (256, 11, False)
    assert hk.row_geometry(32768, 8, False) == (256, 16, False)        # 512 x 8 chunks of 8: too many values
    assert hk.row_geometry(32768, 4, False) == (1024, 8, False)
    assert hk.row_geometry(4097, 1, False) == (832, 5, False)
    assert hk.row_geometry(5001, 1, False) == (1024, 5, False)
    assert hk.row_geometry(32767, 1, False) == (1024, 32, False)
    assert hk.row_geometry(1 << 20, 4, True) == (1024, 256, True)      # a reduction streams
    with pytest.raises(NotImplementedError):
        hk.row_geometry(32769, 1, False)
    for n, dt in [(5001, DType.f32), (32767, DType.f32), (32768, DType.f32), (32768, DType.bf16), (20000, DType.f16)]:
        fn = lambda x, g: (tj.layer_norm(x, g), tj.softmax(x))  # noqa: E731
        p = C.lower(tj.trace(fn, [TensorType((4, n), dt), TensorType((n,), dt)]), "hip")
        assert [k.kind for k in p.kernels] == ["row", "row"], (n, dt)
        src, launches = hb.generate(p)
        for launch in launches:
            vec, T, nch = launch.meta["vec"], launch.meta["threads"], launch.meta["chunks"]
            assert T <= 1024 and T * nch * vec >= n and (T <= 256 or nch * vec <= hk.ROW_MAX_FLOATS)
        if n in (5001, 32768):
            hb.compile_source(src, "gfx950")


def test_transpose_then_reduce_folds_into_a_column_reduction(tj_env, monkeypatch):
    """A transpose whose only reader is a reduction of its last axis becomes one column
    reduction (with a folded elementwise prologue and the reduction's epilogue), unless the
    transpose reorders other axes, has another reader, or a row of B is under 512 bytes.
    Its block, column and row-slice decode (replayed on the CPU) visits every element of
    every (A, Rd, B) source once, and every partial lands in its own workspace slot."""
    import numpy as np
    from tensorjit.backends import hip_kernels as hk

    def plan(fn, shapes, dt=DType.f32):
        p = C.lower(tj.trace(fn, [TensorType(s, dt) for s in shapes]), "hip")
        return hb.fold_transpose_into_reduce(p)

    q = plan(lambda x: tj.max(x * 2.0 + 1.0, axis=0, keepdim=True), [(4096, 4096)])
    assert [k.kind for k in q.kernels] == ["colreduce"] and q.kernels[0].col == (1, 4096, 4096)
    q = plan(lambda x, g: tj.tanh(tj.mean(x, axis=1) * 0.5) + g, [(8, 4096, 1024), (8, 1024)], DType.bf16)
    assert [k.kind for k in q.kernels] == ["colreduce"] and q.kernels[0].col == (8, 4096, 1024)
    src, launches = hb.generate(q)
    assert [l.meta["family"] for l in launches] == ["colreduce", "colreduce_combine"]
    hb.compile_source(src, "gfx950")
    q = plan(lambda x: tj.sum(x, axis=1), [(2048, 8, 256)])
    src, (launch,) = hb.generate(q)                      # one slice of Rd: no combine launch
    assert launch.meta["splits"] == 1
    hb.compile_source(src, "gfx950")
    # not folded: a transpose that reorders the kept axes, a second reader, narrow rows, row kernels
    assert [k.kind for k in plan(lambda x: tj.sum(tj.permute(x, 2, 0, 1), axis=-1), [(3, 64, 256)]).kernels] == \
        ["copy", "reduce"]
    assert "colreduce" not in [k.kind for k in plan(
        lambda x: (tj.sum(tj.transpose(x, 0, 1), axis=-1), tj.transpose(x, 0, 1)), [(64, 256)]).kernels]
    assert "colreduce" not in [k.kind for k in plan(lambda x: tj.sum(x, axis=1), [(4, 300, 96)]).kernels]
    # a column mean subtracted back: the mean (with its epilogue) folds, the subtraction
    # stays a pointwise kernel
    assert [k.kind for k in plan(lambda x, g: x - tj.mean(x, axis=0) * g, [(512, 512), (512,)]).kernels] == \
        ["colreduce", "elementwise"]
    monkeypatch.setenv("TENSORJIT_HIP_COLREDUCE", "0")
    assert [k.kind for k in plan(lambda x: tj.sum(x, axis=0), [(4096, 4096)]).kernels] == ["copy", "reduce"]

    for A, Rd, B, vec in [(1, 600, 1024, 4), (8, 1000, 1024, 8), (5, 37, 168, 4), (3, 100, 200, 1), (512, 8, 256, 4)]:
        nb, RS, S = hk.col_layout(A, Rd, B, vec)
        L = -(-B // vec)
        seen = np.zeros(A * Rd * B, dtype=np.int64)
        slots = np.zeros(S * A * B, dtype=np.int64)
        for blk in range(nb * A * S):
            bb, ai, s = blk % nb, (blk // nb) % A, blk // (nb * A)
            j0, j1 = s * RS, min(s * RS + RS, Rd)
            assert j0 < j1
            for lane in range(64):
                lv = bb * 64 + lane
                if lv >= L:
                    continue
                for w in range(hk.COL_WAVES):
                    for j in range(j0 + w, j1, hk.COL_WAVES):
                        e = (ai * Rd + j) * B + lv * vec
                        seen[e:e + vec] += 1
                r = ai * B + lv * vec
                slots[s * A * B + r:s * A * B + r + vec] += 1
        assert (seen == 1).all() and (slots == 1).all(), (A, Rd, B, vec)
        cw = min(16, S)          # the combine launch's waves split each output's S partials
        assert sorted(s for w in range(cw) for s in range(w, S, cw)) == list(range(S))


def test_contiguous_pointwise_kernels_vectorise_across_rows(tj_env):
    """A pointwise kernel whose inputs all read the whole iteration space contiguously (or
    as one scalar) takes 16-byte vectors by element count, whatever the row length; a
    row-broadcast or transposed input keeps the row structure (and odd rows scalar)."""
    def vec_of(fn, shapes, dt=DType.f32):
        p = C.lower(tj.trace(fn, [TensorType(s, dt) for s in shapes]), "hip")
        src, launches = hb.generate(p)
        return [l.meta["vec"] for l in launches], src

    assert vec_of(lambda x, y: x * 2.0 + y, [(16384, 4095)] * 2)[0] == [4]
    assert vec_of(lambda x, y: x * 2.0 + y, [(16384, 4095)] * 2, DType.bf16)[0] == [8]
    v, src = vec_of(lambda x: tj.gelu(x), [(1000, 1001)])
    assert v == [4]
    hb.compile_source(src, "gfx950")
    assert vec_of(lambda x, y: x * 2.0 + y, [(16384, 4095), (4095,)])[0] == [1]
    assert vec_of(lambda x: x * 2.0, [(999, 1001)])[0] == [1]                 # 999999 elements
    assert vec_of(lambda x: x * 2.0, [(64, 4096)])[0] == [4]
