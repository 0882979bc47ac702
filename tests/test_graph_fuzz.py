"""Seeded random programs (tests/graph_fuzz.py) through the hip backend.

CPU: every program lowers, gets the backend rewrites and generates HIP that hipRTC
compiles for gfx950.  GPU: the programs run against the CPU oracle -- float32 within
1e-5 of the output's magnitude; bfloat16 within 5e-2, since every kernel boundary
rounds the intermediates to bfloat16 where the oracle keeps float32."""

import pytest
import torch

import graph_fuzz
import tensorjit as tj
from tensorjit.backends import hip_backend as hb
from tensorjit.compiler import lower
from tensorjit.ir import DType, TensorType

CPU_SEEDS = range(16)
GPU_SEEDS = range(40)


@pytest.mark.parametrize("seed", CPU_SEEDS)
def test_random_program_generates_and_compiles(seed, tj_env):
    fn, shapes = graph_fuzz.program(seed)
    for dt in (DType.f32, DType.bf16):
        p = lower(tj.trace(fn, [TensorType(s, dt) for s in shapes]), "hip")
        p = hb.fold_elementwise_into_gemm(hb.fuse_attention(p))
        src, launches = hb.generate(p)
        assert len(launches) >= len(p.kernels)
        hb.compile_source(src, "gfx950")


def test_the_programs_cover_every_kernel_family(tj_env):
    kinds = set()
    for seed in range(64):
        fn, shapes = graph_fuzz.program(seed)
        p = lower(tj.trace(fn, [TensorType(s, DType.f32) for s in shapes]), "hip")
        kinds |= {k.kind for k in p.kernels}
    assert kinds >= {"elementwise", "copy", "row", "reduce", "matmul"}


@pytest.mark.gpu
@pytest.mark.parametrize("seed", GPU_SEEDS)
def test_random_program_matches_the_oracle(seed, monkeypatch):
    import oracle

    monkeypatch.setenv("TENSORJIT_NO_AUTOTUNE", "1")
    fn, shapes = graph_fuzz.program(seed)
    g = torch.Generator().manual_seed(seed)
    ins = [torch.randn(s, generator=g) for s in shapes]
    for dt, tol in ((torch.float32, 1e-5), (torch.bfloat16, 5e-2)):
        print(f"random program {seed} {dt} {shapes}", flush=True)
        outs = tj.jit(fn)(*[t.to(dt).cuda() for t in ins])
        outs = outs if isinstance(outs, (tuple, list)) else [outs]
        refs = oracle.run(fn, *[t.to(dt).float() for t in ins])
        assert len(outs) == len(refs)
        for o, r in zip(outs, refs):
            o = o.float().cpu()
            assert o.shape == r.shape
            assert torch.isfinite(o).all() == torch.isfinite(r).all()
            scale = float(r.abs().max()) or 1.0
            err = float(((o - r).abs() / (r.abs() + scale)).max())
            assert err <= tol, (seed, dt, err)
