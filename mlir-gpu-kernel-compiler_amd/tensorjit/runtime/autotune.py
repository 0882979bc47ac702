"""GEMM tile autotuning for gfx950 (CDNA4).

Flow as in the reference autotuner (``tensorjit/runtime/autotune.py:83-118``):
an analytic cost model ranks the candidate tile configurations, only the
best ``top_k`` are compiled and timed on real buffers, and the winner is
persisted in ``AutotuneStore`` so later processes start warm.

The model is re-derived for MI355X instead of the reference's GPU branch
(``autotune.py:73-79``).  It prices one call as the slowest of

* MFMA time: 2*M*N*K at the dense matrix-core peak, scaled by how well the
  tile grid fills 256 CUs (tail rounds of workgroups) and by edge waste;
* LDS time: every wave re-reads its A and B fragments from LDS each K step
  (128 B/clk/CU);
* L2 time: each workgroup streams a (BM + BN) x K panel;
* HBM time: A, B and C once at 8 TB/s;

and rejects tiles that exceed 160 KiB of double-buffered LDS or 512 VGPRs
(accumulators + fragments + staging) per lane.
"""
from __future__ import annotations

import math
import os
import time
from dataclasses import dataclass
from typing import Callable, Sequence

from .cache import AutotuneStore

# MI355X (gfx950) figures used by the model.
CU_COUNT = 256
CLOCK_HZ = 2.4e9
LDS_BYTES_PER_CU = 160 * 1024
LDS_BYTES_PER_CLK = 128
MFMA_FLOP_PER_CLK_BF16 = 4096   # per CU: 2.5 PF / 256 CU / 2.4 GHz
MFMA_FLOP_PER_CLK_F32 = 256     # per CU: 157.3 TF / 256 CU / 2.4 GHz
HBM_BYTES_PER_S = 8.0e12
L2_BYTES_PER_S = 16.0e12


@dataclass(frozen=True)
class MatmulConfig:
    """A GEMM tiling: block tile TM x TN, K step TK, ``num_warps`` waves of 64 lanes.

    ``WM`` x ``WN`` is the wave grid inside the workgroup (``WM * WN == num_warps``)
    and ``MI`` the MFMA tile edge (32 -> 32x32 blocks, 16 -> 16x16 blocks).
    ``SPLIT_K`` > 1 splits K across the waves of a workgroup (skinny GEMMs).
    """

    TM: int
    TN: int
    TK: int = 0
    num_warps: int = 4
    WM: int = 2
    WN: int = 2
    MI: int = 32
    SPLIT_K: int = 1
    GROUP_M: int = 8        # tile rows per group of the XCD-aware tile order (0 = plain row-major order)
    PINGPONG: int = 0       # two wave groups alternate MFMA and memory phases: 1/2 = loads 2/3 K steps ahead, 3 = K-split tiles
    INTERLEAVE: int = 0     # 1: one wave per SIMD, memory instructions threaded between its MFMAs
    DIRECT: int = 0         # 1: one wave per SIMD, tiles loaded straight into LDS (buffer_load_dwordx4 ... lds)
    KSPLIT: int = 1         # > 1: K split over that many workgroups, partials summed by the last of them
    PERSIST: int = 0        # > 0 (DIRECT only): that many workgroups (one per CU) loop over the output tiles

    def as_dict(self) -> dict:
        return {"TM": self.TM, "TN": self.TN, "TK": self.TK, "num_warps": self.num_warps,
                "WM": self.WM, "WN": self.WN, "MI": self.MI, "SPLIT_K": self.SPLIT_K, "GROUP_M": self.GROUP_M,
                "PINGPONG": self.PINGPONG, "INTERLEAVE": self.INTERLEAVE, "DIRECT": self.DIRECT, "KSPLIT": self.KSPLIT,
                "PERSIST": self.PERSIST}

    @staticmethod
    def from_dict(d: dict) -> "MatmulConfig":
        return MatmulConfig(d["TM"], d["TN"], d.get("TK", 0), d.get("num_warps", 4), d.get("WM", 2),
                            d.get("WN", 2), d.get("MI", 32), d.get("SPLIT_K", 1), d.get("GROUP_M", 8),
                            d.get("PINGPONG", 0), d.get("INTERLEAVE", 0), d.get("DIRECT", 0), d.get("KSPLIT", 1),
                            d.get("PERSIST", 0))


# bf16 / fp16 candidates (MFMA 32x32x16 or 16x16x32)
HIP_CANDIDATES: list[MatmulConfig] = [
    # persistent direct-to-LDS kernels: one workgroup per CU looping over the output tiles
    MatmulConfig(256, 256, 64, 4, 2, 2, 16, 1, 8, 0, 0, 1, 1, CU_COUNT),
    MatmulConfig(256, 128, 64, 4, 2, 2, 16, 1, 8, 0, 0, 1, 1, CU_COUNT),
    MatmulConfig(256, 256, 64, 4, 2, 2, 16, 1, 8, 0, 0, 1),
    MatmulConfig(256, 128, 64, 4, 2, 2, 16, 1, 8, 0, 0, 1),
    MatmulConfig(256, 256, 64, 4, 2, 2, 32, 1, 8, 0, 0, 1),
    MatmulConfig(256, 128, 64, 4, 2, 2, 32, 1, 8, 0, 0, 1),
    # mid-size products (a few hundred 256x256 tiles or fewer): smaller direct tiles fill the CUs
    MatmulConfig(128, 128, 64, 4, 2, 2, 16, 1, 8, 0, 0, 1),
    MatmulConfig(128, 64, 64, 4, 2, 2, 16, 1, 8, 0, 0, 1),
    MatmulConfig(64, 128, 64, 4, 2, 2, 16, 1, 8, 0, 0, 1),
    MatmulConfig(256, 256, 64, 8, 2, 4, 32, 1, 8, 3),
    MatmulConfig(256, 256, 64, 8, 4, 2, 32, 1, 8, 3),
    MatmulConfig(256, 256, 32, 8, 2, 4, 32, 1, 8, 2),
    MatmulConfig(256, 256, 32, 8, 4, 2, 32, 1, 8, 2),
    MatmulConfig(256, 256, 32, 8, 2, 4, 32, 1, 8, 1),
    MatmulConfig(256, 256, 32, 8, 4, 2, 32, 1, 8, 1),
    MatmulConfig(256, 128, 32, 8, 4, 2, 32, 1, 8, 2),
    MatmulConfig(256, 128, 32, 8, 4, 2, 32, 1, 8, 1),
    MatmulConfig(256, 256, 64, 8, 2, 4, 32),
    MatmulConfig(256, 256, 32, 8, 2, 4, 32),
    MatmulConfig(256, 128, 64, 8, 4, 2, 32),
    MatmulConfig(256, 256, 64, 4, 2, 2, 32, 1, 8, 0, 1),
    MatmulConfig(256, 256, 32, 4, 2, 2, 32, 1, 8, 0, 1),
    MatmulConfig(256, 128, 64, 4, 2, 2, 32),
    MatmulConfig(128, 256, 64, 4, 2, 2, 32),
    MatmulConfig(128, 128, 64, 4, 2, 2, 32),
    MatmulConfig(128, 128, 32, 4, 2, 2, 32),
    MatmulConfig(128, 64, 64, 4, 2, 2, 32),
    MatmulConfig(64, 128, 64, 4, 2, 2, 32),
    MatmulConfig(64, 64, 64, 4, 2, 2, 16),
    MatmulConfig(64, 64, 32, 4, 2, 2, 16),
    MatmulConfig(32, 64, 64, 4, 2, 2, 16),
    # skinny (M <= 16 / 32): one MI x MI tile per workgroup, K split over its waves
    MatmulConfig(16, 32, 64, 4, 1, 1, 16, 4, 0),
    MatmulConfig(16, 32, 128, 4, 1, 1, 16, 4, 0),
    MatmulConfig(16, 32, 128, 2, 1, 1, 16, 2, 0),
    MatmulConfig(32, 32, 64, 4, 1, 1, 32, 4, 0),
    MatmulConfig(16, 32, 256, 8, 1, 1, 16, 8, 0),
    MatmulConfig(16, 64, 256, 8, 1, 1, 16, 8, 0),
    MatmulConfig(16, 32, 128, 16, 1, 1, 16, 16, 0),
    MatmulConfig(16, 64, 128, 16, 1, 1, 16, 16, 0),
    MatmulConfig(16, 16, 256, 8, 1, 1, 16, 8, 0),
    MatmulConfig(32, 32, 128, 8, 1, 1, 32, 8, 0),
    MatmulConfig(32, 64, 64, 16, 1, 1, 32, 16, 0),
]

# fp32 candidates (MFMA 32x32x2 / 16x16x4 f32)
HIP_F32_CANDIDATES: list[MatmulConfig] = [
    # direct-to-LDS (32-deep K tiles: the bf16 kernel's 128-byte rows), 16x16x4 MFMAs
    MatmulConfig(128, 128, 32, 4, 2, 2, 16, 1, 8, 0, 0, 1),
    MatmulConfig(128, 256, 32, 4, 2, 2, 16, 1, 8, 0, 0, 1),
    MatmulConfig(256, 128, 32, 4, 2, 2, 16, 1, 8, 0, 0, 1),
    MatmulConfig(128, 128, 32, 4, 2, 2, 16, 1, 8, 0, 0, 1, 1, CU_COUNT),
    MatmulConfig(64, 64, 32, 4, 2, 2, 16, 1, 8, 0, 0, 1),
    MatmulConfig(128, 128, 16, 4, 2, 2, 32),
    MatmulConfig(128, 128, 32, 4, 2, 2, 32),
    MatmulConfig(128, 64, 32, 4, 2, 2, 32),
    MatmulConfig(64, 128, 32, 4, 2, 2, 32),
    MatmulConfig(64, 64, 32, 4, 2, 2, 16),
    MatmulConfig(64, 64, 16, 4, 2, 2, 16),
    MatmulConfig(32, 32, 32, 4, 2, 2, 16),
    MatmulConfig(32, 64, 32, 4, 2, 2, 16),
    MatmulConfig(64, 32, 32, 4, 2, 2, 16),
    MatmulConfig(32, 32, 64, 4, 2, 2, 16),
    # K split over workgroups (few output tiles, long K: config 1's 512x768x3072)
    MatmulConfig(64, 64, 32, 4, 2, 2, 16, 1, 8, 0, 0, 0, 8),
    MatmulConfig(64, 64, 32, 4, 2, 2, 16, 1, 8, 0, 0, 0, 4),
    MatmulConfig(32, 32, 64, 4, 2, 2, 16, 1, 8, 0, 0, 0, 4),
    MatmulConfig(32, 64, 64, 4, 2, 2, 16, 1, 8, 0, 0, 0, 4),
]


def _skinny_cost(cfg: MatmulConfig, M: int, N: int, K: int, batch: int, elem: int) -> float:
    """Streaming kernel: the B panel once from HBM, A re-read (from L2) by every
    workgroup.  Measured on MI355X for 16 x 8192 x 8192 (TN 32, one workgroup per CU):
    4 waves per workgroup stream B at 5.5 TB/s whatever the unroll depth (2-16 MFMA
    steps ahead), 2 waves at 5.3, 8 waves at 4.9, 16 at 3.9; fewer workgroups than
    CUs leave CUs idle (TN 64: 3.6 TB/s)."""
    if M > cfg.TM or elem != 2:
        return math.inf
    t_hbm = (M * K + N * K + M * N) * batch * elem / HBM_BYTES_PER_S
    wgs = -(-N // cfg.TN) * batch
    fill = min(1.0, wgs / CU_COUNT)
    per_wave = {4: 1.0, 2: 1.04, 8: 1.13, 16: 1.4}.get(cfg.SPLIT_K, 1.5)
    a_reads = 1.0 + cfg.TM / cfg.TN * 0.5                # A panel re-read per TN columns (from L2)
    return t_hbm / max(fill, 1e-3) * per_wave * a_reads * 1e6


def _sched_factor(cfg: MatmulConfig) -> float:
    """Relative MFMA-phase cost of a loop schedule, from bf16 8192^3 runs on MI355X
    (direct-to-LDS loads 3-7% ahead of ping-pong with K-split tiles, and another ~10%
    with 16x16x32 MFMAs, which hold a higher clock on random data than 32x32x16;
    plain double-buffered loop ~9% behind ping-pong; the persistent direct kernel
    1-2% ahead of the direct one at 8192^3, 1-8% on config 5's projections)."""
    if cfg.PERSIST:
        return 0.85
    if cfg.DIRECT:
        return 0.86 if cfg.MI == 16 else 0.95
    if cfg.INTERLEAVE:
        return 1.15
    return {3: 1.0, 2: 1.04, 1: 1.05}.get(cfg.PINGPONG, 1.09)


def _hip_cost(cfg: MatmulConfig, M: int, N: int, K: int, batch: int, elem: int) -> float:
    if cfg.SPLIT_K > 1:
        return _skinny_cost(cfg, M, N, K, batch, elem)
    tm, tn, tk = cfg.TM, cfg.TN, cfg.TK or 32
    waves = cfg.num_warps
    if cfg.SPLIT_K == 1 and (tm % (cfg.WM * cfg.MI) or tn % (cfg.WN * cfg.MI)):
        return math.inf
    pad = 16 // elem
    lds = 2 * (tm + tn) * (tk + pad) * elem
    if lds > LDS_BYTES_PER_CU:
        return math.inf
    acc = tm * tn / (64 * waves) * (cfg.SPLIT_K if cfg.SPLIT_K > 1 else 1)
    frags = 2 * (tm / cfg.WM + tn / cfg.WN) / cfg.MI * (4 if elem == 2 else 1)  # double-buffered
    if cfg.DIRECT and cfg.MI == 16:
        frags -= tm / cfg.WM / cfg.MI * 4                                   # A re-read in place
    staging = 0 if cfg.DIRECT else (tm + tn) * tk * elem / (64 * waves * 4)  # staged K step per lane, 4 B per VGPR
    regs = acc + frags + staging + 32
    if regs > 512:
        return math.inf
    # workgroups per CU: LDS, and registers (a SIMD holds 512 per lane; waves spread over 4 SIMDs)
    occ = max(1, min(LDS_BYTES_PER_CU // lds, int(512 // regs) * 4 // waves, 32 // waves))
    S = cfg.KSPLIT
    tiles = -(-M // tm) * -(-N // tn) * batch * S                  # a K split multiplies the workgroups
    kt = K / S                                                     # ... each over 1/S of K
    slots = CU_COUNT * occ
    rounds = -(-tiles // slots)
    fill = tiles / (rounds * slots)
    busy_cus = min(1.0, tiles / CU_COUNT)
    edge = (M / (-(-M // tm) * tm)) * (N / (-(-N // tn) * tn))
    flops = 2.0 * M * N * K * batch
    peak = (MFMA_FLOP_PER_CLK_BF16 if elem == 2 else MFMA_FLOP_PER_CLK_F32) * CU_COUNT * CLOCK_HZ
    t_mfma = flops / (peak * max(fill, 1e-3) * max(busy_cus, 1e-3) * edge) * _sched_factor(cfg)
    # LDS: per K step each wave reads (tm/WM + tn/WN) x tk elements; per CU per tile
    lds_bytes_tile = waves * (tm / cfg.WM + tn / cfg.WN) * kt * elem
    lds_bytes_tile += (tm + tn) * kt * elem                        # the global->LDS writes
    t_lds = tiles * lds_bytes_tile / (LDS_BYTES_PER_CLK * CLOCK_HZ * min(CU_COUNT, tiles))
    t_l2 = tiles * (tm + tn) * kt * elem / L2_BYTES_PER_S
    t_hbm = (M * K + N * K + M * N) * batch * elem / HBM_BYTES_PER_S
    # a workgroup writes its output tile after its K loop; with one workgroup per CU
    # nothing overlaps that store, which matters when the output dominates (small K);
    # a persistent workgroup starts its next tile while the stores drain (about half
    # of them overlap: the second K step of the next tile waits for them)
    t_out = M * N * batch * (4 * S if S > 1 else elem) / HBM_BYTES_PER_S / occ
    if cfg.PERSIST and tiles > CU_COUNT:
        t_out *= 0.5
    # split K: the S fp32 partials are read back and the output written after the last
    # split finishes (in the tile's last workgroup, ~2.3 us of tail at config 1, or a second launch)
    t_sum = ((S * 4 + elem) * M * N * batch / HBM_BYTES_PER_S + 4e-6) if S > 1 else 0.0
    t = max(t_mfma, t_lds, t_l2, t_hbm) + t_out + t_sum
    return t * 1e6


def cost_model(cfg: MatmulConfig, M: int, N: int, K: int, backend: str, batch: int = 1) -> float:
    """Lower is better.  ``backend``: "hip" (bf16/fp16) or "hip_f32"; CPU kinds
    "c" / "c_dot" keep the reference's register-pressure heuristic."""
    if backend in ("hip", "hip_f32"):
        return _hip_cost(cfg, M, N, K, batch, 2 if backend == "hip" else 4)
    tm, tn = cfg.TM, cfg.TN
    tk = cfg.TK or K
    cost = (4.0 * (tm * tk + tk * tn)) / (2.0 * tm * tn * tk)
    cost /= (M / (-(-M // tm) * tm)) * (N / (-(-N // tn) * tn))
    if backend == "c_dot":
        regs = tm * tn + tm
        if regs > 14:
            cost *= (regs / 14.0) ** 2
    elif backend == "c":
        regs = tm * tn / 8.0
        if regs > 12:
            cost *= 1.0 + (regs - 12) / 4.0
    if M / tm < 2 * (os.cpu_count() or 1):
        cost *= 1.3
    return cost


def _wall_timer(run: Callable[[], None], warmup: int, iters: int) -> float:
    for _ in range(warmup):
        run()
    t0 = time.perf_counter()
    for _ in range(iters):
        run()
    return (time.perf_counter() - t0) / iters * 1e3


def autotune(
    key: str,
    candidates: Sequence[MatmulConfig],
    build: Callable[[MatmulConfig], Callable[[], None]],
    shape: tuple,
    backend: str,
    top_k: int = 4,
    store: AutotuneStore | None = None,
    warmup: int = 2,
    iters: int = 5,
    timer: Callable[[Callable[[], None], int, int], float] | None = None,
    rounds: int = 1,
) -> MatmulConfig:
    """Fastest candidate by measurement; ``build(cfg)`` returns a runner for ``timer``.

    ``timer(run, warmup, iters) -> ms`` measures one runner (device-event timing for
    GPU kernels).  All runners are built first, then timed in ``rounds`` interleaved
    passes keeping each candidate's best time, so clock ramp-up or a noisy
    neighbour cannot favour whichever candidate happened to run last.  Candidates
    whose build or run raises are skipped.
    """
    store = store or AutotuneStore()
    M, N, K = shape[:3]
    batch = shape[3] if len(shape) > 3 else 1
    rank = lambda c: cost_model(c, M, N, K, backend, batch)  # noqa: E731
    if os.environ.get("TENSORJIT_NO_AUTOTUNE") == "1":
        return min(candidates, key=rank)
    cached = store.get(key)
    if cached is not None:
        return MatmulConfig.from_dict(cached["config"])
    ranked = [c for c in sorted(candidates, key=rank) if math.isfinite(rank(c))][:top_k]
    if not ranked:
        ranked = [min(candidates, key=rank)]
    timer = timer or _wall_timer
    runners = []
    for cfg in ranked:
        try:
            runners.append((cfg, build(cfg)))
        except Exception:  # invalid for this shape: skip it
            continue
    best_of = {}
    for _ in range(max(1, rounds)):
        for cfg, run in runners:
            try:
                ms = timer(run, warmup, iters)
            except Exception:
                continue
            best_of[cfg] = min(ms, best_of.get(cfg, math.inf))
    if not best_of:
        best, best_ms = ranked[0], math.inf
    else:
        best = min(best_of, key=best_of.get)
        best_ms = best_of[best]
    store.put(key, best.as_dict(), best_ms)
    return best


__all__ = ["MatmulConfig", "HIP_CANDIDATES", "HIP_F32_CANDIDATES", "cost_model", "autotune"]
