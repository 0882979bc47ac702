#!/usr/bin/env python
"""Benchmark of the tensorjit hip backend on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Prints ONE JSON line.  The headline (``value``) is BASELINE.json's fused
elementwise/broadcast chain (config 2): ``y = gelu(x*a+b) * sigmoid(c) + x`` over
fp32 x, c [16384, 4096] and a, b [4096], compiled by ``tj.jit`` into one kernel;
a step is one call of the compiled function on inputs already resident in HBM,
and ``value`` is algorithmic HBM bytes per step / wall time per step (GB/s).

``roofline`` is that kernel's achieved bandwidth (algorithmic bytes / average
kernel duration from hipEvents on the stream the kernel runs on) against the
8 TB/s HBM3E peak; ``traffic`` is the measured HBM bytes per launch from the
committed rocprofv3 counter summary when one exists for this workload.
``cpu_baseline`` is the CPU oracle (the C/OpenMP restatement of the reference
``c`` backend) on the same workload.  ``secondary`` carries the other
BASELINE.json configurations (row kernels, GEMMs, MLP block per-call time).
"""
from __future__ import annotations

import argparse
import hashlib
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "mlir-gpu-kernel-compiler_amd"))
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP32_PEAK_TFLOPS = 157.3
METRIC = "HBM GB/s (eltwise/row) + bf16 GEMM TFLOPS, % of peak; MLP block us/call"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _fn_c2(x, a, b, c):
    import tensorjit as tj

    return tj.gelu(x * a + b) * tj.sigmoid(c) + x


def _fn_ln(x, g):
    import tensorjit as tj

    return tj.layer_norm(x, g)


def _fn_rms(x, g):
    import tensorjit as tj

    return tj.rms_norm(x, g)


def _fn_sum_all(x):
    import tensorjit as tj

    return tj.sum(x)


def _fn_sum_axis0(x):
    import tensorjit as tj

    return tj.sum(x, axis=0)


def _fn_softmax(s):
    import tensorjit as tj

    return tj.softmax(s)


def _fn_gemm(x, w, b):
    import tensorjit as tj

    return tj.gelu(tj.linear(x, w, b))


def _fn_attn(q, k, v):
    """Config 5's attention core: softmax(q k^T / sqrt(d)) v over [B, H, S, 128] heads."""
    import tensorjit as tj

    return tj.matmul(tj.softmax(tj.matmul(q, tj.transpose(k, -1, -2)) * (1.0 / q.shape[-1] ** 0.5)), v)


def _fn_mlp(x, g, w1, b1, w2, b2):
    import tensorjit as tj

    return x + tj.linear(tj.gelu(tj.linear(tj.layer_norm(x, g), w1, b1)), w2, b2)


def _fn_block(x, g1, wq, wk, wv, wo, g2, w1, w2):
    """Config 5: one pre-norm transformer layer (RMSNorm, q/k/v projections, attention
    with materialised scores, out-projection + residual, RMSNorm, gelu MLP + residual)."""
    import tensorjit as tj

    B, S, D = x.shape
    H, Dh = 32, D // 32
    h = tj.rms_norm(x, g1)
    q = tj.linear(h, wq).reshape(B, S, H, Dh).transpose(1, 2)
    k = tj.linear(h, wk).reshape(B, S, H, Dh).transpose(1, 2)
    v = tj.linear(h, wv).reshape(B, S, H, Dh).transpose(1, 2)
    p = tj.softmax(tj.matmul(q, k.transpose(-1, -2)) * (1.0 / Dh ** 0.5))
    o = tj.matmul(p, v).transpose(1, 2).reshape(B, S, D)
    x = x + tj.linear(o, wo)
    return x + tj.linear(tj.gelu(tj.linear(tj.rms_norm(x, g2), w1)), w2)


def _fn_chain(x, w):
    """The reference's per-call overhead harness (benchmarks/bench_overhead.py:21-25):
    8 x softmax(x @ w + 0.5), 16 kernels on tiny tensors."""
    import tensorjit as tj

    y = x
    for _ in range(8):
        y = tj.softmax(tj.matmul(y, w) + 0.5)
    return y


def overhead_chain(torch, dev) -> dict:
    """Per-call wall time of the overhead chain on x[16,32], w[32,32], timed like the
    reference (benchmarks/bench_overhead.py:28-38: 50 warmup calls, 500 timed, synchronised
    at both ends; best of 3): hip direct launches, hipGraph replay, the default (replay from
    12 launches), torch eager; plus the native runtime's host time per call."""
    import tensorjit as tj

    gen = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn(16, 32, device=dev, generator=gen)
    w = torch.randn(32, 32, device=dev, generator=gen)

    def per_call_us(f):
        best = float("inf")
        for _ in range(3):
            for _ in range(50):
                f(x, w)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(500):
                f(x, w)
            torch.cuda.synchronize()
            best = min(best, (time.perf_counter() - t0) / 500 * 1e6)
        return round(best, 2)

    res = {}
    for name, mode in (("direct", "0"), ("graph", "1"), ("default", None)):
        if mode is None:
            os.environ.pop("TENSORJIT_HIP_GRAPH", None)
        else:
            os.environ["TENSORJIT_HIP_GRAPH"] = mode
        f = tj.jit(_fn_chain)
        f(x, w)
        cp = f.compiled(x, w)
        res[f"{name}_us"] = per_call_us(f)
        st = cp.native_stats()
        res[f"{name}_host_us"] = round(st["host_us"] / max(st["calls"], 1), 2)
        res["launches"] = len(cp.launches)
        if mode is None:
            res["default_uses_graph"] = cp.use_graph
    os.environ.pop("TENSORJIT_HIP_GRAPH", None)

    def eager(a, b):
        for _ in range(8):
            a = torch.softmax(a @ b + 0.5, -1)
        return a

    res["torch_eager_us"] = per_call_us(eager)
    return res


def _ref_workloads():
    """The reference's GPU benchmark workloads (reference benchmarks/bench.py:20-52): name ->
    (tensorjit function, eager PyTorch function, shapes at sequence length T and hidden D)."""
    import torch
    import torch.nn.functional as F

    import tensorjit as tj

    return {
        "bias_gelu": (lambda x, b: tj.gelu(x + b), lambda x, b: F.gelu(x + b),
                      lambda T, D: [(T, 4 * D), (4 * D,)]),
        # the reference times softmax over [8, min(T, 2048), min(T, 2048)] (its bench.py:97-98)
        "softmax": (lambda t: tj.softmax(t), lambda t: torch.softmax(t, -1),
                    lambda T, D: [(8, min(T, 2048), min(T, 2048))]),
        "layernorm": (lambda x, g, b: tj.layer_norm(x, g, b), lambda x, g, b: F.layer_norm(x, (x.shape[-1],), g, b),
                      lambda T, D: [(T, D), (D,), (D,)]),
        "rmsnorm": (lambda x, g: tj.rms_norm(x, g),
                    lambda x, g: x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6) * g,
                    lambda T, D: [(T, D), (D,)]),
        "linear_gelu": (lambda x, w, b: tj.gelu(tj.linear(x, w, b)), lambda x, w, b: F.gelu(F.linear(x, w, b)),
                        lambda T, D: [(T, D), (4 * D, D), (4 * D,)]),
        "mlp_block": (lambda x, g, w1, b1, w2, b2: x + tj.linear(tj.gelu(tj.linear(tj.layer_norm(x, g), w1, b1)), w2, b2),
                      lambda x, g, w1, b1, w2, b2: x + F.linear(F.gelu(F.linear(F.layer_norm(x, (x.shape[-1],), g),
                                                                               w1, b1)), w2, b2),
                      lambda T, D: [(T, D), (D,), (4 * D, D), (4 * D,), (D, 4 * D), (D,)]),
    }


def reference_gpu_table(torch, dev, seqs=(256, 1024, 4096), hidden=1024) -> dict:
    """The reference's GPU comparison (reference benchmarks/bench.py:55-70, README.md:188-193)
    for the hip backend: each workload at hidden 1024 and seq 256 / 1024 / 4096, in fp32 and
    bf16, timed the reference's way (hipEvents on the current stream around 50 calls after 10
    warmup calls) for eager PyTorch-ROCm, hip with direct launches and hip with hipGraph
    replay of the same compiled program.  Inputs are plain ``torch.randn`` as in the
    reference.  GEMM tiles come from the packaged table or the CDNA4 cost model (no
    on-device tuning inside the benchmark).  torch.compile (inductor) is not timed: it
    would generate Triton kernels at run time.  ``max_abs_err`` is the reference's check,
    hip against eager."""

    def timeit(fn, iters=50, warmup=10):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(iters):
            fn()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / iters

    import tensorjit as tj

    saved = os.environ.get("TENSORJIT_NO_AUTOTUNE")
    os.environ["TENSORJIT_NO_AUTOTUNE"] = "1"
    rows = []
    for dtname, dt in (("fp32", torch.float32), ("bf16", torch.bfloat16)):
        for name, (tj_fn, torch_fn, shapes) in _ref_workloads().items():
            for T in seqs:
                g = torch.Generator(device=dev).manual_seed(T)
                args = [torch.randn(*sh, device=dev, generator=g).to(dt) for sh in shapes(T, hidden)]
                jf = tj.jit(tj_fn)
                out = jf(*args)
                cp = jf.compiled(*args)
                err = float((out.float() - torch_fn(*args).float()).abs().max())
                t_eager = timeit(lambda: torch_fn(*args))
                cp.use_graph = False
                t_direct = timeit(lambda: jf(*args))
                cp.use_graph = True
                t_graph = timeit(lambda: jf(*args))
                cp.use_graph = len(cp.launches) >= 12
                rows.append({"workload": name, "seq": T, "dtype": dtname, "eager_ms": round(t_eager, 4),
                             "hip_ms": round(t_direct, 4), "hip_graph_ms": round(t_graph, 4),
                             "speedup_vs_eager": round(t_eager / min(t_direct, t_graph), 2),
                             "kernels": cp.num_kernels, "launches": len(cp.launches), "max_abs_err": float(f"{err:.3g}")})
                del args, out, jf, cp
    if saved is None:
        os.environ.pop("TENSORJIT_NO_AUTOTUNE", None)
    else:
        os.environ["TENSORJIT_NO_AUTOTUNE"] = saved
    readme = {f"{r['workload']} T={r['seq']} {r['dtype']}": {k: r[k] for k in ("eager_ms", "hip_ms", "hip_graph_ms")}
              for r in rows if (r["workload"], r["seq"]) in (("mlp_block", 4096), ("softmax", 4096))}
    return {"hidden": hidden, "timing": "hipEvents, warmup 10, iters 50 (reference benchmarks/bench.py:55-70)",
            "inductor": None, "rows": rows, "readme_rows": readme}


def block_inputs(torch, dev, B=4, S=2048, D=4096, F=11008, dt=None):
    dt = dt or torch.bfloat16
    g = torch.Generator(device=dev).manual_seed(0)
    w = lambda *s: (0.02 * torch.randn(*s, device=dev, generator=g)).to(dt)  # noqa: E731
    x = torch.randn(B, S, D, device=dev, generator=g).to(dt)
    ones = torch.ones(D, device=dev, dtype=dt)
    return [x, ones, w(D, D), w(D, D), w(D, D), w(D, D), ones.clone(), w(F, D), w(D, F)]


def c2_inputs(torch, dt, dev):
    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn(16384, 4096, device=dev, generator=g)
    a = torch.randn(4096, device=dev, generator=g)
    b = torch.randn(4096, device=dev, generator=g)
    c = torch.rand(16384, 4096, device=dev, generator=g) * 8 - 4
    return [t.to(dt) for t in (x, a, b, c)]


def ramp(torch, fn, args, seconds):
    """Untimed calls for at least ``seconds`` of wall time: a GPU left idle while the
    process starts can take tens of milliseconds to reach its clocks, which a fixed
    count of warmup steps of a ~0.1 ms kernel does not cover."""
    t0 = time.perf_counter()
    while True:
        for _ in range(8):
            fn(*args)
        torch.cuda.synchronize()
        if time.perf_counter() - t0 >= seconds:
            return


def timed_steps(torch, fn, args, steps, warmup, ramp_s=0.1):
    ramp(torch, fn, args, ramp_s)
    for _ in range(warmup):
        fn(*args)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn(*args)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps * 1e3


def kernel_ms(f, args, k=None, iters=20):
    """Device time of launch ``k``, or of all the program's launches (``k=None``: a
    split-K decode GEMM is one kernel with two launches)."""
    cp = f.compiled(*args)
    ks = range(len(cp.launches)) if k is None else [k]
    return sum(cp.kernel_time_ms(i, *args, warmup=3, iters=iters) for i in ks)


def kernel_ms_settled(cp, args, k=None, rounds=3, iters=10, settle_s=0.5):
    """Best of ``rounds`` averages of ``iters`` launches, once the clocks have settled:
    averages of ``iters`` back-to-back launches are taken until two in a row agree within
    1% (or ``settle_s`` of device time has passed).  An MFMA-bound kernel needs dozens of
    launches after a cold start: config 4's GEMM reads 868, 757 and 726 us in its first
    three averages of 10 and 697-703 us from then on.  ``k=None`` sums all the program's
    launches."""
    ks = range(len(cp.launches)) if k is None else [k]
    total = 0.0
    for i in ks:
        prev, spent = None, 0.0
        while spent < settle_s * 1e3:
            ms = cp.kernel_time_ms(i, *args, warmup=0, iters=iters)
            spent += ms * iters
            if prev is not None and abs(ms - prev) <= 0.01 * prev:
                break
            prev = ms
        total += min(cp.kernel_time_ms(i, *args, warmup=1, iters=iters) for _ in range(rounds))
    return total


def source_sha16(cp) -> str:
    """Digest of a compiled program's HIP source: names the exact kernels a profile measured."""
    return hashlib.sha256(cp.source.encode()).hexdigest()[:16]


def load_traffic(workload: str, sha16: str):
    """HBM bytes per launch from the committed rocprofv3 PMC summary, when it was taken
    of this very kernel source (the summary records each program's source digest);
    otherwise (None, why)."""
    p = ROOT / "profiles" / "hbm_traffic.json"
    try:
        data = json.loads(p.read_text())
    except (OSError, ValueError):
        return None, "no PMC summary"
    entry = data.get(workload)
    if entry is None:
        return None, "workload not in the PMC summary"
    if entry.get("source_sha16") != sha16:
        return None, f"PMC summary is of source {entry.get('source_sha16')}, this kernel is {sha16}"
    return entry.get("traffic_bytes"), None


def host_cpus() -> dict:
    """CPU counts of the host the baseline runs on: logical CPUs, the CPUs this process
    may run on (its affinity mask: the box's share), physical cores (distinct
    (package, core) pairs in /proc/cpuinfo), and the OpenMP threads the oracle uses
    (``OMP_NUM_THREADS`` when set -- the GPU boxes set it to their CPU share -- else
    libgomp's default, one per CPU in the affinity mask)."""
    logical = os.cpu_count() or 1
    try:
        allowed = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        allowed = logical
    cores, pkg = set(), "0"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            key, _, val = line.partition(":")
            key, val = key.strip(), val.strip()
            if key == "physical id":
                pkg = val
            elif key == "core id":
                cores.add((pkg, val))
    except OSError:
        pass
    threads = int(os.environ.get("OMP_NUM_THREADS") or allowed)
    return {"omp_threads": threads, "logical_cpus": logical, "affinity_cpus": allowed,
            "physical_cores": len(cores) or None}


def cpu_baseline(torch, args_gpu, nbytes, seconds):
    import oracle

    host = [t.float().cpu() for t in args_gpu]
    prog = oracle.compile_program(oracle.lower_f32(_fn_c2, *[t.shape for t in host]))
    prog(*host)                               # warm (page-in, OpenMP pool)
    n, t0 = 0, time.perf_counter()
    while True:
        prog(*host)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds or n >= 5000:
            break
    per = el / n
    host = host_cpus()
    cores = host["omp_threads"]
    return {"value": round(nbytes / per / 1e9, 2), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"full config-2 fp32 workload [16384,4096] x {n} calls ({el:.1f} s), "
                      f"oracle C/OpenMP restatement of the reference c backend, {cores} OpenMP threads "
                      f"(host: {host['physical_cores']} physical cores, {host['logical_cpus']} logical CPUs, "
                      f"{host['affinity_cpus']} in this process's CPU share)",
            "host": host, "ms_per_call": round(per * 1e3, 3)}


def cpu_secondary(torch, seconds_cap: float = 20.0) -> dict:
    """The CPU oracle (C/OpenMP restatement of the reference ``c`` backend, fp32 only)
    on the secondary configurations: config 1 per call (warmup 3, iters 20), the
    config-3 rows on fp32 copies (1 warmup, 3 iters),
    and config 4 on a 128-row sample of x scaled to the full 8192 rows."""
    import oracle

    cores = host_cpus()["omp_threads"]
    gen = torch.Generator().manual_seed(0)
    out = {"kind": "port", "cores": cores, "dtype": "f32 (bf16 configs on fp32 copies)"}
    t_start = time.perf_counter()

    def timed(fn, args, warmup, iters):
        prog = oracle.compile_program(oracle.lower_f32(fn, *[t.shape for t in args]))
        for _ in range(warmup):
            prog(*args)
        t0 = time.perf_counter()
        for _ in range(iters):
            prog(*args)
        return (time.perf_counter() - t0) / iters

    shapes = [(512, 768), (768,), (3072, 768), (3072,), (768, 3072), (768,)]
    margs = [torch.randn(sh, generator=gen) * (1 if i < 2 else 0.02) for i, sh in enumerate(shapes)]
    out["c1_mlp_us_per_call"] = round(timed(_fn_mlp, margs, 3, 20) * 1e6, 1)
    x = torch.randn(65536, 4096, generator=gen).bfloat16().float()
    gn = (1 + 0.1 * torch.randn(4096, generator=gen)).bfloat16().float()
    nb = 2 * 65536 * 4096 * 2 + 4096 * 2
    for name, fn in (("c3_layernorm", _fn_ln), ("c3_rmsnorm", _fn_rms)):
        if time.perf_counter() - t_start < seconds_cap:
            t = timed(fn, [x, gn], 1, 3)
            out[name] = {"ms_per_call": round(t * 1e3, 2), "GB/s_bf16_equiv": round(nb / t / 1e9, 2)}
    del x
    sm = torch.randn(65536, 2048, generator=gen) * 3
    if time.perf_counter() - t_start < seconds_cap:
        t = timed(_fn_softmax, [sm], 1, 3)
        out["c3_softmax"] = {"ms_per_call": round(t * 1e3, 2), "GB/s": round(2 * 65536 * 2048 * 4 / t / 1e9, 2)}
    del sm
    if time.perf_counter() - t_start < seconds_cap:
        rows = 128
        xg = torch.randn(rows, 8192, generator=gen).bfloat16().float()
        wg = (0.02 * torch.randn(8192, 8192, generator=gen)).bfloat16().float()
        bg = (0.02 * torch.randn(8192, generator=gen)).bfloat16().float()
        t = timed(_fn_gemm, [xg, wg, bg], 1, 1) * (8192 / rows)
        out["c4_gemm_8192"] = {"ms_per_call_est": round(t * 1e3, 1), "TFLOP/s": round(2 * 8192 ** 3 / t / 1e12, 3),
                               "sample": f"{rows} of 8192 rows of x, time scaled by {8192 // rows}"}
    log(f"cpu secondary: {out}")
    return out


def secondary(torch, dev, quick):
    import tensorjit as tj

    out = {}

    def row(name, fn, args, nbytes):
        f = tj.jit(fn)
        f(*args)
        wall = timed_steps(torch, f, args, 20, 3)       # includes the clock ramp
        ms = kernel_ms_settled(f.compiled(*args), args, iters=20)
        out[name] = {"GB/s": round(nbytes / ms / 1e6, 1), "frac_hbm": round(nbytes / ms / 1e6 / HBM_PEAK_GBS, 4),
                     "kernel_us": round(ms * 1e3, 2), "us_per_call": round(wall * 1e3, 2), "bytes": nbytes}
        log(f"{name}: {out[name]}")

    gen = torch.Generator(device=dev).manual_seed(0)
    bf = torch.bfloat16
    # config 2 in bf16
    args = c2_inputs(torch, bf, dev)
    row("c2_eltwise_bf16", _fn_c2, args, 3 * 16384 * 4096 * 2 + 2 * 4096 * 2)
    del args
    # config 3: rows
    x = torch.randn(65536, 4096, device=dev, generator=gen).to(bf)
    gn = (1 + 0.1 * torch.randn(4096, device=dev, generator=gen)).to(bf)
    nb = 2 * 65536 * 4096 * 2 + 4096 * 2
    row("c3_layernorm_bf16", _fn_ln, [x, gn], nb)
    row("c3_rmsnorm_bf16", _fn_rms, [x, gn], nb)
    del x
    s = torch.randn(65536, 2048, device=dev, generator=gen) * 3
    row("c3_softmax_f32", _fn_softmax, [s], 2 * 65536 * 2048 * 4)
    del s
    # reductions and rows past the reference plan's shapes: one long row split over
    # workgroups, a reduction over the leading axis read in place, a row-fused LayerNorm
    # over rows of 16384
    xr = torch.randn(1 << 26, device=dev, generator=gen)
    row("reduce_sum_f32_1x67108864_split", _fn_sum_all, [xr], (1 << 26) * 4 + 4)
    del xr
    xc = torch.randn(16384, 4096, device=dev, generator=gen)
    row("colreduce_sum_axis0_f32_16384x4096", _fn_sum_axis0, [xc], 16384 * 4096 * 4 + 4096 * 4)
    del xc
    xw = torch.randn(8192, 16384, device=dev, generator=gen)
    gw = 1 + 0.1 * torch.randn(16384, device=dev, generator=gen)
    row("layernorm_f32_8192x16384_one_row_kernel", _fn_ln, [xw, gw], 2 * 8192 * 16384 * 4 + 16384 * 4)
    del xw, gw
    if quick:
        return out
    # config 4: GEMMs

    def gemm(name, M, N, K, dt, peak):
        xg = torch.randn(M, K, device=dev, generator=gen).to(dt)
        wg = (0.02 * torch.randn(N, K, device=dev, generator=gen)).to(dt)
        bg = (0.02 * torch.randn(N, device=dev, generator=gen)).to(dt)
        f = tj.jit(_fn_gemm)
        f(xg, wg, bg)
        ms = kernel_ms_settled(f.compiled(xg, wg, bg), [xg, wg, bg])
        wall = timed_steps(torch, f, [xg, wg, bg], 10, 2)
        flops = 2.0 * M * N * K
        esz = 2 if dt == bf else 4
        nbytes = (M * K + N * K + N + M * N) * esz
        cfg = f.compiled(xg, wg, bg).matmul_configs[0].as_dict()
        out[name] = {"TFLOP/s": round(flops / ms / 1e9, 1), "frac_peak": round(flops / ms / 1e9 / peak, 4),
                     "GB/s": round(nbytes / ms / 1e6, 1), "frac_hbm": round(nbytes / ms / 1e6 / HBM_PEAK_GBS, 4),
                     "kernel_us": round(ms * 1e3, 2), "us_per_call": round(wall * 1e3, 2), "tile": cfg}
        log(f"{name}: {out[name]}")

    gemm("c4_gemm_bf16_8192", 8192, 8192, 8192, bf, BF16_PEAK_TFLOPS)
    gemm("c4_gemm_f32_4096", 4096, 4096, 4096, torch.float32, FP32_PEAK_TFLOPS)
    gemm("c4_skinny_bf16_m16", 16, 8192, 8192, bf, BF16_PEAK_TFLOPS)
    # config 1: MLP block per-call time (hip eager launches and hipGraph replay)
    shapes = [(512, 768), (768,), (3072, 768), (3072,), (768, 3072), (768,)]
    margs = [torch.randn(s, device=dev, generator=gen) * (1 if i < 2 else 0.02) for i, s in enumerate(shapes)]
    res = {}
    for mode in ("0", "1"):
        os.environ["TENSORJIT_HIP_GRAPH"] = mode
        f = tj.jit(_fn_mlp)
        f(*margs)
        res["graph" if mode == "1" else "eager"] = round(timed_steps(torch, f, margs, 200, 20) * 1e3, 2)
    os.environ.pop("TENSORJIT_HIP_GRAPH", None)
    out["c1_mlp_f32_us_per_call"] = res
    log(f"c1_mlp: {res}")
    out["overhead_chain_16_kernels"] = overhead_chain(torch, dev)
    log(f"overhead chain: {out['overhead_chain_16_kernels']}")
    # config 5: chained transformer block, bf16, arena + (optional) hipGraph
    bargs = block_inputs(torch, dev)
    res = {}
    for mode in ("0", "1"):
        os.environ["TENSORJIT_HIP_GRAPH"] = mode
        f = tj.jit(_fn_block)
        f(*bargs)
        res["graph_us" if mode == "1" else "eager_us"] = round(timed_steps(torch, f, bargs, 10, 2) * 1e3, 1)
    os.environ.pop("TENSORJIT_HIP_GRAPH", None)
    cp = f.compiled(*bargs)
    flops = 2851.9e9
    # per-kernel device time inside calls of the whole layer (hipEvents between its
    # launches; the median call of 7 by total), and each kernel repeated alone
    incall = [cp.kernel_times_in_call_ms(*bargs) for _ in range(7)]
    mid = sorted(incall, key=sum)[len(incall) // 2]
    kernels = []
    for i, l in enumerate(cp.launches):
        kus = kernel_ms_settled(cp, bargs, i, rounds=2, iters=5) * 1e3
        entry = {"kernel": l.name, "us_in_call": round(mid[i] * 1e3, 1), "us_alone": round(kus, 1)}
        if "flops" in l.meta:
            entry["TFLOP/s_in_call"] = round(l.meta["flops"] / (mid[i] * 1e3) / 1e6, 1)
            entry["TFLOP/s_alone"] = round(l.meta["flops"] / kus / 1e6, 1)
        kernels.append(entry)
    best = min(res.values())
    out["c5_block_bf16"] = {**res, "TFLOP/s": round(flops / best / 1e6, 1), "frac_peak": round(flops / best / 1e6 / BF16_PEAK_TFLOPS, 4),
                            "kernels": len(cp.launches), "arena_MiB": round(cp.plan.arena_bytes / 2**20, 1),
                            "sum_in_call_us": round(sum(mid) * 1e3, 1),
                            "sum_alone_us": round(sum(k["us_alone"] for k in kernels), 1),
                            "per_kernel": kernels}
    log(f"c5_block: {out['c5_block_bf16']}")
    del bargs, f, cp
    # config 5's attention alone: the fused flash kernel vs the reference plan's three
    # kernels (scores, softmax row kernel, PV product) at the block's shape
    qkv = [torch.randn(4, 32, 2048, 128, device=dev, generator=gen).to(bf) for _ in range(3)]
    res = {}
    for mode in ("1", "0"):
        os.environ["TENSORJIT_HIP_ATTENTION"] = mode
        f = tj.jit(_fn_attn)
        f(*qkv)
        cp = f.compiled(*qkv)
        us = sum(kernel_ms_settled(cp, qkv, i) for i in range(len(cp.launches))) * 1e3
        res["fused_us" if mode == "1" else "unfused_us"] = round(us, 1)
        if mode == "1":
            res["kernel"] = cp.launches[0].name
    os.environ.pop("TENSORJIT_HIP_ATTENTION", None)
    flops = 4.0 * 4 * 32 * 2048 * 2048 * 128
    res["TFLOP/s"] = round(flops / res["fused_us"] / 1e6, 1)
    res["frac_peak"] = round(flops / res["fused_us"] / 1e6 / BF16_PEAK_TFLOPS, 4)
    res["speedup_vs_unfused"] = round(res["unfused_us"] / res["fused_us"], 2)
    out["c5_attention_bf16"] = res
    log(f"c5_attention: {res}")
    out["mfma_sustained_bf16"] = mfma_sustained(torch)
    log(f"mfma_sustained: {out['mfma_sustained_bf16']}")
    out["reference_gpu_table"] = reference_gpu_table(torch, dev)
    log(f"reference GPU table: {out['reference_gpu_table']['readme_rows']}")
    return out


MFMA_PROBE = r"""
extern "C" __global__ __launch_bounds__(256) void mfma_probe(const unsigned short* in0_p, float* out0_p) {
  __shared__ float pad[25600];           // one workgroup (four waves, one per SIMD) per CU
  tj_bf16x8 a[4], b[4];
  const unsigned int base = (blockIdx.x * 256u + threadIdx.x) * 64u;
  for (int f = 0; f < 4; ++f) {
    a[f] = *(const tj_bf16x8*)(in0_p + base + f * 16u);
    b[f] = *(const tj_bf16x8*)(in0_p + base + f * 16u + 8u);
  }
  tj_f32x16 c[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) c[j] = (tj_f32x16)(0.0f);
  pad[threadIdx.x] = (float)threadIdx.x;
  for (int it = 0; it < 2048; ++it) {
#pragma unroll
    for (int x = 0; x < 4; ++x)
#pragma unroll
      for (int y = 0; y < 4; ++y) c[x * 4 + y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[x], b[y], c[x * 4 + y], 0, 0, 0);
  }
  float s = pad[(threadIdx.x + 1) & 255];
#pragma unroll
  for (int j = 0; j < 16; ++j) for (int i = 0; i < 16; ++i) s += c[j][i];
  out0_p[blockIdx.x * 256 + threadIdx.x] = s;
}
extern "C" __global__ __launch_bounds__(256) void mfma_probe16(const unsigned short* in0_p, float* out0_p) {
  __shared__ float pad[25600];           // one workgroup (four waves, one per SIMD) per CU
  tj_bf16x8 a[4], b[4];
  const unsigned int base = (blockIdx.x * 256u + threadIdx.x) * 64u;
  for (int f = 0; f < 4; ++f) {
    a[f] = *(const tj_bf16x8*)(in0_p + base + f * 16u);
    b[f] = *(const tj_bf16x8*)(in0_p + base + f * 16u + 8u);
  }
  tj_f32x4 c[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) c[j] = (tj_f32x4)(0.0f);
  pad[threadIdx.x] = (float)threadIdx.x;
  for (int it = 0; it < 4096; ++it) {
#pragma unroll
    for (int x = 0; x < 4; ++x)
#pragma unroll
      for (int y = 0; y < 4; ++y) c[x * 4 + y] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[x], b[y], c[x * 4 + y], 0, 0, 0);
  }
  float s = pad[(threadIdx.x + 1) & 255];
#pragma unroll
  for (int j = 0; j < 16; ++j) for (int i = 0; i < 4; ++i) s += c[j][i];
  out0_p[blockIdx.x * 256 + threadIdx.x] = s;
}
"""


def mfma_sustained(torch) -> dict:
    """Sustained bf16 MFMA rate of a register-only loop (32x32x16 and 16x16x32, 16
    accumulators, one wave per SIMD) on constant operands and on N(0,1) operands: the
    same instruction stream, timed on the data a GEMM actually multiplies.  The card
    holds a lower clock on random data, so the random-operand rate, not the 2.5 PF
    dense figure, is the ceiling the GEMM fractions should be read against; the
    16x16x32 stream holds a higher one."""
    from tensorjit.backends.hip_backend import compile_source, arch_of
    from tensorjit.backends.hip_prelude import PRELUDE
    from tensorjit.runtime import hip as rt

    code = compile_source(PRELUDE + MFMA_PROBE, arch_of(0))
    nblk = 1024
    n = nblk * 256 * 64
    s = torch.cuda.current_stream().cuda_stream
    res = {}
    # (kernel, key suffix, FLOP per launch): 16 MFMAs per iteration per wave, 4 waves per workgroup
    probes = (("mfma_probe", "", nblk * 4 * 2048 * 16 * 32 * 32 * 16 * 2),
              ("mfma_probe16", "_16x16x32", nblk * 4 * 4096 * 16 * 16 * 16 * 32 * 2))
    for kname, suffix, flops in probes:
        for name, data in (("constant", torch.ones(n, device="cuda")), ("randn", torch.randn(n, device="cuda"))):
            inp = data.to(torch.bfloat16)
            outp = torch.empty(nblk * 256, device="cuda")
            prog = rt.NativeHipProgram(0, code, [kname], [((nblk, 1, 1), (256, 1, 1), 0)],
                                       [[(rt.INPUT, 0), (rt.OUTPUT, 0)]], 0, 1, 1)
            prog.kernel_time(0, [inp.data_ptr()], [outp.data_ptr()], s, 2, 3)
            ms = min(prog.kernel_time(0, [inp.data_ptr()], [outp.data_ptr()], s, 1, 5) for _ in range(3))
            res[f"{name}{suffix}_TFLOP/s"] = round(flops / ms / 1e9, 1)
    res["randn_frac_of_2.5PF"] = round(res["randn_TFLOP/s"] / BF16_PEAK_TFLOPS, 4)
    res["randn_16x16x32_frac_of_2.5PF"] = round(res["randn_16x16x32_TFLOP/s"] / BF16_PEAK_TFLOPS, 4)
    return res


def profile_set(torch, dev, steps, which="all") -> None:
    """Kernels for rocprofv3 runs.  ``all``: the headline kernel, a plain copy-like
    calibration kernel of known traffic (y = x + 0.5, fp32 [16384,4096]: 256 MiB
    read + 256 MiB written), the row configs, the column reduction of fp32 [16384,4096]
    and the split sum of the same 2^26 values, the config-4 bf16 GEMM, its decode
    shape and its fp32 variant, config 5's bf16 softmax rows and fused attention,
    ``steps`` launches each.
    ``c5``: ``steps`` calls of config 5's whole layer (direct launches), for a kernel
    trace of the layer in its own context.  ``c1``: ``steps`` calls of config 1's MLP
    block with direct launches, then ``steps`` with hipGraph replay, back to back (the
    trace's dispatch timestamps show each mode's gaps between kernels).  Each program's
    source digest is logged, so a counter summary names the kernel source it measured.
    ``clock``: ``steps`` launches each of config 5's attention and config 4's bf16 GEMM,
    then the register-only MFMA streams of ``mfma_sustained``; with ``GRBM_COUNT`` (GPU
    clocks per XCD) over each dispatch's own timestamps it gives the clock each kernel
    ran at."""
    import tensorjit as tj

    def run(fn, fargs):
        jf = tj.jit(fn)
        for _ in range(steps):
            jf(*fargs)
        cp = jf.compiled(*fargs)
        log("profile_source " + json.dumps({"launches": [l.name for l in cp.launches], "sha16": source_sha16(cp)}))

    if which == "clock":
        gen = torch.Generator(device=dev).manual_seed(0)
        qkv = [torch.randn(4, 32, 2048, 128, device=dev, generator=gen).bfloat16() for _ in range(3)]
        run(_fn_attn, qkv)
        del qkv
        xg = torch.randn(8192, 8192, device=dev, generator=gen).bfloat16()
        wg = (0.02 * torch.randn(8192, 8192, device=dev, generator=gen)).bfloat16()
        bg = (0.02 * torch.randn(8192, device=dev, generator=gen)).bfloat16()
        run(_fn_gemm, [xg, wg, bg])
        del xg, wg, bg
        log(f"mfma streams: {mfma_sustained(torch)}")
        torch.cuda.synchronize()
        log(f"profile set clock done ({steps} launches per kernel)")
        return

    if which == "c5":
        os.environ["TENSORJIT_HIP_GRAPH"] = "0"
        run(_fn_block, block_inputs(torch, dev))
        torch.cuda.synchronize()
        log(f"profile set c5 done ({steps} calls)")
        return
    if which == "c1":
        gen = torch.Generator(device=dev).manual_seed(0)
        shapes = [(512, 768), (768,), (3072, 768), (3072,), (768, 3072), (768,)]
        margs = [torch.randn(sh, device=dev, generator=gen) * (1 if i < 2 else 0.02) for i, sh in enumerate(shapes)]
        for mode in ("0", "1"):
            os.environ["TENSORJIT_HIP_GRAPH"] = mode
            run(_fn_mlp, margs)
            torch.cuda.synchronize()
            time.sleep(0.05)           # a quiet gap between the two modes in the trace
        os.environ.pop("TENSORJIT_HIP_GRAPH", None)
        log(f"profile set c1 done ({steps} calls per mode)")
        return
    args = c2_inputs(torch, torch.float32, dev)
    run(_fn_c2, args)
    x = args[0]
    run(lambda t: t + 0.5, [x])
    del args, x
    gen = torch.Generator(device=dev).manual_seed(0)
    xb = torch.randn(65536, 4096, device=dev, generator=gen).bfloat16()
    gb = (1 + 0.1 * torch.randn(4096, device=dev, generator=gen)).bfloat16()
    for fn, fargs in ((_fn_ln, [xb, gb]), (_fn_rms, [xb, gb])):
        run(fn, fargs)
    del xb
    s = torch.randn(65536, 2048, device=dev, generator=gen) * 3
    run(_fn_softmax, [s])
    del s
    xc = torch.randn(16384, 4096, device=dev, generator=gen)
    run(_fn_sum_axis0, [xc])
    run(_fn_sum_all, [xc.reshape(-1)])
    del xc
    xg = torch.randn(8192, 8192, device=dev, generator=gen).bfloat16()
    wg = (0.02 * torch.randn(8192, 8192, device=dev, generator=gen)).bfloat16()
    bg = (0.02 * torch.randn(8192, device=dev, generator=gen)).bfloat16()
    run(_fn_gemm, [xg, wg, bg])
    del xg, wg, bg
    xs = torch.randn(16, 8192, device=dev, generator=gen).bfloat16()
    ws = (0.02 * torch.randn(8192, 8192, device=dev, generator=gen)).bfloat16()
    bs = (0.02 * torch.randn(8192, device=dev, generator=gen)).bfloat16()
    run(_fn_gemm, [xs, ws, bs])
    del xs, ws, bs
    xf = torch.randn(4096, 4096, device=dev, generator=gen)
    wf = 0.02 * torch.randn(4096, 4096, device=dev, generator=gen)
    bf = 0.02 * torch.randn(4096, device=dev, generator=gen)
    run(_fn_gemm, [xf, wf, bf])
    del xf, wf, bf
    s5 = (torch.randn(262144, 2048, device=dev, generator=gen) * 3).bfloat16()
    run(_fn_softmax, [s5])
    del s5
    qkv = [torch.randn(4, 32, 2048, 128, device=dev, generator=gen).bfloat16() for _ in range(3)]
    run(_fn_attn, qkv)
    torch.cuda.synchronize()
    log(f"profile set done ({steps} launches per kernel)")


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="CPU baseline sample budget (seconds)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--quick", action="store_true", help="skip the GEMM / MLP secondaries")
    ap.add_argument("--profile-set", nargs="?", const="all", choices=["all", "c5", "c1", "clock"], default=None,
                    help="only launch the kernels used for rocprofv3 runs (no JSON line): 'all' (default) "
                         "the counter set, 'c5' config 5's whole layer, 'c1' config 1 direct then replayed, "
                         "'clock' the MFMA kernels and the register-only MFMA streams (for GRBM_COUNT)")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (every box has one MI355X); "
              "run with --gpus 1", file=sys.stderr)
        return 2

    import torch

    import tensorjit as tj

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    log(f"device {torch.cuda.get_device_name(0)}")
    if a.profile_set:
        profile_set(torch, dev, a.steps, a.profile_set)
        return 0

    args = c2_inputs(torch, torch.float32, dev)
    nbytes = 3 * 16384 * 4096 * 4 + 2 * 4096 * 4       # read x, c, a, b; write y
    f = tj.jit(_fn_c2)
    f(*args)
    cp = f.compiled(*args)
    assert cp.num_kernels == 1 and cp.backend == "hip"
    torch.cuda.synchronize()
    ms_step = timed_steps(torch, f, args, a.steps, a.warmup, ramp_s=0.5)
    kms = kernel_ms(f, args, iters=max(20, a.steps))
    value = nbytes / (ms_step / 1e3) / 1e9
    achieved = nbytes / (kms / 1e3) / 1e9
    log(f"c2 fp32: {value:.1f} GB/s per step ({ms_step * 1e3:.1f} us), kernel {kms * 1e3:.1f} us = {achieved:.1f} GB/s")
    workload = "c2_eltwise_f32"
    sha = source_sha16(cp)
    traffic, traffic_note = load_traffic(workload, sha)
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded torch.randn / rand, BASELINE.json config 2 distributions)",
        "config": {"workload": "config 2: y = gelu(x*a+b)*sigmoid(c)+x, fp32 x,c[16384,4096], a,b[4096]; "
                               "one fused hip kernel via tj.jit", "numel": 16384 * 4096,
                   "algorithmic_bytes": nbytes, "kernels": cp.num_kernels,
                   "hip_graph": cp.use_graph, "kernel": cp.launches[0].name},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel_us": round(kms * 1e3, 2), "source_sha16": sha},
    }
    if traffic_note:
        line["roofline"]["traffic_note"] = traffic_note
    if not a.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(torch, args, nbytes, a.cpu_seconds)
        log(f"cpu baseline: {line['cpu_baseline']}")
    else:
        line["cpu_baseline"] = None
    del args
    if not a.no_secondary:
        line["secondary"] = secondary(torch, dev, a.quick)
        if not a.no_cpu_baseline and not a.quick:
            line["secondary"]["cpu_oracle"] = cpu_secondary(torch)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
