"""hip backend: fused kernel program -> gfx950 HIP C++ -> hipRTC -> C-ABI executor.

``compile_program(program, device, tune)`` is the backend entry point that
``tensorjit.compiler.compile_graph`` dispatches to for ``backend="hip"``,
in the place of the reference's ``cuda_backend.compile_program``
(``tensorjit/backends/cuda_backend.py:556-557``).  It returns a
``HipProgram`` with the executor protocol of the reference's
``CudaProgram`` (``tensorjit/backends/cuda_backend.py:459-553``): callable on
torch tensors, ``num_kernels``, ``source`` (HIP), ``launches``, ``plan``,
``stats`` (``calls`` / ``graph_replays``), ``matmul_configs``.

Everything below ``HipProgram.__call__`` is native: the pointer tables go to
``libtjhip.so`` (``tj_hip_program_run`` / ``tj_hip_program_replay``), which
launches the kernels on torch's current HIP stream.  There is no other
execution path; a missing library or GPU raises.
"""
from __future__ import annotations

import logging
import math
import os
import threading

import torch

from ..ir import DType, Node, OpKind
from ..passes import Kernel, Program
from ..passes.fusion import _finalize
from ..passes.memory_planner import MemoryPlan, plan_memory
from ..runtime import hip as rt
from ..runtime.autotune import HIP_CANDIDATES, HIP_F32_CANDIDATES, MatmulConfig, autotune, cost_model
from ..runtime.cache import AutotuneStore, CodeObjectCache
from ..runtime.dtypes import TORCH_DTYPE
from ..runtime.pool import BufferPool
from .hip_attention import fuse_attention, gen_attention
from .hip_gemm import compute_dtype, config_ok, gen_matmul, matmul_dims
from .hip_kernels import KernelGen, Launch, gen_colreduce, gen_copy, gen_elementwise, gen_row
from .hip_prelude import PRELUDE

log = logging.getLogger("tensorjit")

DEFAULT_ARCH = "gfx950"
NO_PACKED_FP32 = ("-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops")
COMPILE_OPTS = ("-O3", "-std=c++17", "-fno-strict-aliasing", *NO_PACKED_FP32)


# ---------------------------------------------------------------------------
# tile selection
# ---------------------------------------------------------------------------


def _candidates(k: Kernel) -> list[MatmulConfig]:
    dt = compute_dtype(k.anchor)
    return [c for c in (HIP_F32_CANDIDATES if dt == DType.f32 else HIP_CANDIDATES) if config_ok(c, dt, k.anchor)]


def matmul_key(k: Kernel, arch: str) -> str:
    mm = k.anchor
    M, N, K, tb = matmul_dims(mm)
    batch = math.prod(mm.shape[:-2]) if len(mm.shape) > 2 else 1
    dt = compute_dtype(mm)
    return f"hip|{arch}|matmul|{batch}x{M}x{N}x{K}|{dt.value}|tb{int(tb)}|epi{len(k.nodes) - 1}"


def analytic_config(k: Kernel) -> MatmulConfig:
    mm = k.anchor
    M, N, K, _ = matmul_dims(mm)
    batch = math.prod(mm.shape[:-2]) if len(mm.shape) > 2 else 1
    dt = compute_dtype(mm)
    kind = "hip_f32" if dt == DType.f32 else "hip"
    return min(_candidates(k), key=lambda c: cost_model(c, M, N, K, kind, batch))


# ---------------------------------------------------------------------------
# code generation
# ---------------------------------------------------------------------------


def reject_zero_size(nodes) -> None:
    """Zero-size tensors are not supported: every generated kernel assumes a non-empty
    iteration space (the pointwise family would run one unguarded workgroup), so such a
    program is refused before any code is generated or memory allocated, with the
    ``NotImplementedError`` that sends torch.compile back to eager."""
    for n in nodes:
        if any(d == 0 for d in n.shape):
            raise NotImplementedError(f"{n.name}: zero-size tensor {tuple(n.shape)} is not supported by the hip backend")


def generate_kernel(k: Kernel, idx: int, cfg: MatmulConfig | None = None) -> tuple[str, Launch | list[Launch]]:
    """HIP source of one fused kernel and its launch(es).  A GEMM whose K is split
    across workgroups (``KSPLIT``) writes partial products into a workspace and sums
    them, with the fused epilogue, in each output tile's last workgroup; the M <= 32
    decode kernel (and ``TENSORJIT_HIP_KSPLIT_FUSED=0``) sums them in a second launch."""
    reject_zero_size(list(k.inputs) + list(k.nodes) + list(k.outputs))
    g = KernelGen.of(k, idx)
    if k.kind == "elementwise":
        return gen_elementwise(g)
    if k.kind == "copy":
        return gen_copy(g)
    if k.kind == "row":
        return gen_row(g, k.stages, tuple(k.rows), k.n)  # type: ignore[attr-defined]
    if k.kind == "reduce":
        x = k.anchor.inputs[0]
        return gen_row(g, [k], tuple(x.shape[:-1]), x.shape[-1])
    if k.kind == "matmul":
        return gen_matmul(g, cfg or analytic_config(k))
    if k.kind == "attention":
        return gen_attention(k, idx)
    if k.kind == "colreduce":
        return gen_colreduce(g)
    raise NotImplementedError(k.kind)


def generate(program: Program, configs: dict[int, MatmulConfig] | None = None) -> tuple[str, list[Launch]]:
    """HIP source of the whole program (prelude + the ``extern "C"`` kernels of every fused
    kernel) and its launches in order; ``meta["kernel"]`` is each launch's kernel index."""
    configs = configs or {}
    sources, launches = [PRELUDE], []
    for idx, k in enumerate(program.kernels):
        src, ls = generate_kernel(k, idx, configs.get(idx))
        sources.append(src)
        for launch in ls if isinstance(ls, list) else [ls]:
            launch.meta["kernel"] = idx
            launches.append(launch)
    return "\n\n".join(sources), launches


WS_ALIGN = 256


def workspace_layout(launches: list[Launch], base: int) -> tuple[dict[int, tuple[int, int]], int]:
    """Arena ``(offset, bytes)`` of each kernel's workspace (split-K partials), placed
    after the planned intermediates (``base`` bytes) in the same allocation, and the
    total arena size."""
    off = -(-base // WS_ALIGN) * WS_ALIGN
    ws: dict[int, tuple[int, int]] = {}
    for launch in launches:
        need = launch.meta.get("workspace", 0)
        if need:
            ws[launch.meta["kernel"]] = (off, need)
            off += -(-need // WS_ALIGN) * WS_ALIGN
    return ws, (off if ws else base)


def launch_args(launches: list[Launch], kernel_args: list[list], ws: dict[int, tuple[int, int]]) -> list[list]:
    """Per-launch pointer refs: the kernel's inputs and outputs, plus its workspace for
    the launches that take one (``meta["ws_arg"]``) as ``(ARENA, offset, bytes)``."""
    out = []
    for launch in launches:
        idx = launch.meta["kernel"]
        refs = list(kernel_args[idx])
        if launch.meta.get("ws_arg"):
            refs.append((rt.ARENA, *ws[idx]))
        out.append(refs)
    return out


# ---------------------------------------------------------------------------
# compilation
# ---------------------------------------------------------------------------

_compile_lock = threading.Lock()


def target_of(device_index: int | None) -> str:
    """The device's full ``gcnArchName`` (e.g. ``gfx950:sramecc+:xnack-``), or
    ``TENSORJIT_HIP_ARCH`` when set."""
    forced = os.environ.get("TENSORJIT_HIP_ARCH")
    if forced:
        return forced
    if device_index is None:
        return DEFAULT_ARCH
    return rt.device_info(device_index).arch.decode()


def arch_of(device_index: int | None) -> str:
    """The gfx processor of the device (``gfx950``): the hipRTC ``--offload-arch``."""
    return target_of(device_index).split(":")[0]


_toolchain: str | None = None


def toolchain_tag() -> str:
    """hipRTC and HIP runtime versions plus this library's ABI: part of every cached
    code object's key, so a ROCm upgrade recompiles instead of loading old code."""
    global _toolchain
    if _toolchain is None:
        major, minor, runtime = rt.toolchain_version()
        _toolchain = f"hiprtc{major}.{minor}-hip{runtime}-abi{rt.ABI_VERSION}"
    return _toolchain


def compile_source(source: str, arch: str, name: str = "tensorjit.hip", target: str | None = None) -> bytes:
    """hipRTC compile for ``--offload-arch=arch`` with an on-disk code-object cache keyed
    by source, options, the full target name (``target``, default ``arch``) and the
    toolchain."""
    opts = (f"--offload-arch={arch}", *COMPILE_OPTS)
    cache = CodeObjectCache(target or arch, toolchain_tag())
    code = cache.get(source, opts)
    if code is not None:
        return code
    with _compile_lock:
        code = rt.compile_source(source, name, opts)
    cache.put(source, opts, code)
    return code


# ---------------------------------------------------------------------------
# executor
# ---------------------------------------------------------------------------

def _stream_of(device_index: int) -> int:
    return torch.cuda.current_stream(device_index).cuda_stream


# torch's current HIP stream of a device as a raw handle: the private accessor skips building
# a Stream object (~1 us per call); torch builds without it use the public API
_current_stream = getattr(torch._C, "_cuda_getCurrentRawStream", _stream_of)


def fold_elementwise_into_gemm(program: Program) -> Program:
    """Move an elementwise kernel into the epilogue of the GEMM that produces one of its
    inputs, when that GEMM result has no other use.

    The reference's greedy fusion joins an elementwise node to the kernel of its
    *first* input only, and gives up when that would form a cycle.  A transformer
    layer's second residual, ``h + linear(gelu(linear(rms(h))), w2)``, whose first input
    ``h`` comes from the out-projection's kernel, therefore stays a kernel of its own
    behind the down-projection, and the 64 MiB down-projection result makes a round
    trip through HBM.  The merged kernel takes the elementwise kernel's place in the
    schedule: the GEMM's inputs exist earlier, and the elementwise kernel's other inputs
    exist there.  ``lower()`` keeps the reference plan; ``TENSORJIT_HIP_GEMM_EPILOGUE=0``
    keeps it here too."""
    if os.environ.get("TENSORJIT_HIP_GEMM_EPILOGUE", "1") == "0":
        return program
    kernels = list(program.kernels)
    outs = {id(program.resolve(o)) for o in program.graph.outputs}
    producer = {id(o): i for i, k in enumerate(kernels) for o in k.outputs}
    changed = False
    e = 0
    while e < len(kernels):
        ek = kernels[e]
        merged = None
        if ek.kind == "elementwise":
            inside = {id(n) for n in ek.nodes}
            for v in ek.inputs:
                m = producer.get(id(v))
                if m is None or m >= e or kernels[m].kind != "matmul":
                    continue
                mk = kernels[m]
                shape = tuple(mk.anchor.shape)
                if (mk.outputs != [v] or id(v) in outs or any(id(u) not in inside for u in v.users)
                        or any(tuple(n.shape) != shape or n.kind != OpKind.ELEMENTWISE for n in ek.nodes)):
                    continue
                ins = list(mk.inputs)
                for i in ek.inputs:
                    if i is not v and all(i is not j for j in ins):
                        ins.append(i)
                merged = (m, Kernel("matmul", nodes=mk.nodes + ek.nodes, anchor=mk.anchor, inputs=ins,
                                    outputs=list(ek.outputs)))
                break
        if merged is None:
            e += 1
            continue
        m, k = merged
        kernels[e] = k
        del kernels[m]
        producer = {id(o): i for i, kk in enumerate(kernels) for o in kk.outputs}
        changed = True
        e = kernels.index(k) + 1
    return Program(program.graph, kernels, program.aliases) if changed else program


COL_MIN_BYTES = 512       # a column block's row (64 lanes) must hold at least this many bytes


def fold_transpose_into_reduce(program: Program) -> Program:
    """Turn a transpose kernel whose every reader is a stand-alone reduction of its last
    axis into ``colreduce`` kernels that reduce the source's axis in place.

    The reference plan reduces a non-last axis by copying it last (a transpose kernel)
    and reducing rows: the tensor crosses HBM three times (read, write, read), four with
    two reductions of it.  Each column reduction reads it once.  It applies when the
    transpose keeps every other axis in order (the source is then [A, Rd, B] with the
    reduced axis Rd in the middle, and the outputs' order is [A, B]), each reduction's
    prologue is elementwise on the transposed value alone, nothing but the reductions'
    values and epilogues escape, and a row of B holds at least COL_MIN_BYTES bytes.  With
    one reduction, an elementwise kernel whose only output is the transposed source, read
    by nothing else, becomes its prologue too.  ``TENSORJIT_HIP_COLREDUCE=0`` keeps the
    reference plan."""
    if os.environ.get("TENSORJIT_HIP_COLREDUCE", "1") == "0":
        return program
    kernels = list(program.kernels)
    outs = {id(program.resolve(o)) for o in program.graph.outputs}
    changed = False
    c = 0
    while c < len(kernels):
        folded = _col_fold(kernels, c, outs)
        if folded is None:
            c += 1
            continue
        new, drop = folded
        for i, k in new.items():
            kernels[i] = k
        for d in sorted(drop, reverse=True):
            del kernels[d]
        changed = True
        c = 0           # the drops shift the indices: scan again from the start
    return Program(program.graph, kernels, program.aliases) if changed else program


def _col_fold(kernels: list[Kernel], c: int, outs: set) -> tuple[dict[int, Kernel], list[int]] | None:
    """Column reductions replacing transpose kernel ``c`` and its readers, or None."""
    ck = kernels[c]
    if ck.kind != "copy" or len(ck.nodes) != 1 or ck.nodes[0].op != "transpose" or ck.outputs != ck.nodes:
        return None
    t = ck.nodes[0]
    if id(t) in outs:
        return None
    perm = tuple(t.attrs["perm"])
    a = perm[-1]
    if a == len(perm) - 1 or list(perm[:-1]) != sorted(perm[:-1]):
        return None
    X = t.inputs[0]
    Sx = tuple(X.shape)
    A, Rd, B = math.prod(Sx[:a]), Sx[a], math.prod(Sx[a + 1:])
    if B * X.dtype.itemsize < COL_MIN_BYTES:
        return None
    owner = {id(n): i for i, k in enumerate(kernels) for n in k.nodes}
    readers = sorted({owner.get(id(u), -1) for u in t.users})
    if not readers or any(r < 0 or not _col_reduce_ok(kernels[r], t) for r in readers):
        return None
    producer = {id(o): j for j, k in enumerate(kernels) for o in k.outputs}
    drop = [c]
    xnodes: list[Node] = []
    xins = [X]
    e = producer.get(id(X))
    if len(readers) == 1 and e is not None and kernels[e].kind == "elementwise":
        ek = kernels[e]
        if (ek.outputs == [X] and id(X) not in outs and all(u is t for u in X.users)
                and all(tuple(n.shape) == Sx and n.kind == OpKind.ELEMENTWISE for n in ek.nodes)):
            xnodes, xins = list(ek.nodes), list(ek.inputs)
            drop.append(e)
    new = {}
    for r in readers:
        rk = kernels[r]
        ins = list(xins)
        for n in rk.inputs:
            if n is not t and all(n is not x for x in ins):
                ins.append(n)
        k = Kernel("colreduce", nodes=xnodes + list(rk.nodes), anchor=rk.anchor, inputs=ins, outputs=list(rk.outputs))
        k.src, k.tnode, k.col, k.xnodes = X, t, (A, Rd, B), xnodes  # type: ignore[attr-defined]
        new[r] = k
    return new, drop


def _col_reduce_ok(rk: Kernel, t: Node) -> bool:
    """``rk`` is a stand-alone sum / mean / max of ``t``'s last axis whose prologue reads
    only ``t`` (and scalar constants), whose epilogue reads only the reduction, itself and
    outside inputs, and which lets only per-output values escape."""
    if rk.kind != "reduce" or rk.anchor.op not in ("sum", "mean", "max"):
        return False
    red = rk.anchor
    pos = rk.nodes.index(red)
    prologue, epilogue = rk.nodes[:pos], rk.nodes[pos + 1:]
    inside = {id(n) for n in rk.nodes}
    vec_in = [n for n in rk.inputs if any(n in m.inputs for m in prologue + [red])]
    if len(vec_in) != 1 or vec_in[0] is not t:
        return False
    for n in prologue:
        if any(id(x) not in inside and x is not t and not (x.op == "const" and x.shape == ()) for x in n.inputs):
            return False
    pro = {id(n) for n in prologue}
    if any(id(x) in pro or x is t for n in epilogue for x in n.inputs):
        return False
    return not any(id(o) in pro for o in rk.outputs)


def sink_epilogue_into_rows(program: Program) -> Program:
    """Move a GEMM epilogue value whose only readers are one stage of a later row kernel
    into that stage, when everything it reads the row kernel can read too.

    Config 5's second RMSNorm squares the out-projection's result ``x1``: the greedy
    fusion puts ``x1 * x1`` into the out-projection's epilogue (its input's kernel), so
    the GEMM stores it (64 MiB) and the row kernel reads it beside ``x1`` itself.
    Computed in the row kernel's reduction stage instead, the GEMM stores one output and
    the row kernel streams one input (its second read of a row hits L2).  The square is
    then taken of the stored ``x1`` (rounded to the storage type) rather than of the
    fp32 accumulator, a rounding difference below the storage precision.
    ``TENSORJIT_HIP_GEMM_EPILOGUE=0`` keeps the reference plan."""
    if os.environ.get("TENSORJIT_HIP_GEMM_EPILOGUE", "1") == "0":
        return program
    kernels = list(program.kernels)
    g = program.graph
    outs = {id(program.resolve(o)) for o in g.outputs}
    changed = False
    for mi in range(len(kernels)):
        mk = kernels[mi]
        if mk.kind != "matmul":
            continue
        for o in list(mk.outputs):
            if o is mk.anchor or o.kind != OpKind.ELEMENTWISE or id(o) in outs or not o.users:
                continue
            ri = next((i for i, k in enumerate(kernels) if any(o.users[0] is n for n in k.nodes)), None)
            if ri is None or ri <= mi or kernels[ri].kind != "row":
                continue
            rk = kernels[ri]
            stage = next(st for st in rk.stages if any(o.users[0] is n for n in st.nodes))
            vec_shape = tuple(rk.rows) + (rk.n,)
            readable = [x for x in mk.outputs if x is not o] + list(mk.inputs)
            if (not all(any(u is n for n in stage.nodes) for u in o.users)
                    or tuple(o.shape) != vec_shape or tuple(stage.iter_shape) != vec_shape
                    or not all(i.op == "const" or any(i is x for x in readable) for i in o.inputs)):
                continue
            new_m = Kernel("matmul", nodes=[n for n in mk.nodes if n is not o], anchor=mk.anchor)
            _finalize(new_m, g)
            new_stages = []
            for st in rk.stages:
                if st is stage:
                    st = Kernel(st.kind, nodes=[o] + st.nodes, anchor=st.anchor)
                    _finalize(st, g)
                new_stages.append(st)
            new_r = Kernel("row", nodes=[o] + rk.nodes)
            new_r.stages, new_r.rows, new_r.n = new_stages, rk.rows, rk.n  # type: ignore[attr-defined]
            _finalize(new_r, g)
            kernels[mi], kernels[ri] = new_m, new_r
            mk = new_m
            changed = True
    return Program(g, kernels, program.aliases) if changed else program


# hipGraph replay by default from this many launches per call.  Measured on MI355X with the
# reference's overhead chain (softmax(x @ w + 0.5) repeated): a direct hipModuleLaunchKernel
# costs 2.3-2.8 us of host time, a graph launch 21-25 us plus ~0.6 us per kernel node, so
# 8 launches run 30 us direct / 33 us replayed and 16 launches 48 / 41 us.
# TENSORJIT_HIP_GRAPH=1 / 0 forces replay on / off.
GRAPH_MIN_LAUNCHES = 12


class HipProgram:
    """A compiled program bound to one GPU (see module docstring for the protocol)."""

    def __init__(self, program: Program, device: str | torch.device = "cuda", use_graph: bool | None = None,
                 tune: bool = True):
        reject_zero_size(list(program.graph.inputs) + [n for k in program.kernels for n in k.nodes])
        # backend-level rewrites of the planned program: attention chains -> one kernel,
        # elementwise kernels behind a GEMM -> its epilogue, epilogue values only a row
        # kernel reads -> that row kernel, transpose -> reduce -> one column reduction
        program = fold_transpose_into_reduce(sink_epilogue_into_rows(fold_elementwise_into_gemm(fuse_attention(program))))
        self.program = program
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError(f"the hip backend runs on ROCm GPU tensors (device 'cuda'), got {self.device}")
        if not torch.cuda.is_available():
            raise rt.HipError("the hip backend needs a ROCm GPU; torch.cuda.is_available() is False")
        self.device_index = self.device.index if self.device.index is not None else torch.cuda.current_device()
        self.backend = "hip"
        self.target = target_of(self.device_index)
        self.arch = self.target.split(":")[0]
        self.plan: MemoryPlan = plan_memory(program)
        self.matmul_configs: dict[int, MatmulConfig] = {}
        self._tuned_ms: dict[int, float] = {}
        self._native: rt.NativeHipProgram | None = None
        g = program.graph
        self._input_index = {id(n): i for i, n in enumerate(g.inputs)}
        returned = {id(program.resolve(o)) for o in g.outputs}
        self._out_nodes: list[Node] = []
        for k in program.kernels:
            for o in k.outputs:
                if id(o) in returned and all(o is not x for x in self._out_nodes):
                    self._out_nodes.append(o)
        self._out_index = {id(o): j for j, o in enumerate(self._out_nodes)}
        self._args = [[self._ref(i) for i in k.inputs] + [self._ref(o) for o in k.outputs] for k in program.kernels]
        self._out_specs = [(tuple(o.shape), TORCH_DTYPE[o.dtype]) for o in self._out_nodes]

        for idx, k in enumerate(program.kernels):
            if k.kind == "matmul":
                self.matmul_configs[idx] = self._pick_config(k, idx, tune)
        self.source, self.launches = generate(program, self.matmul_configs)
        self.code = compile_source(self.source, self.arch, target=self.target)
        self._workspace, self.arena_bytes = workspace_layout(self.launches, self.plan.arena_bytes)
        self._native = self._load(self.code, self.launches, launch_args(self.launches, self._args, self._workspace))

        self.pool = BufferPool()
        self._init_call_path()
        env = os.environ.get("TENSORJIT_HIP_GRAPH")
        if use_graph is None:
            use_graph = env == "1" if env in ("0", "1") else len(self.launches) >= GRAPH_MIN_LAUNCHES
        self.use_graph = use_graph
        self._calls = 0

    # -- construction helpers -------------------------------------------------------
    def _ref(self, n: Node) -> tuple[int, ...]:
        src = self.program.resolve(n)
        if id(src) in self._input_index:
            return rt.INPUT, self._input_index[id(src)]
        if id(src) in self._out_index:
            return rt.OUTPUT, self._out_index[id(src)]
        off = self.plan.offset(src)
        if off is None:
            raise RuntimeError(f"{n.name} has no storage (not an input, output or planned intermediate)")
        return rt.ARENA, off, (math.prod(src.shape) if src.shape else 1) * src.dtype.itemsize

    def _load(self, code: bytes, launches: list[Launch], args) -> rt.NativeHipProgram:
        return rt.NativeHipProgram(self.device_index, code, [l.name for l in launches],
                                   [(l.grid, l.block, l.shared) for l in launches], args,
                                   self.arena_bytes, len(self.program.graph.inputs), len(self._out_nodes))

    def _pick_config(self, k: Kernel, idx: int, tune: bool) -> MatmulConfig:
        store = AutotuneStore()
        key = matmul_key(k, self.arch)
        cached = store.get(key)
        if cached is not None:
            cfg = MatmulConfig.from_dict(cached["config"])
            if config_ok(cfg, compute_dtype(k.anchor), k.anchor):
                return cfg
        if not tune or os.environ.get("TENSORJIT_NO_AUTOTUNE") == "1":
            return analytic_config(k)
        return self._autotune(k, idx, key, store)

    def _autotune(self, k: Kernel, idx: int, key: str, store: AutotuneStore) -> MatmulConfig:
        """Time the cost model's best candidates on random buffers of the kernel's shapes."""
        mm = k.anchor
        M, N, K, _ = matmul_dims(mm)
        batch = math.prod(mm.shape[:-2]) if len(mm.shape) > 2 else 1
        dt = compute_dtype(mm)
        kind = "hip_f32" if dt == DType.f32 else "hip"
        dev = self.device
        ins = [torch.randn(i.shape, device=dev).to(TORCH_DTYPE[i.dtype]) for i in k.inputs]
        outs = [torch.empty(o.shape, device=dev, dtype=TORCH_DTYPE[o.dtype]) for o in k.outputs]
        single = Program(self.program.graph, [k], {})
        args = [[(rt.INPUT, j) for j in range(len(k.inputs))] + [(rt.OUTPUT, j) for j in range(len(k.outputs))]]
        stream = torch.cuda.current_stream(dev).cuda_stream

        def build(cfg: MatmulConfig):
            src, launches = generate(single, {0: cfg})
            code = compile_source(src, self.arch, target=self.target)
            ws, arena = workspace_layout(launches, 0)
            prog = rt.NativeHipProgram(self.device_index, code, [l.name for l in launches],
                                       [(l.grid, l.block, 0) for l in launches], launch_args(launches, args, ws),
                                       arena, len(ins), len(outs))
            ip, op = [t.data_ptr() for t in ins], [t.data_ptr() for t in outs]
            # a kernel of several launches (the decode split-K and its sum) is timed as their sum
            return lambda warmup, iters: sum(prog.kernel_time(i, ip, op, stream, warmup, iters)
                                             for i in range(len(launches)))

        def timer(run, warmup, iters):
            # enough launches for ~2 ms of device time per measurement (>= 3)
            first = run(1, 1)
            n = int(min(max(3, 2.0 / max(first, 1e-3)), 200))
            return run(warmup, n)

        return autotune(key, _candidates(k), build, (M, N, K, batch), kind, store=store, timer=timer, top_k=6,
                        rounds=3)

    # -- protocol ---------------------------------------------------------------
    @property
    def stats(self) -> dict:
        """Calls, and of the graph-mode calls: hipGraph replays, captures, and calls that
        launched directly because their pointer sets did not recur (the native runtime's
        counters; the reference's ``CudaProgram.stats`` has the first two)."""
        n = self._native.stats() if self._native is not None else {}
        return {"calls": self._calls, "graph_replays": n.get("graph_replays", 0),
                "graph_captures": n.get("graph_captures", 0), "direct_fallbacks": n.get("direct_fallbacks", 0)}

    @property
    def num_kernels(self) -> int:
        """Fused kernels of the plan (a split-K decode GEMM is one kernel with two launches)."""
        return len(self.program.kernels)

    @property
    def native(self) -> rt.NativeHipProgram:
        return self._native

    def _init_call_path(self) -> None:
        """Everything a call needs that does not depend on the call's tensors."""
        g = self.program.graph
        self._in_checks = [(n.name, torch.Size(n.shape), TORCH_DTYPE[n.dtype]) for n in g.inputs]
        self._dev = torch.device("cuda", self.device_index)
        out_pos = {id(o): j for j, o in enumerate(self._out_nodes)}
        in_pos = {id(n): i for i, n in enumerate(g.inputs)}
        # per graph output: (0, output j) / (1, input i) / (2, const node), and its shape when
        # it is a reshape alias of that value
        self._result_plan = []
        for o in g.outputs:
            src = self.program.resolve(o)
            if id(src) in out_pos:
                kind, what = 0, out_pos[id(src)]
            elif id(src) in in_pos:
                kind, what = 1, in_pos[id(src)]
            elif src.op == "const":
                kind, what = 2, src
            else:
                raise RuntimeError(f"output {o.name} is not produced by any kernel")
            reshape = tuple(o.shape) if tuple(src.shape) != tuple(o.shape) else None
            self._result_plan.append((kind, what, reshape))

    def _prepare(self, inputs) -> list[torch.Tensor]:
        if len(inputs) != len(self._in_checks):
            raise TypeError(f"expected {len(self._in_checks)} inputs, got {len(inputs)}")
        ins = []
        for (name, shape, dtype), t in zip(self._in_checks, inputs):
            if not isinstance(t, torch.Tensor):
                raise TypeError(f"{name}: expected a torch.Tensor, got {type(t)}")
            if t.shape != shape or t.dtype != dtype:
                raise ValueError(f"{name}: expected {tuple(shape)} {dtype}, got {tuple(t.shape)} {t.dtype}")
            if t.get_device() != self.device_index:
                raise ValueError(f"{name}: tensor on {t.device}, program compiled for {self._dev}")
            if not t.is_contiguous():
                t = t.contiguous()
            if t.data_ptr() % 16:
                t = t.clone()   # 16-byte vector loads need 16-byte aligned bases
            ins.append(t)
        return ins

    def __call__(self, *inputs: torch.Tensor) -> list[torch.Tensor]:
        ins = self._prepare(inputs)
        take, dev = self.pool.take_output, self._dev
        outs = [take(shape, dtype, dev) for shape, dtype in self._out_specs]
        stream = _current_stream(self.device_index)
        self._calls += 1
        if self.launches:
            if self.use_graph:
                self._native.replay_tensors(ins, outs, stream)
            else:
                self._native.run_tensors(ins, outs, stream)
        return self._results(ins, outs)

    def _results(self, ins: list[torch.Tensor], outs: list[torch.Tensor]) -> list[torch.Tensor]:
        result = []
        for kind, what, reshape in self._result_plan:
            if kind == 0:
                t = outs[what]
            elif kind == 1:
                t = ins[what]
            else:
                t = torch.full(what.shape, what.attrs["value"], dtype=TORCH_DTYPE[what.dtype], device=self._dev)
            result.append(t if reshape is None else t.reshape(reshape))
        return result

    # -- measurement helpers --------------------------------------------------------
    def kernel_time_ms(self, k: int, *inputs: torch.Tensor, warmup: int = 3, iters: int = 20,
                       outputs: list[torch.Tensor] | None = None) -> float:
        """Average device time of kernel ``k`` (hipEvents on torch's current stream)."""
        ins = self._prepare(inputs)
        outs = outputs or [torch.empty(s, dtype=d, device=self.device) for s, d in self._out_specs]
        stream = torch.cuda.current_stream(self.device).cuda_stream
        return self._native.kernel_time(k, [t.data_ptr() for t in ins], [t.data_ptr() for t in outs], stream,
                                        warmup, iters)

    def kernel_times_in_call_ms(self, *inputs: torch.Tensor) -> list[float]:
        """Device time of every launch within one call of the whole program (hipEvents
        between the launches on torch's current stream), in launch order."""
        ins = self._prepare(inputs)
        outs = [torch.empty(s, dtype=d, device=self.device) for s, d in self._out_specs]
        stream = torch.cuda.current_stream(self.device).cuda_stream
        return self._native.time_kernels([t.data_ptr() for t in ins], [t.data_ptr() for t in outs], stream,
                                         len(self.launches))

    def native_stats(self) -> dict:
        return self._native.stats()


def compile_program(program: Program, device: str = "cuda", tune: bool = True) -> HipProgram:
    return HipProgram(program, device=device, tune=tune)
