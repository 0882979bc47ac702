"""The flash-attention kernel's DMA schedule (head dim 128, 8 waves), checked on the CPU
from its generated source.

K and V blocks move from memory into LDS with ``buffer_load_dwordx4 ... lds``: one
instruction writes lane ``l``'s 16 bytes at byte ``16 l`` of a 1 KiB block, so the
swizzle lives in which global chunk each lane fetches.  These tests evaluate the
generated expressions for every wave and lane and check that (a) the DMA of one block
fills each 16-byte LDS slot of a stage exactly once, with the 64 rows x 16 chunks of
the block, (b) each score-fragment read returns K row ``t*32 + lane % 32``, chunk
``2c + lane / 32`` (the 32x32x16 MFMA's operand), (c) each transposing V read returns
the 8 bytes the padded-row kernel reads (row ``ch*16 + g*4 + (lane % 16)/4`` (+8),
columns ``u*32 + ((lane/16) % 2)*16 + (lane % 4)*4`` .. +3), (d) the reads are
conflict-free under the LDS model of the GEMM layout test for 16-byte reads (32 lanes a
pass over 512 bytes of banks) and with 16 or 8 lanes a pass over 256 or 128 bytes (the
padded rows' property) and, for the transposing 8-byte reads, with each half-wave
over 256 bytes (a V swizzle that was conflict-free only over 512 bytes measured 3.4e7
conflict cycles per [4,32,2048,128] launch, the padded rows 0) and the whole wave over
512 bytes, and (e) the
ping-pong schedule itself -- DMA issues, wait counts and barriers of both wave groups,
expanded from the source -- never reads a stage before both groups' halves of the
expected block have landed and been published, and never overwrites one that a group
may still read.
"""
import os
import re

import pytest

import tensorjit as tj
import tensorjit.compiler as C
from tensorjit.backends import hip_backend as hb
from tensorjit.backends.hip_attention import fuse_attention
from tensorjit.ir import DType, TensorType

BKV = 64


@pytest.fixture(autouse=True)
def _eight_waves(monkeypatch):
    monkeypatch.setenv("TENSORJIT_HIP_ATTENTION_WAVES", "8")
    monkeypatch.delenv("TENSORJIT_HIP_ATTENTION_DMA", raising=False)


def _source(Sk=2048, Sq=1024, layout="bhsd", H=2, mi16=False):
    """The generated source and launch; ``mi16``: the 16x16x32 form of the schedule."""
    old = os.environ.get("TENSORJIT_HIP_ATTENTION_MI16")
    os.environ["TENSORJIT_HIP_ATTENTION_MI16"] = "1" if mi16 else "0"
    try:
        return _source_env(Sk, Sq, layout, H, mi16)
    finally:
        if old is None:
            os.environ.pop("TENSORJIT_HIP_ATTENTION_MI16")
        else:
            os.environ["TENSORJIT_HIP_ATTENTION_MI16"] = old


def _source_env(Sk, Sq, layout, H, mi16):
    fn = lambda q, k, v: tj.matmul(tj.softmax(tj.matmul(q, tj.transpose(k, -1, -2)) * 0.088), v)  # noqa: E731
    if layout == "bshd":
        tq = lambda t: tj.transpose(t, 1, 2)  # noqa: E731
        fn2 = lambda q, k, v: fn(tq(q), tq(k), tq(v))  # noqa: E731
        shapes = [(1, Sq, H, 128), (1, Sk, H, 128), (1, Sk, H, 128)]
    else:
        fn2 = fn
        shapes = [(1, H, Sq, 128), (1, H, Sk, 128), (1, H, Sk, 128)]
    p = fuse_attention(C.lower(tj.trace(fn2, [TensorType(s, DType.bf16) for s in shapes]), "hip"))
    src, launches = hb.generate(p)
    (launch,) = launches if isinstance(launches, list) else [launches]
    assert launch.meta["family"] == "attention" and launch.meta["schedule"] == "pingpong-dma", launch.meta
    assert launch.meta["mfma"] == ("16x16x32" if mi16 else "32x32x16"), launch.meta
    return src, launch


def _c_eval(expr: str, env: dict) -> int:
    py = re.sub(r"(\d+)u\b", r"\1", expr).replace("(unsigned int)", "").replace("/", "//")
    return int(eval(py, {}, dict(env))) & 0xFFFFFFFF


def _expr(src: str, pattern: str) -> str:
    m = re.search(pattern, src)
    assert m, pattern
    return m.group(1)


def _lane_env(lane: int, wave: int) -> dict:
    return {"lane": lane, "wave": wave, "wv": wave, "gq": wave // 4, "g": lane // 32, "col": lane % 32}


def _setup(src: str):
    """The per-lane set-up expressions, as generated."""
    e = {
        "dmo": _expr(src, r"    dmo\[q\] = (.*);\n"),
        "r": _expr(src, r"    const unsigned int r = (.*);\n"),
        "voK": _expr(src, r"    voK\[q\] = (.*);\n"),
        "voV": _expr(src, r"    voV\[q\] = (.*);\n"),
        "kx": _expr(src, r"  const unsigned int kx = (.*);\n"),
        "vr": _expr(src, r"  const unsigned int vr = (.*?), vsw"),
        "vsw": _expr(src, r", vsw = (.*);\n"),
        "vcl": _expr(src, r"  const unsigned int vcl = (.*);\n"),
        "va": _expr(src, r"    va\[u\] = (.*);\n"),
        "kstep": _expr(src, r"voK\[\d\] \+ \(.*?\) \* (\d+)u"),
        "vstep": _expr(src, r"voV\[\d\] \+ \(.*?\) \* (\d+)u"),
    }
    return e


KREAD_RE = re.compile(r"const tj_bf16x8 kt(\d+) = \*\(const tj_bf16x8\*\)\(Ks(\d) \+ (.*?)\);")
VREAD_RE = re.compile(r"const tj_i16x4 vt(\d+)([ab]) = .*?\(Vs(\d) \+ (.*?)\)\);")
KMMA_RE = re.compile(r"(s[AB])\[0\]\[(\d)\] = __builtin_amdgcn_mfma_f32_32x32x16_bf16\(kt(\d+), qf\[0\]\[(\d)\], (s[AB])\[0\]\[(\d)\]")
VMMA_RE = re.compile(r"o\[0\]\[(\d)\] = __builtin_amdgcn_mfma_f32_32x32x16_bf16\(.*?shufflevector\(vt(\d+)a, vt(\d+)b, "
                     r"0, 1, 2, 3, 4, 5, 6, 7\)\), pf\[0\]\[(\d)\], o\[0\]\[(\d)\]")


def _block_reads(src: str):
    """One block's score and PV sections as generated: K fragment p's address expression
    and the MFMA that takes it (accumulator tile t, Q chunk c); Vᵀ fragment p's two
    address expressions and its MFMA (output tile u, probability chunk ch)."""
    blk = src.split("// block")[1]
    kreads = {int(p): e for p, _, e in KREAD_RE.findall(blk)}
    vreads = {}
    for p, h, _, e in VREAD_RE.findall(blk):
        vreads.setdefault(int(p), {})[h] = e
    kmma = {}
    for dst, t, p, c, src_acc, t2 in KMMA_RE.findall(blk):
        assert dst == src_acc and t == t2
        kmma[int(p)] = (int(t), int(c))
    vmma = {}
    for u, pa, pb, ch, u2 in VMMA_RE.findall(blk):
        assert pa == pb and u == u2
        vmma[int(pa)] = (int(u), int(ch))
    return kreads, kmma, vreads, vmma


def _dma_map(e: dict, which: str, kst: int):
    """LDS slot (16-byte index in a stage) -> (row, chunk) of the block, from both groups'
    DMA loads of one block (block 0: offsets relative to the block's first row)."""
    slots = {}
    for wave in range(8):
        for q in range(2):
            base = _c_eval(e["dmo"], dict(_lane_env(0, wave), q=q))
            assert base % 1024 == 0 and 0 <= base < BKV * 256
            for lane in range(64):
                env = dict(_lane_env(lane, wave), q=q)
                env["r"] = _c_eval(e["r"], env)
                off = _c_eval(e["voK" if which == "k" else "voV"], env)
                row, byte = divmod(off, kst * 2)
                assert byte % 16 == 0 and byte < 256
                slot = (base + 16 * lane) // 16
                assert slot not in slots, (which, wave, q, lane)
                slots[slot] = (row, byte // 16)
    assert sorted(slots) == list(range(BKV * 16))
    assert sorted(slots.values()) == [(r, c) for r in range(BKV) for c in range(16)]
    return slots


@pytest.mark.parametrize("layout", ["bhsd", "bshd"])
def test_dma_placement_and_fragment_reads_agree(layout):
    src, _ = _source(layout=layout)
    kst = 128 * (2 if layout == "bshd" else 1)
    e = _setup(src)
    assert int(e["kstep"]) == BKV * kst * 2 and int(e["vstep"]) == BKV * kst * 2
    kmap, vmap = _dma_map(e, "k", kst), _dma_map(e, "v", kst)
    kreads, kmma, vreads, vmma = _block_reads(src)
    # every score MFMA takes one K fragment read, every (tile, chunk) once; likewise PV
    assert sorted(kreads) == sorted(kmma) == list(range(16))
    assert sorted(kmma.values()) == [(t, c) for t in range(2) for c in range(8)]
    assert sorted(vreads) == sorted(vmma) == list(range(16))
    assert sorted(vmma.values()) == [(u, ch) for u in range(4) for ch in range(4)]
    for lane in range(64):
        env = _lane_env(lane, 0)
        for name in ("kx", "vr", "vsw", "vcl"):
            env[name] = _c_eval(e[name], env)
        env["va"] = [_c_eval(e["va"], dict(env, u=u)) for u in range(4)]
        g, col = lane // 32, lane % 32
        for p, expr in kreads.items():
            t, c = kmma[p]
            a = _c_eval(expr, env)
            assert a % 16 == 0
            assert kmap[a // 16] == (t * 32 + col, 2 * c + g), (lane, p, t, c)
        for p, pair in vreads.items():
            u, ch = vmma[p]
            for second, h in ((0, "a"), (1, "b")):
                a = _c_eval(pair[h], env)
                assert a % 8 == 0
                row, chunk = vmap[a // 16]
                vrow = ch * 16 + g * 4 + (lane % 16) // 4 + 8 * second
                vcol = u * 32 + ((lane // 16) % 2) * 16 + (lane % 4) * 4
                assert (row, chunk * 8 + ((a % 16) // 8) * 4) == (vrow, vcol), (lane, p, u, ch, second)


def test_fragment_reads_are_bank_conflict_free():
    src, _ = _source()
    e = _setup(src)
    envs = []
    for lane in range(64):
        env = _lane_env(lane, 0)
        for name in ("kx", "vr", "vsw", "vcl"):
            env[name] = _c_eval(e[name], env)
        env["va"] = [_c_eval(e["va"], dict(env, u=u)) for u in range(4)]
        envs.append(env)
    kreads, _, vreads, _ = _block_reads(src)
    for p, expr in kreads.items():
        a = [_c_eval(expr, env) for env in envs]
        # 16-byte reads: 32 lanes a pass over 512 bytes of banks, and the padded layout's
        # stronger property, 16 lanes over 256 bytes and 8 over 128 (a swizzle without it
        # measured 1.7e7 conflict cycles per [4,32,2048,128] launch, the padded rows 0)
        for lanes, groups in ((32, 32), (16, 16), (8, 8)):
            for h in range(64 // lanes):
                assert len({(x // 16) % groups for x in a[lanes * h:lanes * (h + 1)]}) == lanes, (p, lanes, h)
    for p, pair in vreads.items():
        for h, expr in pair.items():
            a = [_c_eval(expr, env) for env in envs]
            # transposing 8-byte reads: each half-wave over 256 bytes of banks (the model the
            # measured conflict counts fit), and the whole wave over 512 bytes
            for half in (0, 1):
                assert len({(x // 8) % 32 for x in a[32 * half:32 * half + 32]}) == 32, (p, h, half)
            assert len({(x // 8) % 64 for x in a}) == 64, (p, h)


# ---------------------------------------------------------------------------
# the schedule, expanded from the source and run for both wave groups
# ---------------------------------------------------------------------------

DMA_RE = re.compile(r"raw_ptr_buffer_load_lds\(rs([KV]), .*?\(([KV])s(\d) \+ dmo\[(\d)\]\), 16, vo[KV]\[\d\] \+ \((.*?)\) \* \d+u")
WAIT_RE = re.compile(r"__builtin_amdgcn_s_waitcnt\((0x[0-9a-f]+)\)")
LOOP_RE = re.compile(r"for \(unsigned int jj = 0; jj < (\d+)u; jj \+= 4u\) \{")


def _body_lines(src: str) -> list[str]:
    start = src.index("wv = __builtin_amdgcn_readfirstlane")
    end = src.index("const float l_tot", start)
    return [x.strip() for x in src[start:end].splitlines()]


def _expand(lines: list[str]) -> list[tuple]:
    """Flatten the body into (kind, payload, group-or-None, block-context) events."""
    out = []
    i, cur_j, only = 0, None, None
    while i < len(lines):
        ln = lines[i]
        m = LOOP_RE.match(ln)
        if m:
            depth, k = 1, i + 1
            while depth:
                depth += lines[k].count("{") - lines[k].count("}")
                k += 1
            body = lines[i + 1:k - 1]
            for jj in range(0, int(m.group(1)), 4):
                out += _expand_block(body, {"jj": jj}, only)
            i = k
            continue
        out += _expand_block([ln], {}, only, cur_j)
        mb = re.match(r"\{  // block (\d+)", ln)
        if mb:
            cur_j = int(mb.group(1))
            out.append(("ctx", cur_j, None, None))
        mg = re.match(r"if \(gq == (\d)u\) \{", ln)
        if mg:
            only = int(mg.group(1))
        elif ln == "}" and only is not None:
            only = None
        i += 1
    return out


def _expand_block(lines, env, only, cur_j=None):
    out = []
    for ln in lines:
        mj = re.match(r"const unsigned int (j\d) = jj \+ (\d)u;", ln)
        if mj:
            env = dict(env, **{mj.group(1): env["jj"] + int(mj.group(2))})
            out.append(("ctx", env[mj.group(1)], None, None))
            continue
        m = DMA_RE.search(ln)
        if m:
            assert m.group(1) == m.group(2)
            blk = _c_eval(m.group(5), env)
            out.append(("dma", (m.group(1), int(m.group(3)), int(m.group(4)), blk), only, None))
            continue
        m = WAIT_RE.search(ln)
        if m:
            imm = int(m.group(1), 16)
            out.append(("wait", ((imm & 15) | (((imm >> 14) & 3) << 4), (imm >> 8) & 15), only, None))
            continue
        if "__builtin_amdgcn_s_barrier()" in ln:
            out.append(("barrier", None, only, None))
            continue
        assert "__syncthreads" not in ln
        mk = KREAD_RE.search(ln)
        if mk:
            out.append(("read", ("K", int(mk.group(2))), only, None))
        mv = VREAD_RE.search(ln)
        if mv:
            out.append(("read", ("V", int(mv.group(3))), only, None))
    return out


def _run_group(events, gq: int):
    """One group's trace: DMA loads (op, stage, block, issue interval, visible-from
    interval) and reads (op, stage, expected block, interval)."""
    interval, cur_j = 0, None
    dmas, reads = [], []
    for kind, pay, only, _ in events:
        if only is not None and only != gq:
            continue
        if kind == "ctx":
            cur_j = pay
        elif kind == "dma":
            op, st, q, blk = pay
            if q == 0:
                dmas.append({"op": op, "stage": st, "block": blk, "issued": interval, "visible": None, "n": 0})
            dmas[-1]["n"] += 1
        elif kind == "wait":
            vm, lgkm = pay
            # vmcnt counts this wave's instructions (two per block half); they land in order
            insts = [d for d in dmas for _ in range(d["n"])]
            for d_i, d in enumerate(dmas):
                last = sum(x["n"] for x in dmas[:d_i + 1])
                if d["visible"] is None and len(insts) - last >= vm:
                    d["visible"] = interval + 1
        elif kind == "barrier":
            interval += 1
        elif kind == "read":
            op, st = pay
            want = (0 if cur_j is None else cur_j + 1) if op == "K" else cur_j
            reads.append({"op": op, "stage": st, "block": want, "at": interval})
    return dmas, reads, interval


@pytest.mark.parametrize("mi16", [False, True])
@pytest.mark.parametrize("Sk", [64, 128, 192, 256, 320, 448, 512, 576, 640, 704, 960, 1024, 1100, 2048, 2000])
def test_schedule_reads_only_published_blocks(Sk, mi16):
    src, _ = _source(Sk=Sk, mi16=mi16)
    lines = _body_lines(src)
    # every barrier is preceded by a wait that includes lgkmcnt(0): a group's fragment
    # reads are done before the barrier after which the other group may overwrite them
    for i, ln in enumerate(lines):
        if "__builtin_amdgcn_s_barrier()" in ln:
            prev = [x for x in lines[:i] if "s_waitcnt" in x][-1]
            assert (int(WAIT_RE.search(prev).group(1), 16) >> 8) & 15 == 0
    events = _expand(lines)
    KB = -(-Sk // BKV)
    traces = [_run_group(events, gq) for gq in (0, 1)]
    assert traces[0][2] == traces[1][2], "both groups pass the same number of barriers"
    for gq in (0, 1):
        dmas = traces[gq][0]
        assert all(d["visible"] is not None for d in dmas), "every DMA load is waited for"
        assert all(d["n"] == 2 for d in dmas)
        for op in ("K", "V"):
            assert sorted(d["block"] for d in dmas if d["op"] == op) == list(range(KB))
            assert all(d["stage"] == d["block"] % 4 for d in dmas if d["op"] == op)
    nread = 0
    for gq in (0, 1):
        for r in traces[gq][1]:
            if r["op"] == "K" and r["block"] >= KB:
                raise AssertionError(f"S({r['block']}) read past the last block")
            for h in (0, 1):
                cands = [d for d in traces[h][0] if d["op"] == r["op"] and d["stage"] == r["stage"]]
                before = [d for d in cands if d["issued"] < r["at"]]
                assert before, (gq, r)
                src_d = before[-1]
                assert src_d["block"] == r["block"], (gq, h, r, src_d)
                assert src_d["visible"] <= r["at"], (gq, h, r, src_d)
                assert not [d for d in cands if d["issued"] == r["at"]], ("overwritten while read", gq, h, r)
            nread += 1
    # group 0 reads K of blocks 0..KB-1 and V of blocks 0..KB-1, as group 1 does
    for gq in (0, 1):
        got = sorted({(r["op"], r["block"]) for r in traces[gq][1]})
        assert got == sorted([("K", b) for b in range(KB)] + [("V", b) for b in range(KB)])
    assert nread


def test_planted_schedule_mistake_is_caught():
    """A wait that lets one more DMA load stay in flight at the end of a block's first
    phase publishes a block before it has landed: the simulation must flag it."""
    src, _ = _source(Sk=1024)
    lines = _body_lines(src)
    i = next(i for i, ln in enumerate(lines) if "s_waitcnt(0x74)" in ln)
    lines[i] = lines[i].replace("0x74", "0x76")
    events = _expand(lines)
    traces = [_run_group(events, gq) for gq in (0, 1)]
    bad = False
    for gq in (0, 1):
        for r in traces[gq][1]:
            for h in (0, 1):
                cands = [d for d in traces[h][0] if d["op"] == r["op"] and d["stage"] == r["stage"]]
                before = [d for d in cands if d["issued"] < r["at"]]
                if not before or before[-1]["block"] != r["block"] or before[-1]["visible"] is None \
                        or before[-1]["visible"] > r["at"]:
                    bad = True
    assert bad


def test_dma_schedule_only_for_head_dim_128(monkeypatch):
    fn = lambda q, k, v: tj.matmul(tj.softmax(tj.matmul(q, tj.transpose(k, -1, -2)) * 0.125), v)  # noqa: E731
    p = fuse_attention(C.lower(tj.trace(fn, [TensorType((1, 2, 1024, 64), DType.bf16)] * 3), "hip"))
    _, launches = hb.generate(p)
    assert launches[0].meta["schedule"] == "pingpong"
    monkeypatch.setenv("TENSORJIT_HIP_ATTENTION_DMA", "0")
    p = fuse_attention(C.lower(tj.trace(fn, [TensorType((1, 2, 1024, 128), DType.bf16)] * 3), "hip"))
    _, launches = hb.generate(p)
    assert launches[0].meta["schedule"] == "pingpong"


# ---------------------------------------------------------------------------
# the 16x16x32 form: same DMA schedule, K layout kept, V stored with its own swizzle
# ---------------------------------------------------------------------------

KMMA16_RE = re.compile(r"(s[AB])\[(\d)\]\[(\d)\] = __builtin_amdgcn_mfma_f32_16x16x32_bf16\(kt(\d+), qf\[(\d)\]\[(\d)\], "
                       r"(s[AB])\[(\d)\]\[(\d)\]")
VVEC16_RE = re.compile(r"const tj_bf16x8 vv(\d+) = .*?shufflevector\(vt(\d+)a, vt(\d+)b, 0, 1, 2, 3, 4, 5, 6, 7\)\);")
VMMA16_RE = re.compile(r"o\[(\d)\]\[(\d)\] = __builtin_amdgcn_mfma_f32_16x16x32_bf16\(vv(\d+), pf\[(\d)\]\[(\d)\], "
                       r"o\[(\d)\]\[(\d)\]")


def _setup16(src: str) -> dict:
    return {
        "dmo": _expr(src, r"    dmo\[q\] = (.*);\n"),
        "r": _expr(src, r"    const unsigned int r = (.*);\n"),
        "voK": _expr(src, r"    voK\[q\] = (.*);\n"),
        "voV": _expr(src, r"    voV\[q\] = (.*);\n"),
        "kx16": _expr(src, r"  const unsigned int kx16 = (.*);\n"),
        "vr16": _expr(src, r"  const unsigned int vr16 = (.*?), vh16"),
        "vh16": _expr(src, r", vh16 = (.*);\n"),
        "va16": _expr(src, r"    va16\[u\] = (.*);\n"),
    }


def _lane_env16(lane: int, e: dict) -> dict:
    env = dict(_lane_env(lane, 0), r16=lane % 16, g16=lane // 16)
    for name in ("kx16", "vr16", "vh16"):
        env[name] = _c_eval(e[name], env)
    env["va16"] = [_c_eval(e["va16"], dict(env, u=u)) for u in range(8)]
    return env


def _block_reads16(src: str):
    """K fragment p -> (key tile t, d chunk c), each feeding the MFMAs of both query tiles
    h = 0, 1 into S[h][t]; Vᵀ fragment p -> (dv tile u, key chunk ch), each feeding
    O[h][u] of both query tiles with P chunk pf[h][ch]."""
    blk = src.split("// block")[1]
    kreads = {int(p): e for p, _, e in KREAD_RE.findall(blk)}
    vreads = {}
    for p, h, _, e in VREAD_RE.findall(blk):
        vreads.setdefault(int(p), {})[h] = e
    kmma = {}
    for dst, h, t, p, hq, c, dst2, h2, t2 in KMMA16_RE.findall(blk):
        assert dst == dst2 and h == hq == h2 and t == t2
        kmma.setdefault(int(p), set()).add((int(h), int(t), int(c)))
    vvec = {int(v): int(a) for v, a, b in VVEC16_RE.findall(blk) if a == b}
    vmma = {}
    for h, u, v, hp, ch, h2, u2 in VMMA16_RE.findall(blk):
        assert h == hp == h2 and u == u2
        vmma.setdefault(vvec[int(v)], set()).add((int(h), int(u), int(ch)))
    return kreads, kmma, vreads, vmma


@pytest.mark.parametrize("layout", ["bhsd", "bshd"])
def test_dma16_placement_and_fragment_reads_agree(layout):
    """The 16x16x32 form reads, per lane, the K row and chunk of its MFMA A operand (key
    16t + lane % 16, d 32c + 8 (lane / 16) .. +7) and, per transposing read, the 8 bytes
    whose 16-lane transpose gives lane i of group g the keys 32ch + 16s + 4g + 0..3 of
    dv 16u + i -- the k order of the lane's own probabilities S[h][2ch + s][0..3]."""
    src, _ = _source(layout=layout, mi16=True)
    kst = 128 * (2 if layout == "bshd" else 1)
    e = _setup16(src)
    kmap, vmap = _dma_map(e, "k", kst), _dma_map(e, "v", kst)
    kreads, kmma, vreads, vmma = _block_reads16(src)
    assert sorted(kreads) == sorted(kmma) == list(range(16))
    assert all(len({(t, c) for _, t, c in v}) == 1 and {h for h, _, _ in v} == {0, 1} for v in kmma.values())
    assert sorted({(t, c) for v in kmma.values() for _, t, c in v}) == [(t, c) for t in range(4) for c in range(4)]
    assert sorted(vreads) == sorted(vmma) == list(range(16))
    assert all(len({(u, ch) for _, u, ch in v}) == 1 and {h for h, _, _ in v} == {0, 1} for v in vmma.values())
    assert sorted({(u, ch) for v in vmma.values() for _, u, ch in v}) == [(u, ch) for u in range(8) for ch in range(2)]
    for lane in range(64):
        env = _lane_env16(lane, e)
        g16, r16 = lane // 16, lane % 16
        for p, expr in kreads.items():
            (_, t, c), = {(0, t, c) for _, t, c in kmma[p]}
            a = _c_eval(expr, env)
            assert a % 16 == 0 and a < BKV * 256
            assert kmap[a // 16] == (16 * t + r16, 4 * c + g16), (lane, p, t, c)
        for p, pair in vreads.items():
            (_, u, ch), = {(0, u, ch) for _, u, ch in vmma[p]}
            for s, h in ((0, "a"), (1, "b")):
                a = _c_eval(pair[h], env)
                assert a % 8 == 0 and a + 8 <= BKV * 256
                row, chunk = vmap[a // 16]
                want = (32 * ch + 16 * s + 4 * g16 + (lane % 16) // 4, 16 * u + (lane % 4) * 4)
                assert (row, chunk * 8 + ((a % 16) // 8) * 4) == want, (lane, p, u, ch, s)


def test_dma16_fragment_reads_are_bank_conflict_free():
    src, _ = _source(mi16=True)
    e = _setup16(src)
    envs = [_lane_env16(lane, e) for lane in range(64)]
    kreads, _, vreads, _ = _block_reads16(src)
    for p, expr in kreads.items():
        a = [_c_eval(expr, env) for env in envs]
        for lanes, groups in ((32, 32), (16, 16), (8, 8)):
            for h in range(64 // lanes):
                assert len({(x // 16) % groups for x in a[lanes * h:lanes * (h + 1)]}) == lanes, (p, lanes, h)
    for p, pair in vreads.items():
        for h, expr in pair.items():
            a = [_c_eval(expr, env) for env in envs]
            for half in (0, 1):
                assert len({(x // 8) % 32 for x in a[32 * half:32 * half + 32]}) == 32, (p, h, half)
            assert len({(x // 8) % 64 for x in a}) == 64, (p, h)


def test_dma16_planted_v_swizzle_mistake_is_caught():
    """The padded-row-era V swizzle of the 32x32x16 form, planted into the 16x16x32 form's
    DMA, leaves the reads pointing at other rows: the placement check must fail."""
    src, _ = _source(mi16=True)
    e = _setup16(src)
    e["voV"] = e["voV"].replace("((((r & 7u) ^ ((r >> 3) & 1u))) << 1)", "(((r ^ (r >> 2)) & 3u) << 2)")
    vmap = _dma_map(e, "v", 128)
    _, _, vreads, vmma = _block_reads16(src)
    bad = 0
    for lane in range(64):
        env = _lane_env16(lane, e)
        for p, pair in vreads.items():
            (_, u, ch), = {(0, u, ch) for _, u, ch in vmma[p]}
            a = _c_eval(pair["a"], env)
            row, chunk = vmap[a // 16]
            bad += (row, chunk * 8 + ((a % 16) // 8) * 4) != (32 * ch + 4 * (lane // 16) + (lane % 16) // 4,
                                                               16 * u + (lane % 4) * 4)
    assert bad


def test_two_16x16x32_attention_kernels_compile_in_one_module(monkeypatch):
    """The quad-lane helpers the 16x16x32 form adds are guarded, so a program with two
    such attention kernels is one valid hipRTC module."""
    monkeypatch.setenv("TENSORJIT_HIP_ATTENTION_MI16", "1")

    def two(q, k, v):
        a = tj.matmul(tj.softmax(tj.matmul(q, tj.transpose(k, -1, -2)) * 0.088), v)
        return tj.matmul(tj.softmax(tj.matmul(a, tj.transpose(k, -1, -2)) * 0.088), v)

    p = fuse_attention(C.lower(tj.trace(two, [TensorType((1, 2, 1024, 128), DType.bf16)] * 3), "hip"))
    src, launches = hb.generate(p)
    assert [ln.meta["mfma"] for ln in launches] == ["16x16x32", "16x16x32"]
    assert hb.compile_source(src, "gfx950")
