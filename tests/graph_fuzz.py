"""Seeded random tensorjit programs for the hip backend's generator tests.

``program(seed)`` returns ``(fn, shapes)``: a function on ``tj`` tensors built from a
random mix of the ops the fusion passes turn into the four kernel families --
pointwise chains with broadcasting, last-axis and non-last-axis reductions (kept and
dropped dims), softmax / LayerNorm / RMSNorm rows, linear layers with and without
bias, batched products, transposes and reshapes -- with one or two outputs.  Every
op takes inputs in its domain (logs and roots of ``|v| + 1``, exponents of bounded
values), so the programs are finite and the oracle's float32 results are
well-conditioned.  ``attention_program``, ``layer_program``, ``broadcast_program``,
``block_program``, ``reduction_program``, ``wide_row_program`` and ``column_program``
draw attention cores, pre-norm residual layers, 3-D / 4-D broadcast-and-permute programs,
transformer stacks, reductions over few long rows, row-op chains over wide rows and
reductions over a non-last axis the same way;
``transpose_case`` draws permutes for the tiled copy.  The same seed always gives the same
program.
"""
from __future__ import annotations

import random

import tensorjit as tj

UNARY = ["exp_tanh", "log1p_abs", "sqrt1p_abs", "rsqrt1p_abs", "tanh", "abs", "relu", "sigmoid", "gelu", "silu",
         "neg"]
BINARY = ["add", "sub", "mul", "div_safe", "maximum", "minimum", "where"]


def _unary(op: str, v):
    if op == "exp_tanh":
        return tj.exp(tj.tanh(v))
    if op == "log1p_abs":
        return tj.log(tj.abs(v) + 1.0)
    if op == "sqrt1p_abs":
        return tj.sqrt(tj.abs(v) + 1.0)
    if op == "rsqrt1p_abs":
        return tj.rsqrt(tj.abs(v) + 1.0)
    if op == "neg":
        return -v
    return getattr(tj, op)(v)


def _binary(op: str, a, b):
    if op == "add":
        return a + b
    if op == "sub":
        return a - b
    if op == "mul":
        return a * b
    if op == "div_safe":
        return a / (tj.abs(b) + 1.0)
    if op == "where":
        return tj.where(a, b, a * 0.5)
    return getattr(tj, op)(a, b)


def program(seed: int):
    """(fn, input shapes) of random program ``seed``."""
    rng = random.Random(seed)
    R = rng.choice([1, 3, 16, 37, 64, 130])
    N = rng.choice([1, 5, 16, 64, 100, 128, 260])
    N2 = rng.choice([8, 32, 96, 128])
    batched = rng.random() < 0.25
    B = rng.choice([2, 3]) if batched else None
    xs = (B, R, N) if batched else (R, N)
    shapes = [xs, (N,) if rng.random() < 0.5 else xs, (N2, N), (N2,)]
    steps = [rng.random() for _ in range(rng.randint(2, 7))]
    choices = [rng.randrange(1 << 30) for _ in range(64)]

    def fn(x, y, w, b):
        c = iter(choices)

        def pick(seq):
            return seq[next(c) % len(seq)]

        vals = [x, x * 0.5 + y]
        for u in steps:
            v = pick(vals)
            if u < 0.30:
                vals.append(_unary(pick(UNARY), v))
            elif u < 0.55:
                same = [t for t in vals if t.shape == v.shape or t.shape == v.shape[-1:]]
                vals.append(_binary(pick(BINARY), v, pick(same)))
            elif u < 0.65:
                red = pick(["sum", "mean", "max"])
                r = getattr(tj, red)(v, axis=-1, keepdim=True)
                vals.append(v - r if red != "sum" else v * tj.rsqrt(tj.abs(r) + 1.0))
            elif u < 0.72:
                vals.append(pick([tj.softmax, tj.rms_norm, tj.layer_norm])(v))
            elif u < 0.84 and v.shape[-1] == N:
                h = tj.linear(v, w, b) if next(c) % 2 else tj.linear(v, w)
                vals.append(pick([tj.relu, tj.gelu, tj.tanh])(h))
            elif u < 0.90 and len(v.shape) >= 2:
                # a transpose through the pointwise / copy family and back
                t = tj.transpose(v, -1, -2)
                vals.append(tj.transpose(_unary(pick(UNARY), t), -1, -2))
            elif u < 0.95 and len(v.shape) >= 2:
                # reduce over the leading axis (moved last by a transpose), broadcast back
                vals.append(v + tj.mean(v, axis=0))
            else:
                flat = 1
                for d in v.shape:
                    flat *= d
                vals.append(tj.reshape(tj.reshape(v, flat), *v.shape) * 2.0)
        outs = [vals[-1]]
        if next(c) % 3 == 0 and vals[-2] is not vals[-1] and vals[-2] is not x:
            outs.append(vals[-2])
        return tuple(outs) if len(outs) > 1 else outs[0]

    return fn, shapes


def attention_program(seed: int):
    """(fn, shapes) of a random attention core ``softmax(q kᵀ · s) v``: batch and head
    dims, query / key lengths (ragged against the 64-key blocks and the 32-query
    tiles), head dims 16-128 for q/k and 32-128 for v, and the scale written as a
    multiply on either side or as a division."""
    rng = random.Random(seed)
    lead = rng.choice([(1,), (2,), (2, 3), (1, 4)])
    sq, sk = rng.choice([1, 31, 64, 200, 513]), rng.choice([1, 40, 64, 130, 700])
    d, dv = rng.choice([16, 32, 64, 128]), rng.choice([32, 64, 128])
    form = rng.choice(["mul", "lmul", "div", "none"])
    c = rng.choice([0.05, 0.125, 0.3])

    scale = {"mul": lambda t: t * c, "lmul": lambda t: c * t, "div": lambda t: t / (1.0 / c),
             "none": lambda t: t}[form]

    def fn(q, k, v):
        return tj.matmul(tj.softmax(scale(tj.matmul(q, tj.transpose(k, -1, -2)))), v)

    fn.scores = scale       # the same scaling, for references that evaluate the scores themselves
    return fn, [(*lead, sq, d), (*lead, sk, d), (*lead, sk, dv)]


def layer_program(seed: int):
    """(fn, shapes) of a random pre-norm residual layer: RMSNorm or LayerNorm, a linear
    (with or without bias) and an activation, a residual, a second norm and a second
    linear whose residual the plan leaves as a kernel of its own."""
    rng = random.Random(seed)
    B = rng.choice([(), (2,)])
    S, D, F = rng.choice([16, 100, 256]), rng.choice([64, 128, 256]), rng.choice([64, 192, 512])
    norm1, norm2 = rng.choice([tj.rms_norm, tj.layer_norm]), rng.choice([tj.rms_norm, tj.layer_norm])
    act = rng.choice([tj.gelu, tj.relu, tj.silu])
    bias = rng.random() < 0.5

    def fn(x, g1, w1, b1, w2, g2, w3):
        h = x + (tj.linear(norm1(x, g1), w1, b1) if bias else tj.linear(norm1(x, g1), w1))
        return h + tj.linear(act(tj.linear(norm2(h, g2), w2)), w3)

    return fn, [(*B, S, D), (D,), (D, D), (D,), (F, D), (D,), (D, F)]


def broadcast_program(seed: int):
    """(fn, shapes) of a random 3-D / 4-D pointwise and reduction program over inputs with
    size-1 (broadcast) dims, with permutes of inner and outer dims, last- and
    middle-axis reductions and a row op over the last axis."""
    rng = random.Random(seed)
    dims = [rng.choice([1, 2, 3, 7]), rng.choice([1, 4, 33]), rng.choice([1, 16, 65]), rng.choice([8, 64, 96, 257])]
    if rng.random() < 0.4:
        dims = dims[1:]
    full = tuple(dims)
    # the second input: the same shape with some dims set to 1, possibly fewer leading dims
    bshape = tuple(1 if rng.random() < 0.4 else d for d in full)[rng.randint(0, 1):]
    steps = [rng.random() for _ in range(rng.randint(2, 6))]
    choices = [rng.randrange(1 << 30) for _ in range(64)]

    def fn(x, y):
        c = iter(choices)

        def pick(seq):
            return seq[next(c) % len(seq)]

        v = x * 0.5 + y
        for u in steps:
            if u < 0.3:
                # the broadcast input only in arithmetic: a clamp or select against a
                # per-row constant can leave rows of nearly equal values, which a later
                # norm's centring turns into rounding noise (ill-conditioned in bf16)
                op = pick(BINARY)
                v = _binary(op, v, pick([x, y, v] if op in ("add", "sub", "mul", "div_safe") else [x, v]))
            elif u < 0.5:
                v = _unary(pick(UNARY), v)
            elif u < 0.65:
                # permute two dims and back: a copy kernel each way around a pointwise op
                a, b = sorted(rng_pair(next(c), v.ndim))
                v = tj.transpose(_unary(pick(UNARY), tj.transpose(v, a, b)), a, b)
            elif u < 0.8:
                axis = next(c) % v.ndim
                if axis == v.ndim - 1:
                    v = v - tj.max(v, axis=-1, keepdim=True)
                else:
                    # a non-last axis reduction moves that axis last and keeps it there:
                    # broadcast it back over v with the axis moved last, then restore the order
                    order = [d for d in range(v.ndim) if d != axis] + [axis]
                    back = [order.index(d) for d in range(v.ndim)]
                    t = tj.permute(v, *order) + tj.sum(v, axis=axis, keepdim=True) * 0.1
                    v = tj.permute(t, *back)
            else:
                v = pick([tj.softmax, tj.rms_norm, tj.layer_norm])(v)
        return v

    return fn, [full, bshape]


def rng_pair(r: int, n: int) -> tuple[int, int]:
    """Two distinct axes of an n-dim value, from one random integer."""
    a = r % n
    b = (a + 1 + (r // n) % (n - 1)) % n
    return a, b


def block_program(seed: int):
    """(fn, shapes, scales) of a random stack of one or two pre-norm transformer blocks
    sharing one set of weights: multi-head attention (head split and merge by reshape
    and transpose, scale 1/sqrt(d) as a multiply or a division) with a residual, then a
    norm, an MLP (with or without biases, gelu / silu / relu) and a residual.  ``scales``
    multiplies each standard-normal input: weights by 1/sqrt(fan-in), biases by 0.1, so
    the activations keep unit size and the scores stay well-conditioned."""
    rng = random.Random(seed)
    B, S = rng.choice([1, 2]), rng.choice([64, 100, 256])
    heads, d = rng.choice([(2, 32), (4, 32), (2, 64), (1, 128)])
    Dm = heads * d
    F = rng.choice([128, 192, 384])
    layers = rng.choice([1, 2])
    norm1, norm2 = rng.choice([tj.rms_norm, tj.layer_norm]), rng.choice([tj.rms_norm, tj.layer_norm])
    act = rng.choice([tj.gelu, tj.silu, tj.relu])
    bias = rng.random() < 0.5
    div = rng.random() < 0.5

    def fn(x, g1, wq, wk, wv, wo, g2, w1, b1, w2, b2):
        def split(t):
            return tj.transpose(tj.reshape(t, B, S, heads, d), 1, 2)

        for _ in range(layers):
            h = norm1(x, g1)
            q, k, v = split(tj.linear(h, wq)), split(tj.linear(h, wk)), split(tj.linear(h, wv))
            s = tj.matmul(q, tj.transpose(k, -1, -2))
            s = s / (d ** 0.5) if div else s * (1.0 / d ** 0.5)
            o = tj.reshape(tj.transpose(tj.matmul(tj.softmax(s), v), 1, 2), B, S, Dm)
            x = x + tj.linear(o, wo)
            h = norm2(x, g2)
            u = act(tj.linear(h, w1, b1) if bias else tj.linear(h, w1))
            x = x + (tj.linear(u, w2, b2) if bias else tj.linear(u, w2))
        return x

    shapes = [(B, S, Dm), (Dm,), (Dm, Dm), (Dm, Dm), (Dm, Dm), (Dm, Dm), (Dm,), (F, Dm), (F,), (Dm, F), (Dm,)]
    w, wf = Dm ** -0.5, F ** -0.5
    return fn, shapes, [1.0, 1.0, w, w, w, w, 1.0, w, 0.1, wf, 0.1]


def reduction_program(seed: int):
    """(fn, shapes) of a random reduction over few long rows (1-16 rows of 262144-524288
    elements, some lengths odd): a pointwise prologue on one or two inputs (the second
    the same shape or broadcast over the rows), sum / mean / max over the last axis with
    or without keepdim, and a per-row epilogue of zero to two ops."""
    rng = random.Random(seed)
    R = rng.choice([1, 2, 3, 7, 16])
    N = rng.choice([262144, 300000, 400003, 524288])
    xs = (R, N) if R > 1 or rng.random() < 0.5 else (N,)
    ys = xs if rng.random() < 0.5 else (N,)
    steps = [rng.random() for _ in range(rng.randint(0, 3))]
    red = rng.choice(["sum", "mean", "max"])
    keep = rng.random() < 0.5
    epi = rng.randint(0, 2)
    choices = [rng.randrange(1 << 30) for _ in range(32)]

    def fn(x, y):
        c = iter(choices)

        def pick(seq):
            return seq[next(c) % len(seq)]

        v = x
        for u in steps:
            v = _unary(pick(UNARY), v) if u < 0.5 else _binary(pick(["add", "sub", "mul", "div_safe", "maximum"]), v, y)
        r = getattr(tj, red)(v, axis=-1, keepdim=keep)
        for _ in range(epi):
            r = pick([lambda t: t * 0.5 + 1.0, lambda t: tj.sqrt(tj.abs(t) + 1.0), tj.tanh, lambda t: -t])(r)
        return r

    return fn, [xs, ys]


def transpose_case(seed: int):
    """(shape, perm) of a random 2-4 dim permute whose output's innermost dim is strided in
    the source, with both innermost dims multiples of 8 (16-byte rows for every dtype up
    to 4 bytes) and ragged against the 64-element tiles."""
    rng = random.Random(seed)
    while True:
        nd = rng.choice([2, 3, 4])
        shape = [rng.choice([1, 2, 3, 5]) for _ in range(nd)]
        perm = list(range(nd))
        rng.shuffle(perm)
        if perm[-1] == nd - 1:
            continue
        for d in (perm[-1], nd - 1):
            shape[d] = 8 * rng.choice([1, 3, 8, 9, 16, 33])
        return tuple(shape), tuple(perm)


def wide_row_program(seed: int):
    """(fn, shapes) of a random chain of row ops over wide rows (4097-32768 elements, odd
    lengths among them; 1-64 rows): softmax / LayerNorm / RMSNorm (with a gain or not),
    pointwise ops with a second input of the same shape or broadcast over the rows, and
    row maxima or means broadcast back, which row fusion keeps in one row kernel."""
    rng = random.Random(seed)
    R = rng.choice([1, 3, 16, 64])
    N = rng.choice([4097, 8193, 12288, 16383, 24576, 32768])
    ys = (R, N) if rng.random() < 0.5 else (N,)
    steps = [rng.random() for _ in range(rng.randint(2, 5))]
    choices = [rng.randrange(1 << 30) for _ in range(32)]

    def fn(x, y, g):
        c = iter(choices)

        def pick(seq):
            return seq[next(c) % len(seq)]

        v = x
        for u in steps:
            if u < 0.35:
                op = pick(["softmax", "layer_norm", "rms_norm", "layer_norm_g", "rms_norm_g"])
                v = {"softmax": tj.softmax, "layer_norm": tj.layer_norm, "rms_norm": tj.rms_norm,
                     "layer_norm_g": lambda t: tj.layer_norm(t, g), "rms_norm_g": lambda t: tj.rms_norm(t, g)}[op](v)
            elif u < 0.6:
                v = _unary(pick(["tanh", "gelu", "silu", "exp_tanh", "sigmoid"]), v)
            elif u < 0.8:
                v = _binary(pick(["add", "sub", "mul"]), v, y)
            elif u < 0.9:
                v = v - tj.max(v, axis=-1, keepdim=True)
            else:
                v = v * tj.rsqrt(tj.mean(v * v, axis=-1, keepdim=True) + 1.0)
        return v

    return fn, [(R, N), ys, (N,)]


def column_program(seed: int):
    """(fn, shapes) of a random reduction over a non-last axis of a 2-4 dim tensor whose
    inner dims span at least 256 elements: an elementwise prologue on one or two inputs
    (the second full-shape or broadcast), sum / mean / max with or without keepdim, at
    times a second reduction of the same axis, and an epilogue that may read an input of
    the output's shape."""
    rng = random.Random(seed)
    nd = rng.choice([2, 3, 4])
    axis = rng.randrange(nd - 1)
    shape = [rng.choice([1, 2, 3, 5]) for _ in range(nd)]
    shape[axis] = rng.choice([7, 64, 300, 1000, 4096])
    shape[-1] = rng.choice([256, 260, 301, 512, 1024, 1032])
    full = tuple(shape)
    ys = full if rng.random() < 0.5 else full[-1:]
    out = tuple(d for i, d in enumerate(full) if i != axis)
    steps = [rng.random() for _ in range(rng.randint(0, 2))]
    red = rng.choice(["sum", "mean", "max"])
    keep = rng.random() < 0.4
    second = rng.random() < 0.3
    epi = rng.random() < 0.5 and not keep
    choices = [rng.randrange(1 << 30) for _ in range(16)]

    def fn(x, y, g):
        c = iter(choices)

        def pick(seq):
            return seq[next(c) % len(seq)]

        v = x
        for u in steps:
            v = _unary(pick(["tanh", "abs", "exp_tanh", "sigmoid"]), v) if u < 0.5 else \
                _binary(pick(["add", "mul", "sub"]), v, y)
        r = getattr(tj, red)(v, axis=axis, keepdim=keep)
        if epi:
            r = tj.tanh(r) * g + 0.5
        if second:
            return r, tj.max(v, axis=axis, keepdim=keep) if red != "max" else tj.mean(v, axis=axis, keepdim=keep)
        return r

    return fn, [full, ys, out]
