"""Pins the CPU oracle (oracle/c_backend.py, the restated reference `c` backend).

The reference ships no golden vectors; its own tests compare every backend with
eager PyTorch on seeded inputs (tests/test_backends.py:37-206).  Here the oracle is
checked the same way, against float64 closed forms, plus the published A&S 7.1.26
error bound of its erf and brute-force sums on tiny matmuls, so a dropped term,
a wrong sign or a transposed operand in the oracle fails one of these checks.
"""
import math

import pytest
import torch
import torch.nn.functional as F

import oracle
import tensorjit as tj


def _close(a, b, tol=1e-4):
    torch.testing.assert_close(a.float(), b.float(), atol=tol, rtol=tol)


def test_oracle_erf_within_published_bound():
    # A&S 7.1.26: |erf(x) - approx| <= 1.5e-7; the fp32 evaluation of 0.5*x*(1+erf)
    # adds a few ulp of 1.0 (2^-23 each), so the bound checked is 1.5e-7 + 6 ulp.
    xs = torch.linspace(-6, 6, 4001)
    (y,) = oracle.run(lambda x: tj.gelu(x), xs)
    ref = torch.tensor([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in xs.double().tolist()], dtype=torch.float64)
    err = (y.double() - ref).abs() / (0.5 * xs.double().abs()).clamp_min(1e-30)
    assert float(err.max()) < 1.5e-7 + 6 * 2.0**-23


@pytest.mark.parametrize("shape", [(17,), (8, 33), (2, 3, 5)])
def test_oracle_elementwise_chain(shape):
    torch.manual_seed(0)
    x, y = torch.randn(*shape), torch.randn(shape[-1])
    (out,) = oracle.run(lambda a, b: tj.exp(tj.relu(a * 2.0 + b)) / (1.0 + tj.sigmoid(a)) - tj.tanh(b), x, y)
    xd, yd = x.double(), y.double()
    _close(out, torch.exp(torch.relu(xd * 2 + yd)) / (1 + torch.sigmoid(xd)) - torch.tanh(yd))


@pytest.mark.parametrize("op", ["gelu", "silu", "log", "sqrt", "rsqrt", "abs", "sigmoid", "exp", "tanh", "relu"])
def test_oracle_unary_ops(op):
    torch.manual_seed(0)
    x = torch.rand(64) + 0.5
    (out,) = oracle.run(getattr(tj, op), x)
    ref = {"gelu": F.gelu, "silu": F.silu, "log": torch.log, "sqrt": torch.sqrt, "rsqrt": torch.rsqrt,
           "abs": torch.abs, "sigmoid": torch.sigmoid, "exp": torch.exp, "tanh": torch.tanh,
           "relu": torch.relu}[op](x.double())
    _close(out, ref, tol=2e-4)


def test_oracle_where_maximum_pow():
    torch.manual_seed(0)
    x, y = torch.randn(40), torch.randn(40)
    x[::7] = 0.0
    (out,) = oracle.run(lambda a, b: tj.where(a, tj.maximum(a, b), tj.minimum(a, b)) + tj.abs(a) ** 2.0, x, y)
    xd, yd = x.double(), y.double()
    _close(out, torch.where(xd != 0, torch.maximum(xd, yd), torch.minimum(xd, yd)) + xd.abs() ** 2)


def test_oracle_matmul_brute_force_tiny():
    torch.manual_seed(0)
    a, b = torch.randn(3, 4), torch.randn(4, 5)
    (nn,) = oracle.run(lambda x, y: tj.matmul(x, y), a, b)
    (nt,) = oracle.run(lambda x, y: tj.linear(x, y), a, b.t().contiguous())
    brute = torch.tensor([[sum(float(a[i, q]) * float(b[q, j]) for q in range(4)) for j in range(5)] for i in range(3)])
    _close(nn, brute, tol=1e-5)
    _close(nt, brute, tol=1e-5)


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (7, 13, 5), (64, 64, 64), (33, 128, 65)])
def test_oracle_matmul_with_epilogue(m, k, n):
    torch.manual_seed(0)
    a, b, bias = torch.randn(m, k), torch.randn(k, n), torch.randn(n)
    (out,) = oracle.run(lambda x, y, z: tj.gelu(tj.matmul(x, y) + z), a, b, bias)
    _close(out, F.gelu(a.double() @ b.double() + bias.double()), tol=1e-3)


def test_oracle_epilogue_reading_the_product_operand():
    """``x + linear(x, w)`` (the residual is the product's A operand) and a layer whose
    last add stays a kernel of its own in the plan, against float64."""
    torch.manual_seed(0)
    x, w, w2 = torch.randn(40, 96), 0.1 * torch.randn(96, 96), 0.1 * torch.randn(96, 96)
    (out,) = oracle.run(lambda a, b: a + tj.linear(a, b), x, w)
    _close(out, x.double() + x.double() @ w.double().t(), tol=1e-4)
    fn = lambda a, b, c: (lambda h: h + tj.linear(tj.relu(h), c))(a + tj.linear(a, b))  # noqa: E731
    (out,) = oracle.run(fn, x, w, w2)
    h = x.double() + x.double() @ w.double().t()
    _close(out, h + torch.relu(h) @ w2.double().t(), tol=1e-4)


def test_oracle_batched_matmul_broadcast_and_linear():
    torch.manual_seed(0)
    a, b = torch.randn(2, 3, 8, 16), torch.randn(3, 16, 8)
    (out,) = oracle.run(lambda x, y: tj.relu(tj.matmul(x, y)), a, b)
    _close(out, torch.relu(a.double() @ b.double()), tol=1e-3)
    x, w, bb = torch.randn(10, 32), torch.randn(48, 32), torch.randn(48)
    (out,) = oracle.run(tj.linear, x, w, bb)
    _close(out, F.linear(x.double(), w.double(), bb.double()), tol=1e-3)


@pytest.mark.parametrize("n", [1, 17, 100, 1000])
def test_oracle_reductions(n):
    torch.manual_seed(0)
    x = torch.randn(6, n)
    s, m, mu = oracle.run(lambda t: (tj.sum(t), tj.max(t), tj.mean(t, keepdim=True)), x)
    _close(s, x.double().sum(-1), tol=1e-3)
    assert torch.equal(m, x.amax(-1))                       # max is exact
    _close(mu, x.double().mean(-1, keepdim=True))


def test_oracle_reduce_non_last_axis_and_movement():
    torch.manual_seed(0)
    x = torch.randn(4, 5, 6)
    (out,) = oracle.run(lambda t: tj.sum(t, axis=1), x)
    _close(out, x.double().sum(1))
    x = torch.randn(3, 4, 5)
    (out,) = oracle.run(lambda t: tj.exp(tj.permute(t, 2, 0, 1)).reshape(5, 12) + 1.0, x)
    _close(out, torch.exp(x.double().permute(2, 0, 1)).reshape(5, 12) + 1)


def test_oracle_softmax_layernorm_rmsnorm():
    torch.manual_seed(0)
    x = torch.randn(9, 70)
    g, b = torch.randn(70), torch.randn(70)
    sm, ln, rms = oracle.run(lambda t, w, c: (tj.softmax(t), tj.layer_norm(t, w, c), tj.rms_norm(t, w)), x, g, b)
    xd, gd, bd = x.double(), g.double(), b.double()
    _close(sm, torch.softmax(xd, -1))
    _close(ln, F.layer_norm(xd, (70,), gd, bd), tol=1e-3)
    _close(rms, xd * torch.rsqrt(xd.pow(2).mean(-1, keepdim=True) + 1e-6) * gd, tol=1e-3)


def test_oracle_config2_chain_small():
    torch.manual_seed(0)
    x, a, b = torch.randn(64, 256), torch.randn(256), torch.randn(256)
    c = torch.rand(64, 256) * 8 - 4
    (y,) = oracle.run(lambda x, a, b, c: tj.gelu(x * a + b) * tj.sigmoid(c) + x, x, a, b, c)
    xd = x.double()
    _close(y, F.gelu(xd * a.double() + b.double()) * torch.sigmoid(c.double()) + xd, tol=1e-5)


def test_oracle_transformer_block():
    torch.manual_seed(0)
    T_, D, H = 12, 32, 64
    x, ln_g = torch.randn(T_, D), torch.randn(D)
    w1, b1, w2, b2 = torch.randn(H, D), torch.randn(H), torch.randn(D, H), torch.randn(D)
    wq, wk = torch.randn(D, D), torch.randn(D, D)

    def block(x, ln_g, w1, b1, w2, b2, wq, wk):
        h = tj.layer_norm(x, ln_g)
        q, k = tj.linear(h, wq), tj.linear(h, wk)
        scores = tj.softmax(tj.matmul(q, k.T) * (1.0 / 8.0))
        return x + tj.linear(tj.gelu(tj.linear(h, w1, b1)), w2, b2), scores

    out, sc = oracle.run(block, x, ln_g, w1, b1, w2, b2, wq, wk)
    d = [t.double() for t in (x, ln_g, w1, b1, w2, b2, wq, wk)]
    h = F.layer_norm(d[0], (D,), d[1])
    q, k = F.linear(h, d[6]), F.linear(h, d[7])
    _close(out, d[0] + F.linear(F.gelu(F.linear(h, d[2], d[3])), d[4], d[5]), tol=2e-3)
    _close(sc, torch.softmax(q @ k.T / 8.0, -1), tol=1e-3)


def test_oracle_rejects_non_f32():
    from tensorjit.compiler import lower
    from tensorjit.ir import DType, TensorType

    p = lower(tj.trace(lambda x: tj.exp(x), [TensorType((4,), DType.bf16)]), "hip")
    with pytest.raises(NotImplementedError):
        oracle.compile_program(p)


def test_a_planted_sign_error_in_the_oracle_is_caught(monkeypatch):
    """The checks above are sensitive: flipping gelu's erf sign in the oracle fails them."""
    from oracle import c_backend

    monkeypatch.setitem(c_backend.C_EXPR, "gelu", "(0.5f * {0} * (1.0f - or_erf({0} * 0.70710678118654752f)))")
    x = torch.linspace(-3, 3, 64)
    (y,) = oracle.run(lambda t: tj.gelu(t), x)
    assert not torch.allclose(y.double(), F.gelu(x.double()), atol=1e-3, rtol=1e-3)
