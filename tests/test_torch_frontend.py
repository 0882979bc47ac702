"""torch.fx -> tensorjit IR translation (CPU): the translated graph, run through the
fp32 CPU oracle, matches eager PyTorch; unsupported variants are rejected (so
torch.compile falls back to eager) instead of being computed differently."""
import pytest
import torch
import torch.nn.functional as F

import oracle
from tensorjit.compiler import lower
from tensorjit.frontend.torch_backend import Unsupported, fx_to_graph


def ops_fn(x, y, w):
    a = torch.tanh(x) + torch.sigmoid(y) * torch.relu(x - 0.5)
    b = torch.rsqrt(torch.abs(y) + 1.0) ** 2.0 - torch.exp(-x.abs())
    c = (torch.maximum(a, b) * 0.75 + torch.minimum(a, b) * 0.25).clamp_min(-0.25)
    d = (c @ w).t().contiguous()
    e = torch.softmax(d.transpose(0, 1) * 0.5, dim=-1) + d.t().amax(dim=-1, keepdim=True)
    return e.sum(dim=-1) + e.mean(dim=-1) * F.silu(e).sum(dim=-1), torch.log(torch.sqrt(a * a + 1.0))


class Block(torch.nn.Module):
    def __init__(self, d=32, h=64):
        super().__init__()
        self.ln = torch.nn.LayerNorm(d)
        self.fc1 = torch.nn.Linear(d, h)
        self.fc2 = torch.nn.Linear(h, d)

    def forward(self, x):
        return x + self.fc2(F.gelu(self.fc1(self.ln(x))))


def run_translated(gm, args):
    g, sources = fx_to_graph(gm, args)
    params = dict(gm.named_parameters())
    feeds = [args[s] if isinstance(s, int) else params[s[1]].detach() for s in sources]
    prog = oracle.compile_program(lower(g, "hip"))
    return prog(*[t.float() for t in feeds])


def test_translated_ops_match_eager_through_the_oracle():
    torch.manual_seed(0)
    args = [torch.randn(48, 40), torch.randn(48, 40), torch.randn(40, 24)]
    got = run_translated(torch.fx.symbolic_trace(ops_fn), args)
    for g_, r_ in zip(got, ops_fn(*args)):
        torch.testing.assert_close(g_, r_, atol=1e-4, rtol=1e-4)


def test_translated_module_with_parameters_matches_eager():
    torch.manual_seed(0)
    m = Block().eval()
    x = torch.randn(16, 32)
    (got,) = run_translated(torch.fx.symbolic_trace(m), [x])
    with torch.no_grad():
        torch.testing.assert_close(got, m(x), atol=1e-4, rtol=1e-4)


def test_tanh_gelu_is_rejected_not_approximated():
    gm = torch.fx.symbolic_trace(lambda x: F.gelu(x, approximate="tanh"))
    with pytest.raises(Unsupported):
        fx_to_graph(gm, [torch.randn(4, 8)])
