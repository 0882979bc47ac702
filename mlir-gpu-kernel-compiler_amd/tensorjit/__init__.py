"""tensorjit with an MI355X-native ``hip`` backend.

    import tensorjit as tj

    @tj.jit
    def mlp(x, g, w1, b1, w2, b2):
        h = tj.layer_norm(x, g)
        return x + tj.linear(tj.gelu(tj.linear(h, w1, b1)), w2, b2)

    y = mlp(x, g, w1, b1, w2, b2)     # ROCm tensors in and out

Pipeline: trace -> SSA tensor IR -> cleanup passes -> fusion (pointwise DAGs,
GEMM epilogues, reduction prologues) -> row fusion -> static arena plan ->
gfx950 HIP C++ (hipRTC) -> native executor with optional hipGraph replay.
"""
from .compiler import JitFunction, compile_graph, jit, lower, pick_backend
from .frontend.tracer import (
    Tensor,
    abs,
    broadcast_to,
    exp,
    gelu,
    layer_norm,
    linear,
    log,
    matmul,
    max,
    maximum,
    mean,
    minimum,
    permute,
    relu,
    reshape,
    rms_norm,
    rsqrt,
    sigmoid,
    silu,
    softmax,
    sqrt,
    sum,
    tanh,
    trace,
    transpose,
    where,
)
from .ir import DType, Graph, Node, TensorType

__version__ = "0.3.0+hip"

__all__ = [
    "jit", "JitFunction", "compile_graph", "lower", "pick_backend", "trace",
    "Tensor", "Graph", "Node", "TensorType", "DType",
    "abs", "broadcast_to", "exp", "gelu", "layer_norm", "linear", "log", "matmul", "max", "maximum", "mean",
    "minimum", "permute", "relu", "reshape", "rms_norm", "rsqrt", "sigmoid", "silu", "softmax", "sqrt", "sum",
    "tanh", "transpose", "where",
]

from .frontend.torch_backend import torch_compile_backend  # noqa: E402, F401

__all__.append("torch_compile_backend")
