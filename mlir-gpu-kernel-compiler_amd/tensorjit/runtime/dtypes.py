"""IR dtype <-> torch dtype (ref ``tensorjit/runtime/executor.py:15-16``)."""
import torch

from ..ir import DType

TORCH_DTYPE = {DType.f32: torch.float32, DType.f16: torch.float16, DType.bf16: torch.bfloat16, DType.i32: torch.int32}
FROM_TORCH = {v: k for k, v in TORCH_DTYPE.items()}
