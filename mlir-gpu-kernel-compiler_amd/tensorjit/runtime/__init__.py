from .autotune import HIP_CANDIDATES, HIP_F32_CANDIDATES, MatmulConfig, autotune, cost_model
from .cache import AutotuneStore, CodeObjectCache, cache_dir, content_hash
from .dtypes import FROM_TORCH, TORCH_DTYPE
from .pool import BufferPool

__all__ = [
    "HIP_CANDIDATES", "HIP_F32_CANDIDATES", "MatmulConfig", "autotune", "cost_model",
    "AutotuneStore", "CodeObjectCache", "cache_dir", "content_hash", "TORCH_DTYPE", "FROM_TORCH", "BufferPool",
]
