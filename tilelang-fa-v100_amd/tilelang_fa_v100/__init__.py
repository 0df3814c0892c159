"""MI355X (gfx950) FlashAttention, drop-in for the tilelang_fa_v100 API.

The kernels are hand-written HIP in ../csrc, built into libfa355.so and called
through a C ABI (include/fa355.h).  Exports match the reference package
(tilelang_fa_v100/__init__.py:3-16), plus reshape_and_cache, the KV-cache
writer that produces the paged layout the paged kernels read, and
set_backward_workspace_limit, the cap on the dense backward's optional dS
workspace (above it the backward needs only the reference's memory).
"""

from ._cache_write import reshape_and_cache
from ._dense import set_backward_workspace_limit
from .interface import (
    FlashAttnTileLangVFunc,
    tilelang_decode_forward,
    tilelang_flash_attn_func,
    tilelang_flash_attn_gpu,
    tilelang_paged_forward,
)

__version__ = "1.0.0"
__all__ = [
    "tilelang_flash_attn_func",
    "tilelang_flash_attn_gpu",
    "tilelang_paged_forward",
    "tilelang_decode_forward",
]
# reshape_and_cache and set_backward_workspace_limit are importable by name;
# __all__ stays the reference's list.
