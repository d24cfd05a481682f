"""qwen_image_kernel_amd: MI355X (gfx950) block-causal flash attention for Qwen-Image 2.1.

Drop-in for the attention path of qwen_image_kernel: ``block_causal_flash_attention``
(triton_attention.py:171) and the ``ContiguousKVCache`` prefix slab
(kv_cache.py:63), computed by a hand-written HIP kernel behind a C ABI
(include/qik_attn.h).  The package directory is ``qwen-image-kernel_amd/``;
the top-level module ``qwen_image_kernel_amd.py`` imports it under this name.
"""

from .attention import (  # noqa: F401
    block_causal_flash_attention,
    block_shape,
    build_prefix_lengths,
    tile_schedule,
)
from .kv_cache import FP8_E4M3_MAX, ContiguousKVCache  # noqa: F401

__all__ = [
    "block_causal_flash_attention",
    "build_prefix_lengths",
    "tile_schedule",
    "block_shape",
    "ContiguousKVCache",
    "FP8_E4M3_MAX",
]
