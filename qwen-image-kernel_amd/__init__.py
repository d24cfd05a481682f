"""qwen_image_kernel_amd: MI355X (gfx950) block-causal flash attention for Qwen-Image 2.1.

Drop-in for the attention path of qwen_image_kernel: ``block_causal_flash_attention``
(triton_attention.py:171) and the ``ContiguousKVCache`` prefix slab
(kv_cache.py:63), computed by hand-written HIP kernels behind a C ABI
(include/qik_attn.h), plus the steps on either side of the attention call:
``fused_rms_norm_rope`` (triton_fused.py:75) and ``QwenImage21KernelProcessor``
(processors.py:39) (include/qik_ops.h), and the W8A8 ``FP8Linear`` of the
layer's projections (fp8.py:63) on the fp8 matrix cores (include/qik_fp8.h).
The package directory is ``qwen-image-kernel_amd/``; the top-level module
``qwen_image_kernel_amd.py`` imports it under this name.
"""

from .attention import (  # noqa: F401
    block_causal_flash_attention,
    block_shape,
    build_prefix_lengths,
    tile_schedule,
)
from .fp8 import FP8Linear, fp8_linear, quantize_tensorwise, quantize_weight_tensorwise  # noqa: F401
from .fused import fused_rms_norm_rope  # noqa: F401
from .kv_cache import FP8_E4M3_MAX, ContiguousKVCache  # noqa: F401
from .processors import QwenImage21KernelProcessor  # noqa: F401

__all__ = [
    "block_causal_flash_attention",
    "build_prefix_lengths",
    "tile_schedule",
    "block_shape",
    "ContiguousKVCache",
    "FP8_E4M3_MAX",
    "fused_rms_norm_rope",
    "QwenImage21KernelProcessor",
    "FP8Linear",
    "fp8_linear",
    "quantize_tensorwise",
    "quantize_weight_tensorwise",
]
