"""CPU oracle for the block-causal attention path.  TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference algorithm of the path the HIP
kernel implements.  It exists to CHECK the product: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and never as the thing measured or shipped.  The product package
(``qwen_image_kernel_amd``) does not import it and has no CPU fallback.

Modules and the reference code each restates (paths relative to the
qwen-image-kernel reference repository):

* ``lengths``   -- per-row causal-length array L (qwen_image_kernel/processors.py:22-36),
                   the mask definition it collapses (triton_attention.py:5-18), and the
                   stock multi-pass SDPA decomposition (tests/test_attention.py:17-53).
* ``schedule``  -- KV-tile schedule per row block: the reference rule
                   (triton_attention.py:79-83, 95, 115-121) and the exact rule.
* ``fp8``       -- OCP e4m3fn decode/encode from the format definition, the per-(b,h)
                   slab quantisation (kv_cache.py:36-42), the in-kernel dequant
                   rounding point (triton_attention.py:154-159), and the W8A8 linear:
                   per-tensor activation / weight quantisation (fp8.py:24-60) and the
                   tensorwise-scaled GEMM (fp8.py:87-88) in fp64.
* ``attention`` -- fp32 explicit-mask attention (triton_attention.py:266-293) extended
                   with fp8 slab V, plus an fp64 brute force for tiny inputs, and the
                   explicit-mask SDPA CPU baseline.
* ``rms_rope``  -- per-head RMSNorm + RoPE (triton_fused.py:28-105): an fp32 restatement
                   in the HIP kernel's operation order, and the stock torch composition
                   the reference tests against (tests/test_fused.py:21-33).

How each function is pinned is stated in its docstring; the tests under
``tests/test_oracle_*.py`` hold the checks.
"""
