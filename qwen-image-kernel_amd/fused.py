"""Per-head RMSNorm + RoPE producing Q and K, same signature as the reference.

``fused_rms_norm_rope(x, weight, freqs_cis, eps)`` keeps the argument list and
result of ``qwen_image_kernel/triton_fused.py:75-105`` and runs the gfx950 HIP
kernel behind ``qik_rms_rope`` (include/qik_ops.h), asynchronously on the
current stream.

Per row of ``x [B, S, H, D]`` (fp32 arithmetic, triton_fused.py:48-69):
``n = round((x / sqrt(mean(x^2) + eps)) * weight)`` to the input dtype, then
each pair ``(n[2i], n[2i+1])`` is rotated by ``freqs_cis[s, i]`` and rounded to
the input dtype.  Differences from the reference, both on the safe side:

* a strided ``x`` (the q or k slice of a fused QKV output) is read in place
  instead of being copied to a contiguous tensor first (triton_fused.py:84-85);
* ``1 / sqrt`` is taken in fp64 and rounded once to fp32 (the reference uses the
  approximate fp32 ``rsqrt``), and every fp32 operation rounds on its own.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib

__all__ = ["fused_rms_norm_rope"]

_DTYPES = {torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_FP16}

# cos/sin tables of recent freqs_cis tensors: Q and K of a layer, and every
# layer of a step, share one.  An entry keeps its freqs_cis alive, so a data
# pointer in a key can never be reused by another tensor; the version counter
# catches in-place updates.
_cos_sin_cache: dict = {}


def _cos_sin(freqs_cis: torch.Tensor, device: torch.device):
    key = (freqs_cis.data_ptr(), freqs_cis._version, tuple(freqs_cis.shape), freqs_cis.device, device)
    hit = _cos_sin_cache.get(key)
    if hit is None:
        cos = freqs_cis.real.float().contiguous().to(device)
        sin = freqs_cis.imag.float().contiguous().to(device)
        if len(_cos_sin_cache) > 8:
            _cos_sin_cache.clear()
        hit = _cos_sin_cache[key] = (freqs_cis, cos, sin)
    return hit[1], hit[2]


def fused_rms_norm_rope(
    x: torch.Tensor,           # [B, S, H, D] bf16 (or fp16)
    weight: torch.Tensor,      # [D] fp32
    freqs_cis: torch.Tensor,   # complex [S, D/2]
    eps: float,
) -> torch.Tensor:
    """RMSNorm over D per (b, s, h), then complex RoPE by position s; returns [B, S, H, D]."""
    # One lookup per call: everything that only depends on the geometry, the
    # weight and freqs_cis tensors (and their in-place versions) and eps is
    # checked and prepared once per key -- the argument struct with the
    # weight and cos/sin pointers filled in, the output shape.  Only x's and
    # the output's data pointers change between calls.
    key = (x.shape, x.stride(), x.data_ptr() & 15, x.dtype, x.device, eps,
           weight.data_ptr(), weight._version, weight.dtype, weight.shape, weight.stride(), weight.device,
           freqs_cis.data_ptr(), freqs_cis._version, freqs_cis.dtype, freqs_cis.shape, freqs_cis.stride(),
           freqs_cis.device)
    ent = _CALLS.get(key)
    if ent is None:
        ent = _prepare(x, weight, freqs_cis, eps)
        if len(_CALLS) >= 64:
            _CALLS.clear()
        _CALLS[key] = ent
    if ent.contig:
        x = x.clone(memory_format=torch.contiguous_format)
    out = x.new_empty(ent.shape)
    a = _lib.QikRmsRopeArgs.from_buffer_copy(ent.args)
    a.x = x.data_ptr()
    a.out = out.data_ptr()
    idx = ent.index
    if idx != torch.cuda.current_device():
        with torch.cuda.device(idx):
            _lib.check(ent.fn(ctypes.byref(a), torch._C._cuda_getCurrentRawStream(idx)), "qik_rms_rope")
    else:
        _lib.check(ent.fn(ctypes.byref(a), torch._C._cuda_getCurrentRawStream(idx)), "qik_rms_rope")
    return out


class _Call:
    """What one (geometry, weight, freqs_cis, eps) key needs at call time."""

    __slots__ = ("args", "shape", "contig", "index", "fn", "keep")


# Prepared calls by key (see fused_rms_norm_rope).  An entry keeps the weight
# and freqs_cis tensors it was built from alive, so the data pointers in a
# key can never be reused by other tensors while the key is cached; their
# version counters catch in-place updates.
_CALLS: dict = {}


def _prepare(x, weight, freqs_cis, eps) -> _Call:
    if x.dim() != 4:
        raise ValueError(f"x must be [B, S, H, D], got shape {tuple(x.shape)}")
    if x.dtype not in _DTYPES:
        raise ValueError(f"x must be bf16 or fp16, got {x.dtype}")
    if not x.is_cuda:
        raise ValueError("x must be a device tensor (the kernel runs on the GPU)")
    B, S, H, D = x.shape
    if tuple(freqs_cis.shape) != (S, D // 2):
        raise ValueError(f"freqs_cis must be [S, D/2] = {(S, D // 2)}, got {tuple(freqs_cis.shape)}")
    # the kernel reads 16-byte chunks in place from a 16-byte aligned base with
    # b/s/h strides in multiples of 8 elements and a unit D stride; any other
    # layout (the reference's kernel reads any strides) goes through a
    # contiguous copy made at each call
    sb, ss, sh, sd = x.stride()
    contig = ((D > 1 and sd != 1) or x.data_ptr() % 16 != 0 or (B > 1 and sb % 8 != 0)
              or (S > 1 and ss % 8 != 0) or (H > 1 and sh % 8 != 0))
    xs = x.clone(memory_format=torch.contiguous_format) if contig else x
    w = weight
    if w.dtype != torch.float32 or w.device != x.device or not w.is_contiguous():
        w = weight.to(device=x.device, dtype=torch.float32).contiguous()
    cos, sin = _cos_sin(freqs_cis, x.device)
    out = torch.empty((B, S, H, D), dtype=x.dtype, device=x.device)
    c = _Call()
    c.args = rms_rope_args(xs, w, cos, sin, out, eps)
    c.shape = (B, S, H, D)
    c.contig = contig
    c.index = x.device.index
    c.fn = _lib.load().qik_rms_rope
    c.keep = (weight, w, freqs_cis, cos, sin)
    return c


def rms_rope_args(x, weight, cos, sin, out, eps) -> _lib.QikRmsRopeArgs:
    """The qik_rms_rope argument struct for device tensors (no device work)."""
    B, S, H, D = x.shape
    a = _lib.QikRmsRopeArgs()
    a.abi_version = _lib.ABI_VERSION
    a.dtype = _DTYPES[x.dtype]
    a.x = x.data_ptr()
    a.out = out.data_ptr()
    a.weight = weight.data_ptr()
    a.cos = cos.data_ptr()
    a.sin = sin.data_ptr()
    a.B, a.S, a.H, a.D = B, S, H, D
    a.stride_x = _lib._i64x3(x.stride(0), x.stride(1), x.stride(2))
    a.stride_out = _lib._i64x3(out.stride(0), out.stride(1), out.stride(2))
    a.eps = float(eps)
    return a
