"""Per-head RMSNorm + RoPE (qwen_image_kernel/triton_fused.py:28-105).  Test infrastructure only.

Two restatements:

* ``rms_norm_rope`` -- numpy fp32, operation for operation in the order the HIP
  kernel evaluates them (triton_fused.py:48-69 fixes the math; the order of the
  fp32 additions and the fp64 reciprocal square root are the kernel's), so the
  kernel must match it bit for bit.
* ``stock_rms_norm_rope`` -- torch, the stock diffusers semantics the reference
  tests its kernel against (tests/test_fused.py:21-33): fp32 RMSNorm, one
  rounding to the input dtype, complex multiply in fp32, rounding.  It pins
  the restatement above up to fp32 rounding, independently of its order.

Pinning of ``rms_norm_rope`` (tests/test_oracle_rms_rope.py): against
``stock_rms_norm_rope`` within the reference's 4e-2 bar and with most
elements equal; a rotation by 0 is the plain RMSNorm; a rotation by 90 degrees
maps (e, o) to (-o, e) exactly; the norm of every rotated pair is preserved;
rows scaled by a power of two give the same normalised output.
"""

from __future__ import annotations

import numpy as np
import torch

from .fp8 import bf16_round


def _round_elem(x: np.ndarray, dtype: str) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    if dtype == "bf16":
        return bf16_round(x)
    return x.astype(np.float16).astype(np.float32)


def rms_norm_rope(x: np.ndarray, weight: np.ndarray, cos: np.ndarray, sin: np.ndarray, eps: float,
                  dtype: str = "bf16") -> np.ndarray:
    """x [B, S, H, D] (fp32 values of the input dtype), weight [D] fp32, cos/sin [S, D/2] fp32.

    Per row: s = sum of x^2 -- each thread of D/8 adds the squares of its 8
    elements left to right, then lane t adds lane t^k for k = D/16 .. 1; ms =
    s / D (exact); r = fp32(1 / sqrt(fp64(fp32(ms + eps)))); n = round(fp32(fp32(x
    * r) * w)); out = round(fp32(fp32(e*c) - fp32(o*s))), round(fp32(fp32(e*s) +
    fp32(o*c))) for the pairs (e, o) = (n[2i], n[2i+1]) and (c, s) = (cos, sin)[s, i].
    Returns float32 values of the output dtype.
    """
    x = np.asarray(x, dtype=np.float32)
    B, S, H, D = x.shape
    f32 = np.float32
    tpr = D // 8
    sq = (x * x).reshape(B, S, H, tpr, 8)           # exact
    part = sq[..., 0]
    for i in range(1, 8):
        part = (part + sq[..., i]).astype(f32)
    lanes = np.arange(tpr)
    k = tpr // 2
    while k >= 1:
        part = (part + part[..., lanes ^ k]).astype(f32)
        k //= 2
    ss = part[..., 0]                                # every lane holds the same sum
    ms = (ss * f32(1.0 / D)).astype(f32)
    v = (ms + f32(eps)).astype(f32)
    r = (1.0 / np.sqrt(v.astype(np.float64))).astype(f32)
    w = np.asarray(weight, dtype=f32)
    n = _round_elem(((x * r[..., None]).astype(f32) * w).astype(f32), dtype)
    e, o = n[..., 0::2], n[..., 1::2]
    c = np.asarray(cos, dtype=f32)[None, :, None, :]
    s = np.asarray(sin, dtype=f32)[None, :, None, :]
    re = ((e * c).astype(f32) - (o * s).astype(f32)).astype(f32)
    im = ((e * s).astype(f32) + (o * c).astype(f32)).astype(f32)
    out = np.empty_like(x)
    out[..., 0::2] = _round_elem(re, dtype)
    out[..., 1::2] = _round_elem(im, dtype)
    return out


def stock_rms_norm_rope(x: torch.Tensor, weight: torch.Tensor, freqs_cis: torch.Tensor, eps: float) -> torch.Tensor:
    """The stock composition of tests/test_fused.py:21-33 (torch, any device)."""
    var = x.float().pow(2).mean(-1, keepdim=True)
    y = x * torch.rsqrt(var + eps)
    y = y * weight.float()
    y = y.to(x.dtype)
    xc = torch.view_as_complex(y.float().reshape(*y.shape[:-1], -1, 2))
    rot = xc * freqs_cis.unsqueeze(1)
    return torch.view_as_real(rot).flatten(-2).to(x.dtype)


def rope_freqs(S: int, D: int, theta: float = 10000.0, offset: int = 0) -> torch.Tensor:
    """complex64 [S, D/2] = exp(i * (offset + s) * theta^(-2j/D)) (tests/test_fused.py:40-42)."""
    inv = 1.0 / (theta ** (torch.arange(0, D, 2, dtype=torch.float64) / D))
    ang = torch.outer(torch.arange(offset, offset + S, dtype=torch.float64), inv)
    return torch.polar(torch.ones_like(ang), ang).to(torch.complex64)
