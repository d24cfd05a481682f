"""fp8e4m3fn (OCP) and bf16 rounding, and the slab quantisation.  Test infrastructure only.

Everything here is derived from the number formats' definitions, not from a
library, so the library casts the product relies on (torch's ``.to(float8_e4m3fn)``,
hipcc's bf16 conversion, the gfx950 fp8 decode) can be checked against it.
"""

from __future__ import annotations

import numpy as np

E4M3_MAX = 448.0


def e4m3fn_decode_table() -> np.ndarray:
    """float32[256]: value of every e4m3fn code (1 sign, 4 exponent bits, bias 7, 3 mantissa bits).

    Exponent 0 is subnormal (m * 2**-9); S.1111.111 is NaN; there is no infinity.
    """
    vals = np.empty(256, dtype=np.float32)
    for c in range(256):
        s, e, m = c >> 7, (c >> 3) & 15, c & 7
        if e == 15 and m == 7:
            v = np.nan
        elif e == 0:
            v = m * 2.0 ** -9
        else:
            v = (1.0 + m / 8.0) * 2.0 ** (e - 7)
        vals[c] = -v if s else v
    return vals


_TABLE = e4m3fn_decode_table()
_POS = _TABLE[:127].astype(np.float64)  # codes 0..126, increasing


def e4m3fn_encode(x: np.ndarray) -> np.ndarray:
    """uint8 codes of fp32 values, round to nearest, ties to even mantissa.

    Defined for |x| <= 448 (callers clamp first, as kv_cache.py:40 does); NaN
    maps to 0x7F/0xFF.
    """
    x = np.asarray(x, dtype=np.float32)
    a = np.abs(x).astype(np.float64)
    hi = np.clip(np.searchsorted(_POS, a, side="left"), 0, 126)
    lo = np.clip(hi - 1, 0, 126)
    dlo = np.abs(a - _POS[lo])
    dhi = np.abs(_POS[hi] - a)
    pick_hi = (dhi < dlo) | ((dhi == dlo) & ((hi & 1) == 0))
    code = np.where(pick_hi, hi, lo).astype(np.uint8)
    code = np.where(np.signbit(x), code | 0x80, code).astype(np.uint8)
    code = np.where(np.isnan(x), np.where(np.signbit(x), 0xFF, 0x7F), code).astype(np.uint8)
    return code


def bf16_round(x: np.ndarray) -> np.ndarray:
    """fp32 -> nearest bf16 (ties to even), returned as float32 values."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32)
    return np.where(np.isnan(x), x, out)


def quantize_per_head(v: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Slab V quantisation of kv_cache.py:36-42 for v [B, P, H, D].

    Returns (codes uint8 [B, H, P, D], scale float32 [B, H]) with
    scale = max(amax|v| * fp32(1/448), 1e-12) and
    code = e4m3fn(clamp(v / scale, -448, 448)) using a true fp32 division.

    The reference runs this on the GPU, where torch evaluates ``tensor / 448.0``
    (a host scalar divisor) as a multiply by the fp32 reciprocal, while
    ``tensor / tensor`` is a true division; both are restated here.
    """
    vt = np.ascontiguousarray(np.asarray(v, dtype=np.float32).transpose(0, 2, 1, 3))
    amax = np.abs(vt).max(axis=(2, 3)).astype(np.float32)
    inv = np.float32(1.0) / np.float32(E4M3_MAX)
    scale = np.maximum(amax * inv, np.float32(1e-12)).astype(np.float32)
    q = np.clip(vt / scale[:, :, None, None], -E4M3_MAX, E4M3_MAX).astype(np.float32)
    return e4m3fn_encode(q), scale


def dequant_bf16(codes: np.ndarray, scale) -> np.ndarray:
    """bf16(fp32(code) * scale): the in-kernel rounding point (triton_attention.py:157-159).

    ``scale`` broadcasts against ``codes`` (e.g. [B, H, 1, 1] for [B, H, P, D]).
    """
    vals = _TABLE[np.asarray(codes, dtype=np.uint8)]
    return bf16_round(vals * np.asarray(scale, dtype=np.float32))


def tensor_scale(x: np.ndarray) -> np.float32:
    """Per-tensor scale of fp8.py:24-26 / :58 as torch forms it on a GPU:
    max(amax|x| * fp32(1/448), 1e-12) (a tensor divided by the host scalar 448
    is multiplied by its fp32 reciprocal there; clamp_min keeps NaN)."""
    a = np.abs(np.asarray(x, dtype=np.float32)).max()
    if np.isnan(a):
        return np.float32(np.nan)
    inv = np.float32(1.0) / np.float32(E4M3_MAX)
    return np.float32(max(np.float32(a * inv), np.float32(1e-12)))


def quantize_tensorwise(x: np.ndarray) -> tuple[np.ndarray, np.float32]:
    """Activation quantisation of fp8.py:43-53: scale as tensor_scale, then
    code = e4m3(x * fp32(1 / scale)) (the reciprocal is one correctly rounded
    fp32 division, fp8.py:37), no clamp (|x * (1/scale)| < 464 for finite x)."""
    x = np.asarray(x, dtype=np.float32)
    s = tensor_scale(x)
    inv = np.float32(1.0) / s
    return e4m3fn_encode((x * inv).astype(np.float32)), s


def quantize_weight_tensorwise(w: np.ndarray) -> tuple[np.ndarray, np.float32]:
    """Weight quantisation of fp8.py:56-60: code = e4m3(clamp(w / scale, +-448))
    with a correctly rounded fp32 division per element."""
    w = np.asarray(w, dtype=np.float32)
    s = tensor_scale(w)
    q = np.clip((w / s).astype(np.float32), -E4M3_MAX, E4M3_MAX).astype(np.float32)
    return e4m3fn_encode(q), s


def decode(codes: np.ndarray) -> np.ndarray:
    """fp32 values of e4m3fn codes (exact)."""
    return _TABLE[np.asarray(codes, dtype=np.uint8)]


def scaled_mm(a_codes: np.ndarray, w_codes: np.ndarray, scale_a, scale_w, bias=None) -> np.ndarray:
    """fp64 value of what torch._scaled_mm(A, W.t(), scale_a, scale_b, bias)
    computes with tensorwise scales (fp8.py:87-88), before the final rounding:
    (sum_k A[m,k] W[n,k]) * fp32(scale_a * scale_w) + bias[n].  The fp8
    products are exact in fp64 and their fp64 sum is far closer to the exact
    sum than any fp32 accumulation, so this is the target an fp32-accumulating
    GEMM approaches.  Returns float64 [M, N]."""
    acc = decode(a_codes).astype(np.float64) @ decode(w_codes).astype(np.float64).T
    ab = np.float64(np.float32(np.float32(scale_a) * np.float32(scale_w)))
    out = acc * ab
    if bias is not None:
        out = out + np.asarray(bias, dtype=np.float64)[None, :]
    return out
