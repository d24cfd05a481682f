"""Pins oracle/rms_rope.py (RMSNorm + RoPE of triton_fused.py:28-105) on the CPU.

The fp32 restatement is checked against the stock torch composition the
reference tests its kernel with (tests/test_fused.py:21-47, bar 4e-2), and
against what the mathematics fixes: rotation by 0 is the plain RMSNorm,
rotation by 90 degrees swaps the pair exactly, rotations preserve the norm,
and a power-of-two scaling of a row cancels exactly.
"""

import numpy as np
import pytest
import torch

from oracle import rms_rope as orr
from oracle.fp8 import bf16_round


def _inputs(B, S, H, D, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(B, S, H, D, generator=g) * 0.7).to(dtype)
    w = torch.randn(D, generator=g) * 0.3
    freqs = orr.rope_freqs(S, D)
    return x, w, freqs


def _oracle(x, w, freqs, eps, dtype="bf16"):
    return orr.rms_norm_rope(x.float().numpy(), w.numpy(), freqs.real.float().numpy(),
                             freqs.imag.float().numpy(), eps, dtype)


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_matches_stock_composition(D, dtype):
    x, w, freqs = _inputs(2, 37, 5, D, seed=D, dtype=dtype)
    got = _oracle(x, w, freqs, 1e-6, "bf16" if dtype == torch.bfloat16 else "fp16")
    ref = orr.stock_rms_norm_rope(x, w, freqs, 1e-6).float().numpy()
    d = np.abs(got - ref)
    assert d.max() < 4e-2                      # the reference's bar (tests/test_fused.py:46)
    assert (d == 0).mean() > 0.95              # same values except near rounding ties


def _rms_only(x, w, eps):
    """bf16((x * r) * w) with r = fp32(1/sqrt(fp64(fp32(mean(x^2) + eps)))) summed in fp64
    (exact for these sizes), i.e. the normalisation without the rotation."""
    xf = x.float().numpy().astype(np.float64)
    ms = np.float32((xf * xf).sum(-1) / x.shape[-1])
    r = (1.0 / np.sqrt(np.float32(ms + np.float32(eps)).astype(np.float64))).astype(np.float32)
    return bf16_round((x.float().numpy() * r[..., None]).astype(np.float32) * w.numpy())


def test_rotation_by_zero_is_rmsnorm():
    B, S, H, D = 1, 9, 3, 128
    x, w, _ = _inputs(B, S, H, D, seed=3)
    cos = np.ones((S, D // 2), np.float32)
    sin = np.zeros((S, D // 2), np.float32)
    got = orr.rms_norm_rope(x.float().numpy(), w.numpy(), cos, sin, 1e-6)
    want = _rms_only(x, w, 1e-6)
    # the fp32 sum of squares may differ from the exact sum by an ulp; compare in bf16 ulps
    assert np.abs(got - want).max() <= np.abs(want).max() * 2.0 ** -7


def test_rotation_by_ninety_degrees_swaps_pairs():
    B, S, H, D = 2, 5, 4, 64
    x, w, _ = _inputs(B, S, H, D, seed=4)
    one = np.ones((S, D // 2), np.float32)
    zero = np.zeros((S, D // 2), np.float32)
    n = orr.rms_norm_rope(x.float().numpy(), w.numpy(), one, zero, 1e-6)
    r = orr.rms_norm_rope(x.float().numpy(), w.numpy(), zero, one, 1e-6)
    assert np.array_equal(r[..., 0::2], -n[..., 1::2])
    assert np.array_equal(r[..., 1::2], n[..., 0::2])


def test_rotation_preserves_pair_norm():
    x, w, freqs = _inputs(1, 64, 2, 128, seed=5)
    one = np.ones((64, 64), np.float32)
    zero = np.zeros((64, 64), np.float32)
    n = orr.rms_norm_rope(x.float().numpy(), w.numpy(), one, zero, 1e-6)
    r = _oracle(x, w, freqs, 1e-6)
    nn = np.hypot(n[..., 0::2], n[..., 1::2])
    rn = np.hypot(r[..., 0::2], r[..., 1::2])
    assert np.allclose(rn, nn, rtol=2.0 ** -6, atol=1e-6)


def test_power_of_two_row_scaling_cancels():
    x, w, freqs = _inputs(1, 11, 3, 128, seed=6)
    a = _oracle(x, w, freqs, 0.0)
    b = _oracle((x.float() * 4).to(torch.bfloat16), w, freqs, 0.0)
    assert np.array_equal(a, b)


def test_planted_sign_error_is_caught():
    """A restatement with the sine term's sign flipped must fail the stock comparison."""
    x, w, freqs = _inputs(1, 20, 2, 128, seed=7)
    ref = orr.stock_rms_norm_rope(x, w, freqs, 1e-6).float().numpy()
    bad = orr.rms_norm_rope(x.float().numpy(), w.numpy(), freqs.real.float().numpy(),
                            -freqs.imag.float().numpy(), 1e-6)
    assert np.abs(bad - ref).max() > 4e-2
