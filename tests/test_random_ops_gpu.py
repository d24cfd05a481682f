"""Randomised GPU sweep of the two steps beside the attention call, bit for bit.

* ``fused_rms_norm_rope`` over seeded random shapes (batch, positions, heads,
  head dim 64 / 128), dtypes, input scales and eps, against the fp32
  restatement oracle/rms_rope.py (triton_fused.py:48-69);
* ``ContiguousKVCache.store`` over seeded random prefixes (batch, P, heads,
  head dim, bf16 or fp8 V, value scales from 1e-3 to 1e3, some heads all
  zero) against the torch ops of kv_cache.py:36-42 on the same device and
  against the oracle's quantisation.
"""

import numpy as np
import pytest
import torch

from oracle import fp8 as of
from oracle import rms_rope as orr

import qwen_image_kernel_amd as qik

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.int16).cpu().numpy()


@pytest.mark.parametrize("i", range(12))
def test_random_rms_rope_bit_exact(i):
    rng = np.random.default_rng(8100 + i)
    B, S, H = int(rng.integers(1, 4)), int(rng.integers(1, 400)), int(rng.integers(1, 31))
    D = int(rng.choice([64, 128]))
    dtype = torch.float16 if rng.random() < 0.3 else torch.bfloat16
    scale = float(10.0 ** rng.uniform(-2, 1)) if dtype == torch.bfloat16 else float(10.0 ** rng.uniform(-2, 0.5))
    eps = float(rng.choice([1e-6, 1e-5]))
    print(f"case random rms_rope {i}: {B}x{S}x{H}x{D} {dtype} scale {scale:.3g} eps {eps}", flush=True)
    g = torch.Generator().manual_seed(int(rng.integers(1 << 30)))
    x = (torch.randn(B, S, H, D, generator=g) * scale).to(dtype)
    w = torch.randn(D, generator=g) * 0.3 + 1.0
    freqs = orr.rope_freqs(S, D)
    out = qik.fused_rms_norm_rope(x.to(DEV), w.to(DEV), freqs.to(DEV), eps)
    want = orr.rms_norm_rope(x.float().numpy(), w.numpy(), freqs.real.float().numpy(), freqs.imag.float().numpy(),
                             eps, "bf16" if dtype == torch.bfloat16 else "fp16")
    np.testing.assert_array_equal(out.float().cpu().numpy(), want)


@pytest.mark.parametrize("i", range(10))
def test_random_slab_store_bit_exact(i):
    rng = np.random.default_rng(8200 + i)
    B, P, H = int(rng.integers(1, 4)), int(rng.integers(1, 700)), int(rng.integers(1, 11))
    D = int(rng.choice([64, 128]))
    v_fp8 = bool(rng.random() < 0.7)
    dtype = torch.bfloat16 if (v_fp8 or rng.random() < 0.5) else torch.float16
    vscale = float(10.0 ** rng.uniform(-3, 3)) if dtype == torch.bfloat16 else float(10.0 ** rng.uniform(-2, 2))
    print(f"case random slab store {i}: B={B} P={P} H={H} D={D} fp8={v_fp8} {dtype} v scale {vscale:.3g}", flush=True)
    g = torch.Generator().manual_seed(int(rng.integers(1 << 30)))
    k = torch.randn(B, P, H, D, generator=g).to(dtype)
    v = (torch.randn(B, P, H, D, generator=g) * vscale).to(dtype)
    if H > 1 and rng.random() < 0.5:
        v[:, :, int(rng.integers(H))] = 0     # an all-zero head: scale 1e-12, codes 0
    k, v = k.to(DEV), v.to(DEV)
    cache = qik.ContiguousKVCache(2, B, P + int(rng.integers(0, 64)), H, D, v_fp8=v_fp8, device=DEV, dtype=dtype)
    cache.get_layer(1).store(k, v)
    kv, vv, sc = cache.get_layer(1).views()
    np.testing.assert_array_equal(_bits(kv.transpose(1, 2)), _bits(k.transpose(1, 2)))
    if not v_fp8:
        np.testing.assert_array_equal(_bits(vv.transpose(1, 2)), _bits(v.transpose(1, 2)))
        return
    # kv_cache.py:36-42 on the device, as the reference runs it
    vt = v.transpose(1, 2).float()
    st = (vt.abs().amax(dim=(2, 3)).float() / 448.0).clamp_min(1e-12)
    vq = (vt / st[:, :, None, None]).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    got = vv.transpose(1, 2).contiguous().view(torch.uint8).cpu().numpy()
    np.testing.assert_array_equal(sc.cpu().numpy(), st.cpu().numpy())
    np.testing.assert_array_equal(got, vq.view(torch.uint8).cpu().numpy())
    codes, scale = of.quantize_per_head(v.float().cpu().numpy())
    np.testing.assert_array_equal(sc.cpu().numpy(), scale)
    np.testing.assert_array_equal(got, codes)
