"""Layouts the kernels cannot read in place still give the result.

The reference's Triton kernels read any strides.  The HIP kernels copy
16-byte chunks, so a base address off 16 bytes, b/s/h strides that are not
multiples of 8 elements or overlapping rows make the wrappers run on
contiguous device copies instead; each case here must match, bit for bit,
the same call on contiguous inputs.
"""

import numpy as np
import pytest
import torch

import qwen_image_kernel_amd as qik
from oracle import rms_rope as orr

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _flush(msg):
    print(msg, flush=True)


def _odd(shape, kind, seed, dtype=torch.bfloat16):
    """A [B, S, H, D] tensor with a layout the kernels cannot read in place,
    and its contiguous copy: `offset` starts 3 elements into a buffer (base
    6 bytes off 16-byte alignment), `pad` gives rows of D + 4 elements (a row
    stride that is not a multiple of 8)."""
    g = torch.Generator().manual_seed(seed)
    B, S, H, D = shape
    if kind == "offset":
        n = B * S * H * D
        buf = torch.randn(n + 3, generator=g).to(dtype).to(DEV)
        t = buf[3:].view(B, S, H, D)
        assert t.data_ptr() % 16 != 0
    else:
        big = torch.randn(B, S, H, D + 4, generator=g).to(dtype).to(DEV)
        t = big[..., :D]
        assert t.stride(2) % 8 != 0
    return t, t.contiguous().clone()


def _bits(t):
    return t.detach().contiguous().view(torch.int16).cpu().numpy()


@pytest.mark.parametrize("kind", ["offset", "pad"])
@pytest.mark.parametrize("split_tail", [True, False])
def test_attention_odd_layouts(kind, split_tail):
    _flush(f"case attention layout {kind} split_tail={split_tail}")
    B, SQ, P, SN, H, D = 1, 200, 96, 200, 3, 128
    q, qc = _odd((B, SQ, H, D), kind, 1)
    k, kc = _odd((B, SN, H, D), kind, 2)
    v, vc = _odd((B, SN, H, D), kind, 3)
    ck, ckc = _odd((B, P, H, D), kind, 4)
    cv, cvc = _odd((B, P, H, D), kind, 5)
    # every row sees the prefix; the fresh keys causally, with a 64-row block of full rows
    L = (torch.arange(SQ) + P).clamp(max=P + SN - 1)
    L[64:128] = P + 127
    L = L.to(torch.int32).to(DEV)
    got = qik.block_causal_flash_attention(q, k, v, L, None, ck, cv, split_tail=split_tail)
    want = qik.block_causal_flash_attention(qc, kc, vc, L, None, ckc, cvc, split_tail=split_tail)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(got), _bits(want))


@pytest.mark.parametrize("kind", ["offset", "pad"])
def test_rms_rope_odd_layouts(kind):
    _flush(f"case rms_rope layout {kind}")
    B, S, H, D = 2, 77, 5, 128
    x, xc = _odd((B, S, H, D), kind, 9)
    w = (torch.randn(D, generator=torch.Generator().manual_seed(3)) * 0.3).to(DEV)
    freqs = orr.rope_freqs(S, D).to(DEV)
    for _ in range(2):                              # the second call takes the cached path
        got = qik.fused_rms_norm_rope(x, w, freqs, 1e-6)
        want = qik.fused_rms_norm_rope(xc, w, freqs, 1e-6)
        np.testing.assert_array_equal(_bits(got), _bits(want))


@pytest.mark.parametrize("kind", ["offset", "pad"])
@pytest.mark.parametrize("v_fp8", [True, False])
def test_slab_store_odd_layouts(kind, v_fp8):
    _flush(f"case slab store layout {kind} fp8={v_fp8}")
    B, P, H, D = 2, 130, 3, 128
    k, kc = _odd((B, P, H, D), kind, 11)
    v, vc = _odd((B, P, H, D), kind, 12)
    caches = [qik.ContiguousKVCache(1, B, P + 8, H, D, v_fp8=v_fp8, device=DEV) for _ in range(2)]
    for _ in range(2):
        caches[0].get_layer(0).store(k, v)
        caches[1].get_layer(0).store(kc, vc)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(caches[0].k_buf[0, :, :, :P]), _bits(caches[1].k_buf[0, :, :, :P]))
    np.testing.assert_array_equal(caches[0].v_buf[0, :, :, :P].contiguous().view(torch.uint8).cpu().numpy(),
                                  caches[1].v_buf[0, :, :, :P].contiguous().view(torch.uint8).cpu().numpy())
    if v_fp8:
        np.testing.assert_array_equal(caches[0].v_scale.cpu().numpy(), caches[1].v_scale.cpu().numpy())
