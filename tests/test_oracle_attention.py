"""Oracle: fp32 attention, fp64 brute force, flash emulation, known answers (CPU)."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as oa
from oracle import fp8 as of
from oracle import lengths as ol


def _qkv(B, S, H, D, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return tuple((torch.randn(B, S, H, D, generator=g) * scale).to(torch.bfloat16) for _ in range(3))


def _fp8_slab(B, P, H, D, seed):
    g = torch.Generator().manual_seed(seed)
    ck = torch.randn(B, P, H, D, generator=g).to(torch.bfloat16)
    cv = torch.randn(B, P, H, D, generator=g).to(torch.bfloat16)
    codes, scale = of.quantize_per_head(cv.float().numpy())          # [B, H, P, D]
    cv8 = torch.from_numpy(np.ascontiguousarray(codes.transpose(0, 2, 1, 3))).view(torch.float8_e4m3fn)
    return ck, cv8, torch.from_numpy(scale)


def test_fp32_oracle_matches_fp64_brute_force():
    segs, S = ol.make_segments([("text", 12), ("img", 20), ("text", 5), ("img", 9)])
    S2 = S + 10
    q, k, v = _qkv(2, S2, 2, 32, 0)
    L = ol.build_prefix_lengths(segs, S, S2)
    kv = torch.ones(2, S2, dtype=torch.bool)
    kv[1, 3:6] = False
    a = oa.attention_fp32(q, k, v, L, kv)
    b = oa.attention_fp64(q, k, v, L, kv)
    np.testing.assert_allclose(a, b, atol=2e-6, rtol=0)


def test_fp32_oracle_with_fp8_slab_matches_fp64():
    P, SN, H, D = 24, 16, 2, 32
    ck, cv8, sc = _fp8_slab(1, P, H, D, 1)
    q, k, v = _qkv(1, SN, H, D, 2)
    L = np.full(SN, P + SN - 1, dtype=np.int32)
    a = oa.attention_fp32(q, k, v, L, None, ck, cv8, sc)
    b = oa.attention_fp64(q, k, v, L, None, ck, cv8, sc)
    np.testing.assert_allclose(a, b, atol=2e-6, rtol=0)


def test_flash_emulation_matches_fp64_within_kernel_rounding():
    """The kernel's rounding points (bf16 P, bf16 out) stay far inside the 2e-2 tolerance."""
    segs, S = ol.make_segments([("text", 40), ("img", 100)])
    q, k, v = _qkv(1, S, 2, 64, 3)
    L = ol.build_prefix_lengths(segs, S, S)
    em = oa.flash_emulation(q, k, v, L, BM=32, BN=16)
    ref = oa.attention_fp64(q, k, v, L)
    d = np.abs(em - ref)
    assert d.max() < 1e-2 and d.mean() < 1e-3


def test_known_answer_first_row_is_v0():
    """L[0] = 0: p = exp2(0) = 1, l = 1, so out[0] = bf16(V[0]) exactly."""
    q, k, v = _qkv(1, 48, 2, 64, 4)
    L = np.arange(48, dtype=np.int32)
    em = oa.flash_emulation(q, k, v, L, BM=16, BN=16)
    np.testing.assert_array_equal(em[0, 0], v[0, 0].float().numpy())
    ref = oa.attention_fp32(q, k, v, L)
    np.testing.assert_array_equal(ref[0, 0], v[0, 0].float().numpy())


def test_known_answer_first_row_fp8_slab():
    """With an fp8 slab, row L=0 returns bf16(fp32(v8[0]) * scale) exactly."""
    P, H, D = 32, 2, 64
    ck, cv8, sc = _fp8_slab(1, P, H, D, 5)
    q, k, v = _qkv(1, 8, H, D, 6)
    L = np.zeros(8, dtype=np.int32)
    em = oa.flash_emulation(q, k, v, L, None, ck, cv8, sc, BM=8, BN=16)
    want = of.dequant_bf16(cv8[0, 0].view(torch.uint8).numpy(), sc[0].numpy()[:, None])
    np.testing.assert_array_equal(em[0, 0], want)


def test_known_answer_empty_rows_are_zero():
    q, k, v = _qkv(1, 20, 2, 32, 7)
    L = np.full(20, 10, dtype=np.int32)
    L[[3, 11]] = -1
    for out in (oa.flash_emulation(q, k, v, L, BM=8, BN=8), oa.attention_fp32(q, k, v, L)):
        assert (out[0, 3] == 0).all() and (out[0, 11] == 0).all()
        assert np.abs(out[0, 4]).sum() > 0


def test_uniform_equals_unmasked_sdpa():
    q, k, v = _qkv(1, 50, 2, 64, 8)
    L = np.full(50, 49, dtype=np.int32)
    ref = F.scaled_dot_product_attention(q.float().transpose(1, 2), k.float().transpose(1, 2),
                                         v.float().transpose(1, 2)).transpose(1, 2).numpy()
    np.testing.assert_allclose(oa.attention_fp32(q, k, v, L), ref, atol=2e-6, rtol=0)


def test_slab_split_invariance():
    """Splitting the keys into slab + fresh at any P changes nothing (bf16 slab V)."""
    S, H, D = 60, 2, 32
    q, k, v = _qkv(1, S, H, D, 9)
    L = np.full(12, S - 1, dtype=np.int32)
    full = oa.attention_fp32(q[:, :12], k, v, L)
    for P in (1, 17, 32, 59):
        split = oa.attention_fp32(q[:, :12], k[:, P:], v[:, P:], L, None, k[:, :P], v[:, :P])
        np.testing.assert_allclose(split, full, atol=1e-6, rtol=0)


def test_key_permutation_invariance():
    S, H, D = 40, 1, 32
    q, k, v = _qkv(1, S, H, D, 10)
    L = np.full(S, S - 1, dtype=np.int32)
    perm = torch.from_numpy(np.random.default_rng(0).permutation(S))
    a = oa.attention_fp32(q, k, v, L)
    b = oa.attention_fp32(q, k[:, perm], v[:, perm], L)
    np.testing.assert_allclose(a, b, atol=1e-6, rtol=0)


def test_reference_signature_returns_query_dtype():
    q, k, v = _qkv(1, 16, 2, 32, 11)
    L = torch.arange(16, dtype=torch.int32)
    out = oa.reference_block_causal_attention(q, k, v, L, None)
    assert out.dtype == torch.bfloat16 and out.shape == q.shape


def test_cpu_baseline_sdpa_matches_oracle():
    segs, S = ol.make_segments([("text", 16), ("img", 30)])
    q, k, v = _qkv(1, S, 2, 64, 12)
    L = ol.build_prefix_lengths(segs, S, S)
    np.testing.assert_allclose(oa.sdpa_explicit_mask_cpu(q, k, v, L).numpy(), oa.attention_fp32(q, k, v, L),
                               atol=2e-6, rtol=0)


@pytest.mark.parametrize("with_slab", [False, True])
def test_timed_cpu_baseline_equals_the_explicit_mask_sdpa(with_slab):
    """CpuSdpaBaseline (the class the benchmark times as its CPU baseline)
    computes, per (b, h), what sdpa_explicit_mask_cpu does, and both are the
    fp32 oracle: the timed work is the reference's CPU path, not less."""
    segs, S = ol.make_segments([("text", 20), ("img", 44), ("img", 36)])
    B, H, D = 2, 3, 64
    q, k, v = _qkv(B, S, H, D, 14)
    P = 0
    ck = cv = sc = None
    if with_slab:
        P = 40
        ck, cv, sc = _fp8_slab(B, P, H, D, 15)
    L = ol.build_prefix_lengths(segs, S, S) + P
    base = oa.CpuSdpaBaseline(q, k, v, L, ck, cv, sc)
    want = oa.sdpa_explicit_mask_cpu(q, k, v, L, None, ck, cv, sc)
    assert base.pairs == int(sum(int(x) + 1 for x in L))
    for b in range(B):
        for h in range(H):
            assert torch.equal(base.run(b, h), want[b, :, h])
    np.testing.assert_allclose(want.numpy(), oa.attention_fp32(q, k, v, L, None, ck, cv, sc), atol=2e-6, rtol=0)


@pytest.mark.parametrize("bad", ["drop_scale", "swap_qk_sign"])
def test_planted_mistakes_are_caught(bad):
    """A plausible oracle mistake must fail the fp64 comparison used above."""
    q, k, v = _qkv(1, 24, 1, 32, 13)
    L = np.arange(24, dtype=np.int32)
    good = oa.attention_fp64(q, k, v, L)
    if bad == "drop_scale":
        wrong = oa.attention_fp64(q * 32 ** 0.25, k * 32 ** 0.25, v, L)   # scores not scaled by 1/sqrt(D)
    else:
        wrong = oa.attention_fp64(-q, k, v, L)
    assert np.abs(wrong - good).max() > 1e-2
