"""GPU parity: the HIP kernel against the CPU oracle on the same seeded inputs.

Tolerances (fp32 explicit-mask oracle, bf16 output): max-abs <= 2e-2 and
mean-abs <= 2e-3.  Against the numpy emulation of the reference kernel's tile
loop and rounding points the bar is tighter (TIGHT_MAX).  Integer results
(causal lengths, the visited-tile schedule) must be bit-exact.
"""

import dataclasses

import numpy as np

import pytest
import torch

from oracle import attention as oa
from oracle import fp8 as of
from oracle import lengths as ol
from oracle import schedule as osch

import qwen_image_kernel_amd as qik
import qwen_image_kernel_amd.workloads as wls

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MEAN_ABS = 2e-3
TIGHT_MAX = 4e-3  # vs the tile-loop emulation: only accumulation order and exp2 ulps differ
DEV = "cuda"


def _rand(shape, gen, scale=1.0, dtype=torch.bfloat16):
    return (torch.randn(*shape, generator=gen) * scale).to(dtype)


def _check(out, ref, max_abs=MAX_ABS, mean_abs=MEAN_ABS, what=""):
    o = out.float().cpu().numpy() if isinstance(out, torch.Tensor) else out
    d = np.abs(o - ref)
    assert np.isfinite(o).all(), f"{what}: non-finite output"
    assert d.max() <= max_abs, f"{what}: max|diff| {d.max():.3e} > {max_abs}"
    assert d.mean() <= mean_abs, f"{what}: mean|diff| {d.mean():.3e} > {mean_abs}"
    return d.max(), d.mean()


def _flush(msg):
    print(msg, flush=True)


# ---------------------------------------------------------------------------
# the reference's own test layouts (tests/test_attention.py:112-117), H=4, D=128, x0.3

PREFILL_CASES = [
    ("t2i prefill", [("text", 256), ("img", 1024)], 1, False),
    ("edit prefill", [("text", 64), ("img", 4096), ("text", 32), ("img", 256)], 1, False),
    ("padded prompt", [("text", 128), ("img", 512)], 1, True),
    ("batch=2", [("text", 96), ("img", 200)], 2, False),
]


@pytest.mark.parametrize("name,layout,batch,padding", PREFILL_CASES, ids=[c[0] for c in PREFILL_CASES])
def test_reference_prefill_layouts(name, layout, batch, padding):
    _flush(f"case {name}")
    segs, S = ol.make_segments(layout)
    g = torch.Generator().manual_seed(100)
    H, D = 4, 128
    q, k, v = (_rand((batch, S, H, D), g, 0.3) for _ in range(3))
    kv = None
    if padding:
        first_text_end = next(e for s, e, t in segs if t)
        kv = torch.ones(batch, S, dtype=torch.bool)
        kv[:, first_text_end - 5:first_text_end] = False
    L = ol.build_prefix_lengths(segs, segs[-1][1], S)
    out = qik.block_causal_flash_attention(
        q.to(DEV), k.to(DEV), v.to(DEV), torch.from_numpy(L).to(DEV), None if kv is None else kv.to(DEV))
    torch.cuda.synchronize()
    ref = oa.attention_fp32(q, k, v, L, kv)
    _check(out, ref, what=name)
    stock = ol.stock_multipass_sdpa(q, k, v, segs, segs[-1][1], kv).numpy()
    _check(out, stock, what=name + " vs stock")


@pytest.mark.parametrize("prefix,target", [(256, 512), (1024, 1024)])
def test_reference_decode_bf16_cache(prefix, target):
    _flush(f"case decode prefix={prefix} target={target}")
    g = torch.Generator().manual_seed(200 + prefix)
    H, D = 4, 128
    q, kn, vn = (_rand((1, target, H, D), g, 0.3) for _ in range(3))
    ck, cv = (_rand((1, prefix, H, D), g, 0.3) for _ in range(2))
    L = np.full(target, prefix + target - 1, dtype=np.int32)
    out = qik.block_causal_flash_attention(q.to(DEV), kn.to(DEV), vn.to(DEV), torch.from_numpy(L).to(DEV), None,
                                           cache_k=ck.to(DEV), cache_v=cv.to(DEV))
    ref = oa.attention_fp32(q, kn, vn, L, None, ck, cv)
    _check(out, ref, what="decode bf16 cache")


def test_tight_against_tile_loop_emulation():
    """Same tiles and rounding points as the reference kernel: differences stay at fp32-ulp level."""
    _flush("case emulation")
    segs, S = ol.make_segments([("text", 70), ("img", 190), ("text", 9), ("img", 60)])
    S2 = S + 100
    g = torch.Generator().manual_seed(300)
    H, D = 2, 128
    q, k, v = (_rand((1, S2, H, D), g) for _ in range(3))
    L = ol.build_prefix_lengths(segs, S, S2)
    out = qik.block_causal_flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), torch.from_numpy(L).to(DEV), None)
    em = oa.flash_emulation(q, k, v, L, BM=128, BN=64)
    _check(out, em, max_abs=TIGHT_MAX, mean_abs=2e-4, what="vs emulation")


# ---------------------------------------------------------------------------
# prefix-KV slab (kv_cache.py) with fp8 V

def _slab_case(B, P, SN, SQ, H, D, seed, v_fp8=True):
    g = torch.Generator().manual_seed(seed)
    q = _rand((B, SQ, H, D), g)
    kn, vn = (_rand((B, SN, H, D), g) for _ in range(2))
    ck, cv = (_rand((B, P, H, D), g) for _ in range(2))
    cache = qik.ContiguousKVCache(2, B, P + 272, H, D, v_fp8=v_fp8, device=DEV)
    cache.get_layer(1).store(ck.to(DEV), cv.to(DEV))
    return q, kn, vn, ck, cv, cache


def test_fp8_slab_store_matches_oracle_quantisation():
    _flush("case slab quantisation")
    q, kn, vn, ck, cv, cache = _slab_case(2, 300, 64, 64, 3, 128, 400)
    k, v, sc = cache.get_layer(1).views()
    codes, scale = of.quantize_per_head(cv.float().numpy())
    np.testing.assert_array_equal(sc.cpu().numpy(), scale)
    got = v.contiguous().view(torch.uint8).cpu().numpy().transpose(0, 2, 1, 3)
    np.testing.assert_array_equal(got, codes)
    np.testing.assert_array_equal(k.cpu().float().numpy(), ck.float().numpy())


@pytest.mark.parametrize("uniform", [True, False])
def test_decode_fp8_slab(uniform):
    _flush(f"case decode fp8 slab uniform={uniform}")
    B, P, SN, H, D = 1, 640, 256, 4, 128
    q, kn, vn, ck, cv, cache = _slab_case(B, P, SN, SN, H, D, 500)
    k8, v8, sc = cache.get_layer(1).views()
    L = np.full(SN, P + SN - 1, dtype=np.int32)
    out = qik.block_causal_flash_attention(q.to(DEV), kn.to(DEV), vn.to(DEV), torch.from_numpy(L).to(DEV), None,
                                           cache_k=k8, cache_v=v8, cache_v_scale=sc, uniform_full=uniform)
    ref = oa.attention_fp32(q, kn, vn, L, None, k8.cpu(), v8.cpu(), sc.cpu())
    _check(out, ref, what="fp8 slab")
    em = oa.flash_emulation(q, kn, vn, L, None, k8.cpu(), v8.cpu(), sc.cpu(), uniform=uniform)
    _check(out, em, max_abs=TIGHT_MAX, mean_abs=2e-4, what="fp8 slab vs emulation")
    # fp8-V vs bf16-V attention, rel-L2 < 0.03 (tests/test_kv_cache.py:40-60)
    out16 = qik.block_causal_flash_attention(q.to(DEV), kn.to(DEV), vn.to(DEV), torch.from_numpy(L).to(DEV), None,
                                             cache_k=ck.to(DEV), cache_v=cv.to(DEV))
    rel = ((out.float() - out16.float()).norm() / out16.float().norm()).item()
    assert rel < 0.03


def test_slab_prefill_ragged_multiref_layout_small():
    """All rows queried against [slab, fresh] with a ragged L (the multi-reference shape, scaled down)."""
    _flush("case slab ragged")
    segs, P = ol.make_segments([("text", 40), ("img", 100), ("img", 70), ("img", 90)])
    SN = 200
    SQ = P + SN
    q, kn, vn, ck, cv, cache = _slab_case(2, P, SN, SQ, 3, 128, 600)
    k8, v8, sc = cache.get_layer(1).views()
    L = ol.build_prefix_lengths(segs, P, SQ)
    out = qik.block_causal_flash_attention(q.to(DEV), kn.to(DEV), vn.to(DEV), torch.from_numpy(L).to(DEV), None,
                                           cache_k=k8, cache_v=v8, cache_v_scale=sc)
    ref = oa.attention_fp32(q, kn, vn, L, None, k8.cpu(), v8.cpu(), sc.cpu())
    _check(out, ref, what="slab ragged")


# ---------------------------------------------------------------------------
# known answers and edge cases

def test_first_row_and_empty_rows_exact():
    _flush("case known answers")
    g = torch.Generator().manual_seed(700)
    S, H, D = 200, 2, 128
    q, k, v = (_rand((1, S, H, D), g) for _ in range(3))
    L = np.arange(S, dtype=np.int32)
    L[[5, 130, 199]] = -1
    out = qik.block_causal_flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), torch.from_numpy(L).to(DEV), None)
    o = out.cpu()
    assert torch.equal(o[0, 0], v[0, 0])           # L = 0: p = 1, l = 1
    for r in (5, 130, 199):
        assert (o[0, r] == 0).all()                # L = -1: no key
    ref = oa.attention_fp32(q, k, v, L)
    _check(out, ref, what="known answers")


def test_empty_query_and_no_fresh_keys():
    """Zero query rows return an empty output without a launch (the reference's grid is
    empty); with no fresh keys (SN = 0) the rows attend the slab alone."""
    _flush("case empty query / no fresh keys")
    g = torch.Generator().manual_seed(31)
    k, v = _rand((1, 64, 2, 128), g), _rand((1, 64, 2, 128), g)
    q0 = torch.empty(1, 0, 2, 128, dtype=torch.bfloat16, device=DEV)
    out0 = qik.block_causal_flash_attention(q0, k.to(DEV), v.to(DEV), torch.empty(0, dtype=torch.int32, device=DEV),
                                            None)
    assert out0.shape == q0.shape
    B, P, H, D, SQ = 2, 200, 3, 128, 96
    q, kn, vn, ck, cv, cache = _slab_case(B, P, 0, SQ, H, D, 700)
    k8, v8, sc = cache.get_layer(1).views()
    rng = np.random.default_rng(31)
    L = rng.integers(-1, P, size=SQ).astype(np.int32)
    for split in (True, False):
        out = qik.block_causal_flash_attention(q.to(DEV), kn.to(DEV), vn.to(DEV), torch.from_numpy(L).to(DEV), None,
                                               cache_k=k8, cache_v=v8, cache_v_scale=sc, split_tail=split)
        ref = oa.attention_fp32(q, kn, vn, L, None, k8.cpu(), v8.cpu(), sc.cpu())
        _check(out, ref, what=f"slab only, split={split}")


def test_all_keys_invalid_gives_zeros():
    g = torch.Generator().manual_seed(710)
    q, k, v = (_rand((1, 96, 2, 128), g) for _ in range(3))
    L = np.full(96, 95, dtype=np.int32)
    kv = torch.zeros(1, 96, dtype=torch.bool)
    kv[0, 50:] = True
    kv_none = torch.zeros(1, 96, dtype=torch.bool)
    out = qik.block_causal_flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), torch.from_numpy(L).to(DEV),
                                           kv_none.to(DEV))
    assert (out == 0).all()
    out = qik.block_causal_flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), torch.from_numpy(L).to(DEV), kv.to(DEV))
    _check(out, oa.attention_fp32(q, k, v, L, kv), what="partial key_valid")


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 128), (torch.float16, 64)])
def test_key_valid_on_some_tiles_only(dtype, D):
    """A KV tile whose keys are all valid runs without the key_valid term.  A mask
    that is all true equals no mask bit for bit; padding confined to one tile per
    batch (fresh keys, then slab and fresh keys of a decode) follows the oracle."""
    _flush(f"case key_valid on some tiles {dtype} D={D}")
    segs, S = ol.make_segments([("text", 256), ("img", 1024)])
    g = torch.Generator().manual_seed(720 + D)
    B, H = 2, 4
    q, k, v = (_rand((B, S, H, D), g, 0.3, dtype) for _ in range(3))
    L = ol.build_prefix_lengths(segs, S, S)
    qd, kd, vd, Ld = q.to(DEV), k.to(DEV), v.to(DEV), torch.from_numpy(L).to(DEV)
    plain = qik.block_causal_flash_attention(qd, kd, vd, Ld, None)
    ones = torch.ones(B, S, dtype=torch.bool)
    assert torch.equal(qik.block_causal_flash_attention(qd, kd, vd, Ld, ones.to(DEV)), plain)
    kv = ones.clone()
    kv[0, 200:256] = False      # padded text of batch 0: keys 192-255 are one tile
    kv[1, 700:710] = False      # a few image keys of batch 1
    out = qik.block_causal_flash_attention(qd, kd, vd, Ld, kv.to(DEV))
    _check(out, oa.attention_fp32(q, k, v, L, kv), what="padding in one tile")

    P, T = 320, 256             # decode against a bf16 slab; the mask spans slab + fresh keys
    ck, cv = (_rand((B, P, H, D), g, 0.3, dtype) for _ in range(2))
    qn, kn, vn = (_rand((B, T, H, D), g, 0.3, dtype) for _ in range(3))
    Lt = np.full(T, P + T - 1, dtype=np.int32)
    kvd = torch.ones(B, P + T, dtype=torch.bool)
    kvd[0, 130:140] = False
    kvd[1, P + 70:P + 75] = False
    out = qik.block_causal_flash_attention(qn.to(DEV), kn.to(DEV), vn.to(DEV), torch.from_numpy(Lt).to(DEV),
                                           kvd.to(DEV), cache_k=ck.to(DEV), cache_v=cv.to(DEV))
    _check(out, oa.attention_fp32(qn, kn, vn, Lt, kvd, ck, cv), what="padding in a slab tile")


def test_decode_fp8_slab_head_dim_64_ragged_with_key_valid():
    """The fp8-slab kernel at D=64 with ragged causal lengths and a key_valid mask
    over slab and fresh keys; the slab ends inside a tile (200 = 3 x 64 + 8)."""
    _flush("case fp8 slab D=64 ragged key_valid")
    B, P, SN, H, D = 2, 200, 130, 3, 64
    q, kn, vn, ck, cv, cache = _slab_case(B, P, SN, SN, H, D, 730)
    k8, v8, sc = cache.get_layer(1).views()
    rng = np.random.default_rng(731)
    L = np.sort(rng.integers(-1, P + SN, size=SN)).astype(np.int32)
    kv = torch.ones(B, P + SN, dtype=torch.bool)
    kv[0, 190:205] = False     # across the slab's end
    kv[1, P + 60:P + 64] = False
    kv[1, 5] = False
    out = qik.block_causal_flash_attention(q.to(DEV), kn.to(DEV), vn.to(DEV), torch.from_numpy(L).to(DEV), kv.to(DEV),
                                           cache_k=k8, cache_v=v8, cache_v_scale=sc)
    ref = oa.attention_fp32(q, kn, vn, L, kv, k8.cpu(), v8.cpu(), sc.cpu())
    _check(out, ref, what="fp8 slab D=64 ragged key_valid")
    em = oa.flash_emulation(q, kn, vn, L, kv, k8.cpu(), v8.cpu(), sc.cpu())
    _check(out, em, max_abs=TIGHT_MAX, mean_abs=2e-4, what="vs emulation")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [32, 64, 128, 256])
def test_dtypes_and_head_dims(dtype, D):
    _flush(f"case dtype={dtype} D={D}")
    segs, S = ol.make_segments([("text", 37), ("img", 16), ("text", 11), ("img", 25)])
    S2 = S + 77
    g = torch.Generator().manual_seed(800 + D)
    q, k, v = (_rand((2, S2, 4, D), g, 1.0, dtype) for _ in range(3))
    L = ol.build_prefix_lengths(segs, S, S2)
    out = qik.block_causal_flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), torch.from_numpy(L).to(DEV), None)
    assert out.dtype == dtype
    _check(out, oa.attention_fp32(q, k, v, L), what=f"{dtype} D={D}")


@pytest.mark.parametrize("D", [32, 256])
def test_other_head_dims_slab_fp8_key_valid_and_long_rows(D):
    """Head dims 32 and 256 (the reference kernel takes any power-of-two
    HEAD_DIM, triton_attention.py:63-74): an fp8 slab with ragged lengths and
    padded keys, and a fresh-key call long enough for several rounds of row
    blocks (the queued launch and its merged pieces; the two-group form for
    D = 32), against the fp32 oracle."""
    _flush(f"case head dim {D}: fp8 slab + key_valid, long rows")
    g = torch.Generator().manual_seed(900 + D)
    B, P, SN, H = 2, 200, 130, 3
    kp, vp = (_rand((B, P, H, D), g) for _ in range(2))
    cache = qik.ContiguousKVCache(1, B, P + 40, H, D, v_fp8=True, device=DEV)
    cache.get_layer(0).store(kp.to(DEV), vp.to(DEV))
    k8, v8, sc = cache.get_layer(0).views()
    q, kn, vn = (_rand((B, SN, H, D), g) for _ in range(3))
    L = (np.arange(SN, dtype=np.int32) + P).clip(max=P + SN - 1)
    L[:40] = P - 1 - np.arange(40)
    kv = torch.ones(B, P + SN, dtype=torch.bool)
    kv[1, 5:30] = False
    kv[0, P + 7:P + 9] = False
    out = qik.block_causal_flash_attention(q.to(DEV), kn.to(DEV), vn.to(DEV), torch.from_numpy(L).to(DEV),
                                           kv.to(DEV), cache_k=k8, cache_v=v8, cache_v_scale=sc)
    _check(out, oa.attention_fp32(q, kn, vn, L, kv, k8.cpu(), v8.cpu(), sc.cpu()), what=f"fp8 slab D={D}")
    for split in (True, False):
        S, H2 = 2100, 6
        segs, S0 = ol.make_segments([("text", 100), ("img", 1500)])
        qq, kk, vv = (_rand((1, S, H2, D), g) for _ in range(3))
        L2 = ol.build_prefix_lengths(segs, S0, S)
        out = qik.block_causal_flash_attention(qq.to(DEV), kk.to(DEV), vv.to(DEV), torch.from_numpy(L2).to(DEV),
                                               None, split_tail=split)
        _check(out, oa.attention_fp32(qq, kk, vv, L2, None, heads=range(H2)), what=f"long rows D={D} split={split}")


def test_fused_qkv_strided_value_view():
    """V as a chunk of a fused QKV output (stride_s = 3*H*D), as processors.py:68-70 passes it."""
    _flush("case strided qkv")
    g = torch.Generator().manual_seed(900)
    B, S, H, D = 1, 333, 4, 128
    qkv = _rand((B, S, 3 * H, D), g).to(DEV)
    q, k, v = qkv.chunk(3, dim=-2)
    L = torch.full((S,), S - 1, dtype=torch.int32, device=DEV)
    out = qik.block_causal_flash_attention(q, k, v, L, None, uniform_full=True)
    out2 = qik.block_causal_flash_attention(q.contiguous(), k.contiguous(), v.contiguous(), L, None)
    assert torch.equal(out, out2)
    _check(out, oa.attention_fp32(q.cpu(), k.cpu(), v.cpu(), L.cpu().numpy()), what="strided")


def test_deterministic():
    g = torch.Generator().manual_seed(950)
    q, k, v = (_rand((1, 700, 4, 128), g).to(DEV) for _ in range(3))
    L = torch.arange(700, dtype=torch.int32, device=DEV)
    a = qik.block_causal_flash_attention(q, k, v, L, None)
    b = qik.block_causal_flash_attention(q, k, v, L, None)
    assert torch.equal(a, b)


def test_misaligned_input_rejected_by_the_abi_and_copied_by_the_wrapper():
    """A base 8 bytes off 16-byte alignment: qik_attn_validate rejects it
    (QIK_ERR_ALIGN, before any launch); the Python entry point runs it through
    a contiguous copy and returns the bits of the call on aligned inputs."""
    import ctypes
    from qwen_image_kernel_amd import _lib, attention
    g = torch.Generator().manual_seed(960)
    base = _rand((64 * 4 * 128 + 4,), g).to(DEV)
    q = base[4:].view(1, 64, 4, 128)                 # 8-byte offset: not 16-byte aligned
    L = torch.arange(64, dtype=torch.int32, device=DEV)
    out = torch.empty(q.shape, dtype=q.dtype, device=DEV)
    a = attention.make_args(q, q, q, L, None, out, None, None, None, False)
    assert _lib.load().qik_attn_validate(ctypes.byref(a)) == -8
    got = qik.block_causal_flash_attention(q, q, q, L, None)
    qc = q.clone()
    want = qik.block_causal_flash_attention(qc, qc, qc, L, None)
    np.testing.assert_array_equal(got.view(torch.int16).cpu().numpy(), want.view(torch.int16).cpu().numpy())


def test_side_inputs_on_the_host_or_misshaped_are_rejected():
    """prefix_lengths, key_valid, cache_v_scale and debug_tiles reach the kernel as raw
    device addresses: host tensors, a key_valid batch that is neither 1 nor B, and an
    undersized or non-int32 debug_tiles raise before any launch."""
    g = torch.Generator().manual_seed(961)
    q, k, v = (_rand((2, 128, 2, 128), g).to(DEV) for _ in range(3))
    L = torch.arange(128, dtype=torch.int32)
    with pytest.raises(ValueError, match="prefix_lengths"):
        qik.block_causal_flash_attention(q, k, v, L, None)
    Ld = L.to(DEV)
    with pytest.raises(ValueError, match="key_valid"):
        qik.block_causal_flash_attention(q, k, v, Ld, torch.ones(2, 128, dtype=torch.bool))
    with pytest.raises(ValueError, match="batch dim"):
        qik.block_causal_flash_attention(q, k, v, Ld, torch.ones(3, 128, dtype=torch.bool, device=DEV))
    with pytest.raises(ValueError, match="debug_tiles"):
        qik.block_causal_flash_attention(q, k, v, Ld, None, debug_tiles=torch.zeros(3, dtype=torch.int32, device=DEV))
    with pytest.raises(ValueError, match="debug_tiles"):
        qik.block_causal_flash_attention(q, k, v, Ld, None, debug_tiles=torch.zeros(4, dtype=torch.int64, device=DEV))
    kc = _rand((2, 64, 2, 128), g).to(DEV)
    vc = kc.to(torch.float8_e4m3fn)
    with pytest.raises(ValueError, match="cache_v_scale"):
        qik.block_causal_flash_attention(q, k, v, Ld, None, cache_k=kc, cache_v=vc,
                                         cache_v_scale=torch.ones(2, 2))
    # the same call with every side input on the device runs
    qik.block_causal_flash_attention(q, k, v, Ld, torch.ones(1, 192, dtype=torch.bool, device=DEV), cache_k=kc,
                                     cache_v=vc, cache_v_scale=torch.ones(2, 2, device=DEV),
                                     debug_tiles=torch.zeros(4, dtype=torch.int32, device=DEV))
    torch.cuda.synchronize()


def test_cached_arguments_follow_new_pointers():
    """The wrapper keeps the argument struct per geometry: a second call of the same
    geometry with other tensors must read those tensors."""
    g = torch.Generator().manual_seed(962)
    L = torch.arange(300, dtype=torch.int32, device=DEV)
    outs = []
    for _ in range(2):
        q, k, v = (_rand((1, 300, 3, 128), g).to(DEV) for _ in range(3))
        out = qik.block_causal_flash_attention(q, k, v, L, None)
        _check(out, oa.attention_fp32(q.cpu(), k.cpu(), v.cpu(), L.cpu().numpy()), what="cached args")
        outs.append(out)
    assert not torch.equal(outs[0], outs[1])


# ---------------------------------------------------------------------------
# causal lengths and the visited-tile schedule: bit-exact

@pytest.mark.parametrize("seed", range(8))
def test_build_prefix_lengths_bit_exact(seed):
    rng = np.random.default_rng(seed)
    runs = [("text" if rng.random() < 0.5 else "img", int(rng.integers(1, 300))) for _ in range(int(rng.integers(1, 9)))]
    segs, pre = ol.make_segments(runs)
    S = pre + int(rng.integers(0, 500))
    got = qik.build_prefix_lengths(segs, pre, S, torch.device(DEV)).cpu().numpy()
    np.testing.assert_array_equal(got, ol.build_prefix_lengths(segs, pre, S))


def test_build_prefix_lengths_many_segments_and_slices():
    segs = [(i * 3, i * 3 + 3, i % 2 == 0) for i in range(150)]   # > 64 image runs per launch
    got = qik.build_prefix_lengths(segs, 400, 450, torch.device(DEV)).cpu().numpy()
    np.testing.assert_array_equal(got, ol.build_prefix_lengths(segs, 400, 450))
    segs = [(0, 4, True), (4, 100, False)]
    got = qik.build_prefix_lengths(segs, 50, 10, torch.device(DEV)).cpu().numpy()
    np.testing.assert_array_equal(got, ol.build_prefix_lengths(segs, 50, 10))


@pytest.mark.parametrize("name", wls.NAMES)
def test_visited_tiles_bit_exact(name):
    _flush(f"case schedule {name}")
    wl = wls.workload(name)
    bm, bn = qik.block_shape()
    nmb = -(-wl.SQ // bm)
    inp = wls.make_inputs(wl, seed=1, device=DEV, gen_device="cuda")
    dbg = torch.full((wl.B * wl.H * nmb,), -7, dtype=torch.int32, device=DEV)
    qik.block_causal_flash_attention(inp["query"], inp["key"], inp["value"], inp["prefix_lengths"], None,
                                     cache_k=inp["cache_k"], cache_v=inp["cache_v"],
                                     cache_v_scale=inp["cache_v_scale"], uniform_full=wl.uniform,
                                     debug_tiles=dbg)
    got = dbg.view(wl.B * wl.H, nmb).cpu().numpy()
    want = osch.exact_rule(wl.lengths(), wl.SQ, wl.P, wl.SN, bm, bn, wl.P > 0, wl.uniform)
    for bh in range(wl.B * wl.H):
        np.testing.assert_array_equal(got[bh], want)


# ---------------------------------------------------------------------------
# the five benchmark shapes

def _wl_run(wl, inp):
    return qik.block_causal_flash_attention(inp["query"], inp["key"], inp["value"], inp["prefix_lengths"], None,
                                            cache_k=inp["cache_k"], cache_v=inp["cache_v"],
                                            cache_v_scale=inp["cache_v_scale"], uniform_full=wl.uniform)


@pytest.mark.parametrize("name,heads", [("tiny", None), ("t2i_512", None), ("t2i_1024", None),
                                        ("edit_768", None), ("multiref_cfg", [0, 5, 17, 23])])
def test_benchmark_shapes_vs_oracle(name, heads):
    """CPU oracle on the same seeded inputs: every head of every shape up to the
    two headline ones (t2i_1024 and edit_768, 24 heads each), four heads of the
    last batch of multiref_cfg."""
    _flush(f"case shape {name}")
    wl = wls.workload(name)
    inp = wls.make_inputs(wl, seed=1000 * (wls.NAMES.index(name) + 1), device=DEV)
    out = _wl_run(wl, inp).float().cpu().numpy()
    cpu = {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}
    batches = None if wl.B == 1 else [wl.B - 1]
    ref = oa.attention_fp32(cpu["query"], cpu["key"], cpu["value"], wl.lengths(), None, cpu["cache_k"],
                            cpu["cache_v"], cpu["cache_v_scale"], heads=heads, batches=batches)
    hs = list(range(wl.H)) if heads is None else heads
    bs = list(range(wl.B)) if batches is None else batches
    o = out[bs][:, :, hs]
    r = ref[bs][:, :, hs]
    mx, mean = _check(o, r, what=name)
    _flush(f"  {name}: max {mx:.2e} mean {mean:.2e}")


def _torch_fp32_reference(wl, inp):
    """All heads on the GPU in fp32 (contiguous operands, explicit mask), one (b, h) at a time."""
    q = inp["query"].float()
    k = inp["key"].float()
    v = inp["value"].float()
    if wl.P > 0:
        kc = inp["cache_k"].float()
        if wl.v_fp8:
            vc = (inp["cache_v"].float() * inp["cache_v_scale"][:, None, :, None]).to(torch.bfloat16).float()
        else:
            vc = inp["cache_v"].float()
        k = torch.cat([kc, k], dim=1)
        v = torch.cat([vc, v], dim=1)
    L = inp["prefix_lengths"].long()
    mask = torch.arange(wl.KV, device=q.device)[None, :] <= L[:, None]
    out = torch.empty(q.shape, dtype=torch.float32, device=q.device)
    for b in range(wl.B):
        for h in range(wl.H):
            qt = q[b, :, h].contiguous()
            kt = k[b, :, h].contiguous()
            vt = v[b, :, h].contiguous()
            s = (qt @ kt.t().contiguous()) * (wl.D ** -0.5)
            s = s.masked_fill(~mask, float("-inf"))
            out[b, :, h] = torch.softmax(s, dim=-1) @ vt
    return out


@pytest.mark.parametrize("name", ["t2i_1024", "edit_768", "multiref_cfg"])
def test_benchmark_shapes_all_heads_vs_torch_fp32(name):
    _flush(f"case all heads {name}")
    wl = wls.workload(name)
    inp = wls.make_inputs(wl, seed=77, device=DEV, gen_device="cuda")
    out = _wl_run(wl, inp).float()
    ref = _torch_fp32_reference(wl, inp)
    d = (out - ref).abs()
    assert torch.isfinite(out).all()
    assert d.max().item() <= MAX_ABS and d.mean().item() <= MEAN_ABS, (d.max().item(), d.mean().item())


def test_multiref_all_heads_vs_host_explicit_mask_sdpa():
    """Every (b, h) of multiref_cfg (48) against the fp32 explicit-mask SDPA on
    the host (oracle.attention.CpuSdpaBaseline, which the oracle tests pin to
    attention_fp32), at the parity bar."""
    _flush("case multiref_cfg all 48 (b, h) vs host")
    wl = wls.workload("multiref_cfg")
    inp = wls.make_inputs(wl, seed=5000, device=DEV)
    out = _wl_run(wl, inp).float().cpu()
    cpu = {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}
    base = oa.CpuSdpaBaseline(cpu["query"], cpu["key"], cpu["value"], wl.lengths(), cpu["cache_k"],
                              cpu["cache_v"], cpu["cache_v_scale"])
    mx, total, n = 0.0, 0.0, 0
    for b in range(wl.B):
        for h in range(wl.H):
            d = (out[b, :, h] - base.run(b, h)).abs()
            mx = max(mx, d.max().item())
            total += d.sum().item()
            n += d.numel()
    _flush(f"  multiref_cfg all heads: max {mx:.2e} mean {total / n:.2e}")
    assert mx <= MAX_ABS and total / n <= MEAN_ABS, (mx, total / n)


@pytest.mark.parametrize("name,H", [("t2i_1024", 25), ("edit_768", 25), ("multiref_cfg", 13)])
def test_odd_head_counts_all_heads_vs_torch_fp32(name, H):
    """Head counts whose row blocks do not split evenly over the 8 XCDs (the
    workgroup -> row block remap then gives some XCDs one more row block), at
    full sequence length."""
    _flush(f"case odd heads {name} H={H}")
    wl = dataclasses.replace(wls.workload(name), H=H)
    inp = wls.make_inputs(wl, seed=91, device=DEV, gen_device="cuda")
    out = _wl_run(wl, inp).float()
    ref = _torch_fp32_reference(wl, inp)
    d = (out - ref).abs()
    assert torch.isfinite(out).all()
    assert d.max().item() <= MAX_ABS and d.mean().item() <= MEAN_ABS, (d.max().item(), d.mean().item())


@pytest.mark.parametrize("name,H", [("t2i_1024", 3), ("edit_768", 3), ("t2i_512", 3), ("multiref_cfg", 1),
                                    ("t2i_1024", 1), ("edit_768", 5)])
def test_one_gpu_head_share_all_heads_vs_torch_fp32(name, H):
    """One GPU's share of the heads (H/8 of 24 at the 1024px and 768px shapes:
    the two-group launch with every row block split over two CUs and merged
    through the workspace) against the torch fp32 reference."""
    _flush(f"case head share {name} H={H}")
    wl = dataclasses.replace(wls.workload(name), H=H)
    inp = wls.make_inputs(wl, seed=93, device=DEV, gen_device="cuda")
    out = _wl_run(wl, inp).float()
    ref = _torch_fp32_reference(wl, inp)
    d = (out - ref).abs()
    assert torch.isfinite(out).all()
    assert d.max().item() <= MAX_ABS and d.mean().item() <= MEAN_ABS, (d.max().item(), d.mean().item())


def test_layers_independent_seeds_size_independent_property():
    """Linearity in V at full 1024px size: attn(q,k,a*v1+b*v2) ~= a*attn(q,k,v1)+b*attn(q,k,v2)."""
    wl = wls.workload("t2i_1024")
    inp = wls.make_inputs(wl, seed=5, device=DEV, gen_device="cuda")
    q, k, v1, L = inp["query"], inp["key"], inp["value"], inp["prefix_lengths"]
    g = torch.Generator(device=DEV).manual_seed(6)
    v2 = torch.randn(v1.shape, generator=g, device=DEV).to(torch.bfloat16)
    vs = (0.5 * v1.float() + 0.25 * v2.float()).to(torch.bfloat16)
    o1 = qik.block_causal_flash_attention(q, k, v1, L, None).float()
    o2 = qik.block_causal_flash_attention(q, k, v2, L, None).float()
    o3 = qik.block_causal_flash_attention(q, k, vs, L, None).float()
    d = (o3 - (0.5 * o1 + 0.25 * o2)).abs()
    assert d.max().item() < 2e-2 and d.mean().item() < 2e-3


def _random_configs(n, seed):
    """Seeded argument sets over the whole entry point: head dims 32-256,
    bf16 / fp16, batch 1-2, 1-5 heads, no slab or a bf16 / fp16 / fp8-V slab
    of 1-599 keys, 1-699 fresh keys, 1-899 query rows (independent of the key
    count), causal lengths from block-causal segments, sorted or unsorted
    random values (some below -1 or past the last key), or uniform, an
    optional key_valid mask in runs, and both launches."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        D = int(rng.choice([32, 64, 128, 128, 128, 256]))
        fp16 = bool(rng.random() < 0.3)
        cache = str(rng.choice(["none", "same", "fp8"]))
        if fp16 and cache == "fp8":
            cache = "same"  # the reference dequantises fp8 V to bf16 (triton_attention.py:159)
        P = 0 if cache == "none" else int(rng.integers(1, 600))
        lengths = str(rng.choice(["segments", "sorted", "unsorted", "uniform"]))
        out.append(dict(seed=seed * 100 + i, D=D, fp16=fp16, B=int(rng.integers(1, 3)), H=int(rng.integers(1, 6)),
                        cache=cache, P=P, SN=int(rng.integers(1, 700)), SQ=int(rng.integers(1, 900)),
                        lengths=lengths, key_valid=bool(rng.random() < 0.35) and lengths != "uniform",
                        split=bool(rng.random() < 0.7)))
    return out


def _random_large_configs(n, seed):
    """As _random_configs, at sizes whose row blocks outnumber the CUs (the
    queued launch and its split last round): 8-24 heads, 1500-4499 query
    rows, up to 3999 fresh keys and a slab of up to 2999."""
    rng = np.random.default_rng(seed)
    out = _random_configs(n, seed)
    for c in out:
        c.update(H=int(rng.integers(8, 25)), SQ=int(rng.integers(1500, 4500)), SN=int(rng.integers(1, 4000)),
                 P=0 if c["cache"] == "none" else int(rng.integers(1, 3000)))
        c["heads"] = sorted({int(rng.integers(0, c["H"])) for _ in range(2)})
    return out


@pytest.mark.parametrize("cfg", _random_configs(64, 31) + _random_large_configs(8, 53),
                         ids=lambda c: f"s{c['seed']}" + ("L" if "heads" in c else ""))
def test_random_configurations_vs_oracle(cfg):
    """Each seeded argument set through block_causal_flash_attention against
    the fp32 explicit-mask oracle at the usual bar (at the large sizes, on two
    heads of every batch)."""
    _flush(f"case random {cfg}")
    rng = np.random.default_rng(cfg["seed"])
    g = torch.Generator().manual_seed(cfg["seed"])
    dtype = torch.float16 if cfg["fp16"] else torch.bfloat16
    B, H, D, P, SN, SQ = cfg["B"], cfg["H"], cfg["D"], cfg["P"], cfg["SN"], cfg["SQ"]
    KV = P + SN
    q = _rand((B, SQ, H, D), g, 1.0, dtype)
    kn, vn = (_rand((B, SN, H, D), g, 1.0, dtype) for _ in range(2))
    ck = cv = sc = None
    if P > 0:
        kp, vp = (_rand((B, P, H, D), g, 1.0, dtype) for _ in range(2))
        cache = qik.ContiguousKVCache(1, B, P + int(rng.integers(0, 100)), H, D, dtype=dtype,
                                      v_fp8=cfg["cache"] == "fp8", device=DEV)
        cache.get_layer(0).store(kp.to(DEV), vp.to(DEV))
        ck, cv, sc = cache.get_layer(0).views()
    if cfg["lengths"] == "segments":
        layout, left = [], SQ
        while left > 0:
            n = int(min(left, rng.integers(1, 300)))
            layout.append((str(rng.choice(["text", "img"])), n))
            left -= n
        segs, S0 = ol.make_segments(layout)
        L = (ol.build_prefix_lengths(segs, S0, SQ) + P).clip(max=KV - 1).astype(np.int32)
    elif cfg["lengths"] == "uniform":
        L = np.full(SQ, KV - 1, dtype=np.int32)
    else:
        L = rng.integers(-3, KV + 40, size=SQ).astype(np.int32)
        if cfg["lengths"] == "sorted":
            L = np.sort(L)
    kv = None
    if cfg["key_valid"]:
        kv = torch.ones(B, KV, dtype=torch.bool)
        for _ in range(int(rng.integers(1, 6))):
            b0, s0 = int(rng.integers(0, B)), int(rng.integers(0, KV))
            kv[b0, s0:s0 + int(rng.integers(1, 90))] = False
    out = qik.block_causal_flash_attention(
        q.to(DEV), kn.to(DEV), vn.to(DEV), torch.from_numpy(L).to(DEV), None if kv is None else kv.to(DEV),
        cache_k=ck, cache_v=cv, cache_v_scale=sc if cfg["cache"] == "fp8" else None,
        uniform_full=cfg["lengths"] == "uniform", split_tail=cfg["split"])
    torch.cuda.synchronize()
    assert out.dtype == dtype and out.shape == q.shape
    heads = cfg.get("heads")
    ref = oa.attention_fp32(q, kn, vn, L, kv, None if ck is None else ck.cpu(), None if cv is None else cv.cpu(),
                            sc.cpu() if cfg["cache"] == "fp8" else None, heads=heads)
    o = out.float().cpu().numpy()
    if heads is not None:
        o, ref = o[:, :, heads], ref[:, :, heads]
    _check(o, ref, what=f"random {cfg['seed']}")
