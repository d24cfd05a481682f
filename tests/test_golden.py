"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle recomputes every stored result from the stored inputs
(bit-exact for integers and bf16 bit patterns, 1e-6 for fp32).
GPU: the HIP kernel reproduces the stored outputs within the path's tolerance.
"""

import os

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import fp8 as of
from oracle import lengths as ol
from oracle import schedule as osch

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FIXTURES = sorted(f for f in os.listdir(HERE) if f.endswith(".npz"))


def bf16(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16)


def bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def load(name):
    z = np.load(os.path.join(HERE, name), allow_pickle=False)
    return {k: z[k] for k in z.files}


def inputs(f):
    q, k, v = bf16(f["q"]), bf16(f["k"]), bf16(f["v"])
    kv = f.get("key_valid")
    cache = None
    if "cache_k" in f:
        cv8 = torch.from_numpy(np.ascontiguousarray(f["cache_v_codes"].transpose(0, 2, 1, 3))).view(torch.float8_e4m3fn)
        cache = (bf16(f["cache_k"]), cv8, torch.from_numpy(f["cache_v_scale"]))
    return q, k, v, kv, cache


def test_fixtures_present():
    assert len(FIXTURES) >= 3


@pytest.mark.parametrize("name", FIXTURES)
def test_oracle_reproduces_fixture(name):
    f = load(name)
    q, k, v, kv, cache = inputs(f)
    L = f["L"]
    if "segments" in f:
        segs = [tuple(int(x) for x in s) for s in f["segments"]]
        np.testing.assert_array_equal(ol.build_prefix_lengths(segs, int(f["prefix_len"]), q.shape[1]), L)
        S = q.shape[1]
        np.testing.assert_array_equal(osch.reference_rule(L, S, 0, S, 128, 64, False, False), f["sched_reference"])
        np.testing.assert_array_equal(osch.exact_rule(L, S, 0, S, 128, 64, False, False), f["sched_exact"])
        args = (q, k, v, L, kv)
        em = oa.flash_emulation(*args)
    else:
        ck, cv8, sc = cache
        codes, scale = of.quantize_per_head(bf16(f["cache_v_bf16"]).float().numpy())
        np.testing.assert_array_equal(codes, f["cache_v_codes"])
        np.testing.assert_array_equal(scale, f["cache_v_scale"])
        P, SN = ck.shape[1], k.shape[1]
        np.testing.assert_array_equal(osch.reference_rule(L, SN, P, SN, 128, 64, True, True), f["sched_reference"])
        np.testing.assert_array_equal(osch.exact_rule(L, SN, P, SN, 128, 64, True, True), f["sched_exact"])
        args = (q, k, v, L, None, ck, cv8, sc)
        em = oa.flash_emulation(*args, uniform=True)
    np.testing.assert_allclose(oa.attention_fp32(*args), f["out_fp32"], atol=1e-6, rtol=0)
    np.testing.assert_allclose(oa.attention_fp64(*args), f["out_fp64"], atol=1e-6, rtol=0)
    np.testing.assert_array_equal(em, bits_to_f32(f["out_emulation_bf16"]))


@pytest.mark.gpu
@pytest.mark.parametrize("name", FIXTURES)
def test_kernel_matches_fixture(name):
    import qwen_image_kernel_amd as qik

    f = load(name)
    q, k, v, kv, cache = inputs(f)
    dev = "cuda"
    L = torch.from_numpy(f["L"]).to(dev)
    kw = {}
    if cache is not None:
        ck, cv8, sc = cache
        kw = dict(cache_k=ck.to(dev), cache_v=cv8.to(dev), cache_v_scale=sc.to(dev), uniform_full=True)
    out = qik.block_causal_flash_attention(q.to(dev), k.to(dev), v.to(dev), L,
                                           None if kv is None else torch.from_numpy(kv).to(dev), **kw)
    o = out.float().cpu().numpy()
    d = np.abs(o - f["out_fp32"])
    assert d.max() <= 2e-2 and d.mean() <= 2e-3, (d.max(), d.mean())
    de = np.abs(o - bits_to_f32(f["out_emulation_bf16"]))
    assert de.max() <= 4e-3, de.max()
