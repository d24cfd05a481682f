"""Randomised GPU parity sweep over the kernel's instances and launch forms.

Each seeded case draws the batch, heads, head dim (64 / 128), dtype (bf16 /
fp16), the slab (none, bf16/fp16 V, or fp8 V with per-(b, h) scales; fp8 V
with bf16 only, as in the reference), its length P, the fresh key count SN,
the query rows (SN, or P + SN: every row against [slab, fresh]), the causal
lengths (uniform, causal over the last keys with some empty rows, or random
in [-1, KV-1]) and an optional key_valid mask.  block_causal_flash_attention
runs once with the split launch and once with one workgroup per row block;
both must be within max-abs 2e-2 and mean-abs 2e-3 of the fp32 oracle
(triton_attention.py:266-293).  Sizes stay small enough for the oracle to
take seconds for the whole sweep.
"""

import numpy as np
import pytest
import torch

from oracle import attention as oa

import qwen_image_kernel_amd as qik

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MEAN_ABS = 2e-3
DEV = "cuda"
N_CASES = 24


def _draw(i):
    rng = np.random.default_rng(7000 + i)
    B = int(rng.integers(1, 3))
    H = int(rng.integers(1, 6))
    D = int(rng.choice([64, 128]))
    dtype = torch.float16 if rng.random() < 0.3 else torch.bfloat16
    kinds = ["none", "plain"] + (["fp8"] if dtype == torch.bfloat16 else [])
    slab = str(rng.choice(kinds))
    P = int(rng.integers(1, 700)) if slab != "none" else 0
    SN = int(rng.integers(1, 700))
    SQ = SN if (slab == "none" or rng.random() < 0.5) else P + SN
    KV = P + SN
    mode = str(rng.choice(["uniform", "causal", "random"]))
    if mode == "uniform":
        L = np.full(SQ, KV - 1, dtype=np.int32)
    elif mode == "causal":
        L = np.minimum(KV - 1, (KV - SQ) + np.arange(SQ)).astype(np.int32)
        L[rng.random(SQ) < 0.05] = -1
    else:
        L = rng.integers(-1, KV, size=SQ).astype(np.int32)
    key_valid = None
    if rng.random() < 0.35:
        key_valid = rng.random((B, KV)) > 0.1
    return dict(B=B, H=H, D=D, dtype=dtype, slab=slab, P=P, SN=SN, SQ=SQ, mode=mode, L=L,
                key_valid=key_valid, seed=int(rng.integers(1 << 30)))


@pytest.mark.parametrize("i", range(N_CASES))
def test_random_case_vs_oracle(i):
    c = _draw(i)
    desc = {k: v for k, v in c.items() if k not in ("L", "key_valid")}
    desc["key_valid"] = c["key_valid"] is not None
    print(f"case random {i}: {desc}", flush=True)
    B, H, D, P, SN, SQ, dt = c["B"], c["H"], c["D"], c["P"], c["SN"], c["SQ"], c["dtype"]
    g = torch.Generator().manual_seed(c["seed"])
    q, kn, vn = ((torch.randn(B, n, H, D, generator=g)).to(dt) for n in (SQ, SN, SN))
    ck = cv = sc = None
    kw = {}
    if c["slab"] != "none":
        k0, v0 = ((torch.randn(B, P, H, D, generator=g)).to(dt) for _ in range(2))
        cache = qik.ContiguousKVCache(1, B, P + 16, H, D, v_fp8=c["slab"] == "fp8", device=DEV, dtype=dt)
        layer = cache.get_layer(0)
        layer.store(k0.to(DEV), v0.to(DEV))
        ck, cv, sc = layer.views()
        kw = dict(cache_k=ck, cache_v=cv)
        if c["slab"] == "fp8":
            kw["cache_v_scale"] = sc
    Ld = torch.from_numpy(c["L"]).to(DEV)
    kv = None if c["key_valid"] is None else torch.from_numpy(c["key_valid"]).to(DEV)
    uniform = c["mode"] == "uniform"
    ref = oa.attention_fp32(q, kn, vn, c["L"], c["key_valid"],
                            None if ck is None else ck.cpu(), None if cv is None else cv.cpu(),
                            sc.cpu() if c["slab"] == "fp8" else None)
    for split in (True, False):
        out = qik.block_causal_flash_attention(q.to(DEV), kn.to(DEV), vn.to(DEV), Ld, kv, uniform_full=uniform,
                                               split_tail=split, **kw)
        o = out.float().cpu().numpy()
        assert np.isfinite(o).all(), (i, split)
        d = np.abs(o - ref)
        assert d.max() <= MAX_ABS and d.mean() <= MEAN_ABS, (i, split, float(d.max()), float(d.mean()))
