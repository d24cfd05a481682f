"""Write the small golden fixtures under tests/golden/ from the CPU oracle.

    python tests/golden/make_golden.py

Each fixture holds seeded inputs (bf16 as uint16 bit patterns, fp8 as uint8
codes), the causal-length array, the tile schedules of both rules at
(BM, BN) = (128, 64), and the expected outputs: the fp32 explicit-mask oracle,
the float64 brute force (stored rounded to float32) and the tile-loop emulation
(bf16, stored as uint16 bit patterns).  The reference ships
no fixtures of its own for this path; these pin the oracle against regressions
and give the GPU tests fixed expected values.
"""

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import attention as oa  # noqa: E402
from oracle import fp8 as of  # noqa: E402
from oracle import lengths as ol  # noqa: E402
from oracle import schedule as osch  # noqa: E402


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def f32_bf16_bits(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).__rshift__(16).astype(np.uint16)


def rand(shape, g):
    return torch.randn(*shape, generator=g).to(torch.bfloat16)


def prefill_case(name, runs, extra, B, H, D, seed, padding=False):
    segs, pre = ol.make_segments(runs)
    S = pre + extra
    g = torch.Generator().manual_seed(seed)
    q, k, v = rand((B, S, H, D), g), rand((B, S, H, D), g), rand((B, S, H, D), g)
    kv = None
    if padding:
        first_text_end = next(e for s, e, t in segs if t)
        kv = np.ones((B, S), dtype=bool)
        kv[:, first_text_end - 5:first_text_end] = False
        kv[B - 1, 1] = False
    L = ol.build_prefix_lengths(segs, pre, S)
    out32 = oa.attention_fp32(q, k, v, L, kv)
    out64 = oa.attention_fp64(q, k, v, L, kv)
    em = oa.flash_emulation(q, k, v, L, kv)
    arrs = dict(q=bf16_bits(q), k=bf16_bits(k), v=bf16_bits(v), L=L, segments=np.array(segs, dtype=np.int32),
                prefix_len=np.int32(pre), out_fp32=out32, out_fp64=out64.astype(np.float32),
                out_emulation_bf16=f32_bf16_bits(em),
                sched_reference=osch.reference_rule(L, S, 0, S, 128, 64, False, False),
                sched_exact=osch.exact_rule(L, S, 0, S, 128, 64, False, False))
    if kv is not None:
        arrs["key_valid"] = kv
    np.savez_compressed(os.path.join(HERE, name), **arrs)
    return arrs


def decode_case(name, P, SN, B, H, D, seed):
    g = torch.Generator().manual_seed(seed)
    q, kn, vn = rand((B, SN, H, D), g), rand((B, SN, H, D), g), rand((B, SN, H, D), g)
    ck, cv = rand((B, P, H, D), g), rand((B, P, H, D), g)
    codes, scale = of.quantize_per_head(cv.float().numpy())           # [B, H, P, D], [B, H]
    cv8 = torch.from_numpy(np.ascontiguousarray(codes.transpose(0, 2, 1, 3))).view(torch.float8_e4m3fn)
    L = np.full(SN, P + SN - 1, dtype=np.int32)
    out32 = oa.attention_fp32(q, kn, vn, L, None, ck, cv8, torch.from_numpy(scale))
    out64 = oa.attention_fp64(q, kn, vn, L, None, ck, cv8, torch.from_numpy(scale))
    em = oa.flash_emulation(q, kn, vn, L, None, ck, cv8, torch.from_numpy(scale), uniform=True)
    arrs = dict(q=bf16_bits(q), k=bf16_bits(kn), v=bf16_bits(vn), cache_k=bf16_bits(ck), cache_v_bf16=bf16_bits(cv),
                cache_v_codes=codes, cache_v_scale=scale, L=L, out_fp32=out32, out_fp64=out64.astype(np.float32),
                out_emulation_bf16=f32_bf16_bits(em),
                sched_reference=osch.reference_rule(L, SN, P, SN, 128, 64, True, True),
                sched_exact=osch.exact_rule(L, SN, P, SN, 128, 64, True, True))
    np.savez_compressed(os.path.join(HERE, name), **arrs)
    return arrs


def main():
    prefill_case("prefill_text_image_target.npz", [("text", 40), ("img", 70), ("text", 9), ("img", 30)], 43,
                 B=1, H=1, D=128, seed=11)
    prefill_case("prefill_padded_batch2_d64.npz", [("text", 33), ("img", 50)], 20, B=2, H=2, D=64, seed=12,
                 padding=True)
    decode_case("decode_fp8_slab.npz", P=100, SN=70, B=1, H=2, D=128, seed=13)
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")


if __name__ == "__main__":
    main()
