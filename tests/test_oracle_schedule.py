"""Oracle: KV-tile schedules (CPU)."""

import numpy as np
import pytest

from oracle import schedule as osch

import qwen_image_kernel_amd.workloads as wls

# Per-(b,h) tile totals of the five benchmark shapes, reference rule / exact rule,
# at (BM, BN) = (128, 64), (128, 128), (256, 64), (256, 128).  These were
# computed independently of this oracle from the reference formula
# (triton_attention.py:95, 117-121).
TOTALS = {
    "tiny": [(15, 15), (9, 9), (10, 10), (6, 6)],
    "t2i_512": [(147, 146), (74, 73), (90, 90), (45, 45)],
    "t2i_1024": [(2184, 2182), (1093, 1091), (1093, 1092), (547, 546)],
    "edit_768": [(3328, 3328), (1664, 1664), (1664, 1664), (832, 832)],
    "multiref_cfg": [(4608, 4582), (2317, 2291), (2305, 2292), (1159, 1146)],
}
GEOMS = [(128, 64), (128, 128), (256, 64), (256, 128)]


@pytest.mark.parametrize("name", list(TOTALS))
def test_schedule_totals_match_independent_count(name):
    wl = wls.workload(name)
    for (bm, bn), (ref_total, exact_total) in zip(GEOMS, TOTALS[name]):
        args = (wl.lengths(), wl.SQ, wl.P, wl.SN, bm, bn, wl.P > 0, wl.uniform)
        assert int(osch.reference_rule(*args).sum()) == ref_total, (bm, bn)
        assert int(osch.exact_rule(*args).sum()) == exact_total, (bm, bn)


def _random_case(rng):
    SQ = int(rng.integers(1, 300))
    P = int(rng.integers(0, 3)) * int(rng.integers(1, 200))
    SN = int(rng.integers(1, 300))
    L = rng.integers(-1, P + SN + 5, size=SQ).astype(np.int32)
    if rng.random() < 0.5:
        L = np.sort(L)
    return L, SQ, P, SN


@pytest.mark.parametrize("seed", range(60))
def test_exact_rule_is_brute_force_and_subset_of_reference(seed):
    rng = np.random.default_rng(seed)
    L, SQ, P, SN = _random_case(rng)
    for bm, bn in [(128, 64), (64, 32), (256, 128)]:
        for uniform in (False, True):
            args = (L, SQ, P, SN, bm, bn, P > 0, uniform)
            ex = osch.exact_rule(*args)
            np.testing.assert_array_equal(ex, osch.brute_force(*args))
            ref = osch.reference_rule(*args)
            assert (ref >= ex).all()
            # every tile the reference runs beyond the exact rule is fully masked
            KV = P + SN
            lmax = osch.block_lmax(L, SQ, P, SN, bm, uniform)
            exact_tiles = osch.visited_tiles(L, SQ, P, SN, bm, bn, P > 0, uniform, rule="exact")
            ref_tiles = osch.visited_tiles(L, SQ, P, SN, bm, bn, P > 0, uniform, rule="reference")
            segs = osch.segments(P, SN, bn, P > 0)
            for m in range(len(ref_tiles)):
                assert set(exact_tiles[m]) <= set(ref_tiles[m])
                for ph, t in set(ref_tiles[m]) - set(exact_tiles[m]):
                    seg_len, start, _ = segs[ph]
                    first_key = start + t * bn
                    assert first_key > lmax[m] or t * bn >= seg_len or first_key >= KV
