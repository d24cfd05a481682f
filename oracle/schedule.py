"""KV-tile schedules per row block.  Test infrastructure only.

Both rules work on segment-local tiles: with a cache, segment 0 is the slab
(keys [0, P)) and segment 1 the fresh keys ([P, P+SN)); tile t of a segment
covers its local keys [t*BN, (t+1)*BN) (triton_attention.py:97-124).  L_max of
a row block is the largest L over its live rows (P+SN-1 when uniform); dead
rows load -1 (:79-83).
"""

from __future__ import annotations

import numpy as np


def cdiv(a: int, b: int) -> int:
    return -(-a // b)


def block_lmax(L, SQ: int, P: int, SN: int, BM: int, uniform: bool) -> list[int]:
    out = []
    for m in range(cdiv(SQ, BM)):
        if uniform:
            out.append(P + SN - 1)
        else:
            rows = np.asarray(L[m * BM : min(SQ, (m + 1) * BM)])
            out.append(int(rows.max()) if rows.size else -1)
    return out


def segments(P: int, SN: int, BN: int, has_cache: bool):
    """(seg_len, seg_start, first_tile) per phase, as triton_attention.py:97-115."""
    if has_cache:
        return [(P, 0, 0), (SN, P, cdiv(P, BN))]
    return [(SN, 0, 0)]


def reference_rule(L, SQ, P, SN, BM, BN, has_cache, uniform) -> np.ndarray:
    """Tiles the Triton kernel runs per row block (triton_attention.py:95, 117-121).

    hi = cdiv(L_max + 1, BN); each phase runs max(0, min(cdiv(seg_len, BN), hi - first + 1))
    tiles.  It can run one extra, fully masked tile per phase (the "+1").
    Pinned by: the per-config tile totals computed independently from the
    reference formula (tests/test_oracle_schedule.py).
    """
    out = []
    for lmax in block_lmax(L, SQ, P, SN, BM, uniform):
        hi = cdiv(lmax + 1, BN)
        n = 0
        for seg_len, _start, first in segments(P, SN, BN, has_cache):
            n += max(0, min(cdiv(seg_len, BN), hi - first + 1))
        out.append(n)
    return np.array(out, dtype=np.int32)


def exact_rule(L, SQ, P, SN, BM, BN, has_cache, uniform) -> np.ndarray:
    """Tiles holding at least one allowed key: tile t runs iff seg_start + t*BN <= L_max.

    Pinned by: ``brute_force`` (any allowed (row, key) pair in the tile) and by
    being the reference rule minus its fully masked extra tiles.
    """
    out = []
    for lmax in block_lmax(L, SQ, P, SN, BM, uniform):
        n = 0
        for seg_len, start, _first in segments(P, SN, BN, has_cache):
            if lmax >= start:
                n += min(cdiv(seg_len, BN), (lmax - start) // BN + 1)
        out.append(n)
    return np.array(out, dtype=np.int32)


def brute_force(L, SQ, P, SN, BM, BN, has_cache, uniform) -> np.ndarray:
    """Count tiles that contain an allowed (row, key) pair, by enumeration."""
    KV = P + SN
    Lv = np.full(SQ, KV - 1) if uniform else np.asarray(L[:SQ])
    out = []
    for m in range(cdiv(SQ, BM)):
        rows = Lv[m * BM : min(SQ, (m + 1) * BM)]
        n = 0
        for seg_len, start, _first in segments(P, SN, BN, has_cache):
            for t in range(cdiv(seg_len, BN)):
                keys = start + np.arange(t * BN, min(seg_len, (t + 1) * BN))
                if (keys[None, :] <= rows[:, None]).any():
                    n += 1
        out.append(n)
    return np.array(out, dtype=np.int32)


def visited_tiles(L, SQ, P, SN, BM, BN, has_cache, uniform, rule: str = "reference"):
    """List of (phase, local_tile) per row block in visiting order, for either rule."""
    lmaxes = block_lmax(L, SQ, P, SN, BM, uniform)
    res = []
    for lmax in lmaxes:
        tiles = []
        hi = cdiv(lmax + 1, BN)
        for ph, (seg_len, start, first) in enumerate(segments(P, SN, BN, has_cache)):
            if rule == "reference":
                run = max(0, min(cdiv(seg_len, BN), hi - first + 1))
            else:
                run = 0 if lmax < start else min(cdiv(seg_len, BN), (lmax - start) // BN + 1)
            tiles += [(ph, t) for t in range(run)]
        res.append(tiles)
    return res
