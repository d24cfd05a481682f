"""Workgroup -> work assignment of the attention launch (qik_attn_work_map, host only).

The kernel and this export share one function (csrc/qik_plan.h).  Checked here:
every row block is run exactly once whole or by exactly two pieces (0 and 1)
that share one workspace group; groups are dense in [0, ngroups); the unsplit
assignment is the contiguous per-XCD layout; the split one runs whole rounds
first, then the first (big) piece of every left-over row block, then their
second pieces; and the workspace size the library reports follows from
ngroups.
"""

import ctypes

import numpy as np
import pytest

from qwen_image_kernel_amd import _lib

NXCD = 8


def work_map(n, nmb, sx, split):
    """(item, piece, group, ngroups, ns) per workgroup of the launch."""
    lib = _lib.load()
    grid, ngroups, ns = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int32()
    assert lib.qik_attn_work_map(n, nmb, sx, split, None, None, None, 0, ctypes.byref(grid),
                                 ctypes.byref(ngroups), ctypes.byref(ns)) == 0
    g = grid.value
    item, piece, group = (np.full(max(g, 1), -7, dtype=np.int32) for _ in range(3))
    st = lib.qik_attn_work_map(n, nmb, sx, split, item.ctypes.data, piece.ctypes.data, group.ctypes.data, g,
                               ctypes.byref(grid), ctypes.byref(ngroups), None)
    assert st == 0
    return item[:g], piece[:g], group[:g], ngroups.value, ns.value


def xcd_items(n):
    per, rem = divmod(n, NXCD)
    return [per + (1 if x < rem else 0) for x in range(NXCD)]


CASES = [
    # (items, row blocks per head, workgroups per XCD at once)
    (816, 34, 64),     # 24 heads x 4352 rows on 256 CUs, 2 per CU
    (768, 32, 64),     # 24 heads x 4096 rows
    (2784, 58, 64),    # 2 x 24 heads x 7424 rows
    (216, 9, 64),      # 24 heads x 1152 rows: one partial round
    (12, 3, 64),       # 4 heads x 320 rows
    (850, 34, 64),     # 25 heads: uneven XCD runs
    (377, 29, 64),     # 13 heads x 3712 rows
    (1, 1, 64),
    (7, 7, 3),
    (1024, 32, 64),    # exactly 2 full rounds: nothing to split
    (1000, 40, 30),    # harvested part: 240 CUs
]


@pytest.mark.parametrize("n,nmb,sx", CASES)
@pytest.mark.parametrize("split", [0, 1])
def test_every_row_block_runs_once(n, nmb, sx, split):
    item, piece, group, ngroups, ns = work_map(n, nmb, sx, split)
    assert len(item) % NXCD == 0
    assert ns == (1 if (not split or ngroups == 0) else 2)
    whole = np.zeros(n, dtype=np.int64)
    pieces = {}
    for it, pc, gr in zip(item, piece, group):
        if it < 0:
            assert pc == 0 and gr == -1
            continue
        assert 0 <= it < n
        if gr < 0:
            assert pc == 0
            whole[it] += 1
        else:
            assert 0 <= gr < ngroups and 0 <= pc < ns
            pieces.setdefault(it, []).append((pc, gr))
    for it, ps in pieces.items():
        assert sorted(pc for pc, _ in ps) == list(range(ns)), it
        assert len({gr for _, gr in ps}) == 1, it
        assert whole[it] == 0, it
    covered = whole + np.array([1 if i in pieces else 0 for i in range(n)])
    assert (covered == 1).all()
    assert sorted(ps[0][1] for ps in pieces.values()) == list(range(ngroups))
    if not split:
        assert ngroups == 0


@pytest.mark.parametrize("n,nmb,sx", CASES)
def test_unsplit_map_is_contiguous_per_xcd(n, nmb, sx):
    """Workgroup bid runs on XCD bid % 8; XCD x holds a contiguous run of row blocks, in order."""
    item, _, _, _, _ = work_map(n, nmb, sx, 0)
    start = 0
    for x, q in enumerate(xcd_items(n)):
        mine = item[x::NXCD]
        assert list(mine[:q]) == list(range(start, start + q))
        assert (mine[q:] == -1).all()
        start += q


@pytest.mark.parametrize("n,nmb,sx", CASES)
def test_split_tail_fits_the_slots(n, nmb, sx):
    """Per XCD: whole rounds of sx row blocks first, then the left-over row blocks' first
    pieces, then their second pieces in the same order; the XCD keeps the same row
    blocks as without the split."""
    item, piece, group, ngroups, ns = work_map(n, nmb, sx, 1)
    item0, _, _, _, _ = work_map(n, nmb, sx, 0)
    total = 0
    for x, q in enumerate(xcd_items(n)):
        full = sx * (q // sx) if q >= sx else 0
        r = q - full
        mine, px, gx = item[x::NXCD], piece[x::NXCD], group[x::NXCD]
        live = mine[mine >= 0]
        assert len(live) == full + ns * r
        assert (gx[:full] == -1).all() and (gx[full:len(live)] >= 0).all()
        if r:
            assert list(px[full:len(live)]) == [0] * r + [1] * r
            assert list(mine[full:full + r]) == list(mine[full + r:full + 2 * r])
            assert list(gx[full:full + r]) == list(gx[full + r:full + 2 * r])
        assert set(live.tolist()) == set(item0[x::NXCD][:q].tolist())
        assert r < sx
        total += r
    assert total == ngroups


def test_piece_counts_of_the_benchmark_shapes():
    """256 CUs x 2 workgroups: 24 heads x 4352 rows leave 38 row blocks per XCD after one
    round of 64, 24 x 4096 rows leave 32; each is split in two."""
    assert work_map(816, 34, 64, 1)[3:] == (8 * 38, 2)
    assert work_map(768, 32, 64, 1)[3:] == (8 * 32, 2)
    assert work_map(1024, 32, 64, 1)[3:] == (0, 1)


def test_pair_rank_major_order_puts_light_row_blocks_last():
    """24 heads x 34 row blocks: each XCD's run is 3 whole heads, walked rank-major over
    its first two heads (heaviest row block of both first), then the third head
    heaviest first, so the split tail holds the lightest ranks of the last head and no
    more than two heads are interleaved anywhere."""
    n, nmb, sx = 816, 34, 64
    item, piece, _, _, _ = work_map(n, nmb, sx, 1)
    for x in range(NXCD):
        mine = item[x::NXCD]
        live = [i for i, pc in zip(mine, piece[x::NXCD]) if i >= 0 and pc == 0]
        assert len(live) == 3 * nmb and len(set(live)) == 3 * nmb
        heads = sorted({i // nmb for i in live})
        assert len(heads) == 3
        first, last = live[:2 * nmb], live[2 * nmb:]
        assert {i // nmb for i in first} == set(heads[:2]) and {i // nmb for i in last} == {heads[2]}
        # item i % nmb == rank (0 = heaviest row block): non-decreasing within each group
        assert [i % nmb for i in first] == sorted(i % nmb for i in first)
        assert [i % nmb for i in last] == list(range(nmb))
        # the two heads of the pair alternate
        assert all(first[2 * r] // nmb != first[2 * r + 1] // nmb for r in range(nmb))


@pytest.mark.parametrize("heads", [1, 2, 3, 4, 5, 6])
def test_pair_order_visits_every_item_once(heads):
    """Any number of whole heads per XCD: the split plan hands every row block out
    exactly once (as one unit or as both pieces)."""
    nmb = 9
    n = NXCD * heads * nmb
    item, piece, group, grid, ns = work_map(n, nmb, 64, 1)
    seen = {}
    for it, pc in zip(item, piece):
        if it >= 0:
            seen.setdefault(it, set()).add(pc)
    assert sorted(seen) == list(range(n))
    assert all(s == {0} or s == set(range(ns)) for s in seen.values())


def test_workspace_size_follows_from_groups():
    """qik_attn_workspace_size needs a device (CU count): checked on the GPU.  Here the
    size formula: the fixed 32 KiB of control words (16 queue words + one per group),
    then ns slots per group of BM x D fp32 accumulators plus (m, l) per thread."""
    _, _, _, ngroups, ns = work_map(816, 34, 64, 1)
    slot128 = 128 * 128 * 4 + 256 * 8
    want = 32768 + ngroups * ns * slot128
    assert 40e6 < want < 42e6
    assert 16 + ngroups <= 32768 // 4


def test_work_map_rejects_bad_arguments():
    lib = _lib.load()
    g, p = ctypes.c_int64(), ctypes.c_int64()
    assert lib.qik_attn_work_map(10, 0, 64, 1, None, None, None, 0, ctypes.byref(g), ctypes.byref(p), None) == -5
    assert lib.qik_attn_work_map(10, 5, 0, 1, None, None, None, 0, ctypes.byref(g), ctypes.byref(p), None) == -5
    assert lib.qik_attn_work_map(-1, 5, 64, 1, None, None, None, 0, ctypes.byref(g), ctypes.byref(p), None) == -5
    assert lib.qik_attn_work_map(10, 5, 64, 1, None, None, None, 0, None, ctypes.byref(p), None) == -1
    buf = np.zeros(4, dtype=np.int32)
    # a buffer shorter than the grid
    assert lib.qik_attn_work_map(100, 5, 64, 1, buf.ctypes.data, buf.ctypes.data, buf.ctypes.data, 4,
                                 ctypes.byref(g), ctypes.byref(p), None) == -5


def work_map_xcds(n, nmb, sx, split, nx):
    lib = _lib.load()
    grid, ngroups, ns = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int32()
    assert lib.qik_attn_work_map_xcds(n, nmb, sx, split, nx, None, None, None, 0, ctypes.byref(grid),
                                      ctypes.byref(ngroups), ctypes.byref(ns)) == 0
    g = grid.value
    item, piece, group = (np.full(max(g, 1), -7, dtype=np.int32) for _ in range(3))
    assert lib.qik_attn_work_map_xcds(n, nmb, sx, split, nx, item.ctypes.data, piece.ctypes.data,
                                      group.ctypes.data, g, ctypes.byref(grid), ctypes.byref(ngroups), None) == 0
    return item[:g], piece[:g], group[:g], ngroups.value, ns.value


@pytest.mark.parametrize("nx", [1, 2, 3, 4, 6, 8, 16, 32])
@pytest.mark.parametrize("n,nmb,sx", [(816, 34, 64), (768, 32, 64), (216, 9, 64), (12, 3, 64), (850, 34, 30),
                                      (2784, 58, 16)])
@pytest.mark.parametrize("split", [0, 1])
def test_plan_for_another_xcd_count_runs_every_row_block_once(n, nmb, sx, split, nx):
    """A device that reports another XCD count (a partitioned MI355X shows 1,
    2 or 4) gets a plan over that many queues: still every row block whole
    exactly once or as both pieces of one group, groups dense, the grid a
    multiple of the XCD count."""
    item, piece, group, ngroups, ns = work_map_xcds(n, nmb, sx, split, nx)
    assert len(item) % nx == 0
    whole = np.zeros(n, dtype=np.int64)
    pieces = {}
    for it, pc, gr in zip(item, piece, group):
        if it < 0:
            continue
        if gr < 0:
            whole[it] += 1
        else:
            assert 0 <= gr < ngroups
            pieces.setdefault(it, []).append((pc, gr))
    for it, ps in pieces.items():
        assert sorted(pc for pc, _ in ps) == list(range(ns)) and len({gr for _, gr in ps}) == 1
        assert whole[it] == 0
    assert sorted({gr for ps in pieces.values() for _, gr in ps}) == list(range(ngroups))
    covered = whole + np.array([1 if i in pieces else 0 for i in range(n)])
    assert (covered == 1).all()
    if nx == NXCD:
        same = work_map(n, nmb, sx, split)
        np.testing.assert_array_equal(same[0], item)


def test_work_map_xcds_rejects_bad_counts():
    lib = _lib.load()
    grid, ngroups = ctypes.c_int64(), ctypes.c_int64()
    for nx in (0, -1, 33):
        assert lib.qik_attn_work_map_xcds(100, 10, 8, 1, nx, None, None, None, 0, ctypes.byref(grid),
                                          ctypes.byref(ngroups), None) == -5
