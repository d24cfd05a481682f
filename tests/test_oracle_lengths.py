"""Oracle: causal-length array L and the stock multi-pass decomposition (CPU)."""

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import lengths as ol


def _random_layout(rng, n_runs):
    runs = []
    for _ in range(n_runs):
        runs.append(("text" if rng.random() < 0.5 else "img", int(rng.integers(1, 40))))
    return runs


@pytest.mark.parametrize("seed", range(40))
def test_lengths_equal_mask_definition(seed):
    """kv <= L[q] reproduces (q >= kv) | same_image_block, target rows see all keys."""
    rng = np.random.default_rng(seed)
    segs, pre = ol.make_segments(_random_layout(rng, int(rng.integers(1, 7))))
    S = pre + int(rng.integers(0, 50))
    L = ol.build_prefix_lengths(segs, pre, S)
    assert L.dtype == np.int32
    np.testing.assert_array_equal(ol.mask_from_lengths(L, S), ol.segment_mask(segs, S, pre))


def test_lengths_baseline_layouts():
    """L of the benchmark layouts, written out by hand."""
    segs, n = ol.make_segments([("text", 64), ("img", 256)])
    L = ol.build_prefix_lengths(segs, n, n)
    np.testing.assert_array_equal(L, np.r_[np.arange(64), np.full(256, 319)])
    segs, n = ol.make_segments([("text", 256), ("img", 4096)])
    L = ol.build_prefix_lengths(segs, n, n)
    np.testing.assert_array_equal(L, np.r_[np.arange(256), np.full(4096, 4351)])
    segs, p = ol.make_segments([("text", 256), ("img", 1024), ("img", 1024), ("img", 1024)])
    L = ol.build_prefix_lengths(segs, p, p + 4096)
    want = np.r_[np.arange(256), np.full(1024, 1279), np.full(1024, 2303), np.full(1024, 3327), np.full(4096, 7423)]
    np.testing.assert_array_equal(L, want)


def test_lengths_python_slice_semantics():
    """Out-of-range and empty runs behave like the reference's slice assignments."""
    # an image run past the end fills end-1 = 99 on the rows that exist; prefix 50 > S assigns nothing
    L = ol.build_prefix_lengths([(0, 4, True), (4, 100, False)], 50, 10)
    np.testing.assert_array_equal(L, np.r_[np.arange(4), np.full(6, 99)])
    L = ol.build_prefix_lengths([(0, 4, True)], -3, 10)
    np.testing.assert_array_equal(L, np.r_[np.arange(7), np.full(3, 9)])
    L = ol.build_prefix_lengths([(3, 3, False)], 10, 10)
    np.testing.assert_array_equal(L, np.arange(10))


@pytest.mark.parametrize(
    "layout,padding,batch",
    [
        ([("text", 48), ("img", 64)], False, 1),
        ([("text", 16), ("img", 40), ("text", 8), ("img", 24)], False, 1),
        ([("text", 32), ("img", 48)], True, 1),
        ([("text", 24), ("img", 30)], False, 2),
    ],
)
def test_stock_multipass_equals_length_oracle(layout, padding, batch):
    """The per-segment SDPA decomposition (never uses L) equals the L-based oracle.

    Layouts are scaled-down versions of tests/test_attention.py:112-115; the
    target here is a trailing run of 20 full-attention rows.
    """
    segs, pre = ol.make_segments(layout)
    S = pre + 20
    g = torch.Generator().manual_seed(7)
    H, D = 2, 64
    q, k, v = (torch.randn(batch, S, H, D, generator=g).to(torch.bfloat16) for _ in range(3))
    kv = None
    if padding:
        first_text_end = next(e for s, e, t in segs if t)
        kv = torch.ones(batch, S, dtype=torch.bool)
        kv[:, first_text_end - 5:first_text_end] = False
    L = ol.build_prefix_lengths(segs, pre, S)
    ref = oa.attention_fp32(q, k, v, L, kv)
    stock = ol.stock_multipass_sdpa(q, k, v, segs, pre, kv).numpy()
    np.testing.assert_allclose(ref, stock, atol=2e-6, rtol=0)
