"""GPU parity of the split launches of qik_attn_fwd_ws.

Three forms, chosen by the number of row blocks n:
* n above the CU count: each row block of the launch's last, partly filled
  round runs as two pieces over its KV tiles, which meet in a workspace, and
  the launch's resident workgroups pull their units from per-XCD queues;
* n at most the CU count: one workgroup of two 4-wave groups per row block,
  the groups taking the two halves of its KV tiles and merging in LDS (no
  workspace);
* n at most half the CU count (one GPU's share of the heads): the same
  two-group workgroups, but every row block split into two equal pieces on two
  CUs that meet in a workspace.
Checked here against the CPU oracle (same bars as the unsplit kernel: max-abs
2e-2, mean-abs 2e-3), against the unsplit launch, run to run (bit-identical),
with rows that see no key in one piece or in any, with garbage in the slots,
with the control words back at zero after every launch, under HIP-graph
replay, and the host-side workspace checks.
"""

import ctypes
import dataclasses

import numpy as np
import pytest
import torch

from oracle import attention as oa

import qwen_image_kernel_amd as qik
import qwen_image_kernel_amd.workloads as wls
from qwen_image_kernel_amd import _lib
from qwen_image_kernel_amd.attention import make_args

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MEAN_ABS = 2e-3
DEV = "cuda"


def _flush(msg):
    print(msg, flush=True)


def _rand(shape, gen, scale=1.0):
    return (torch.randn(*shape, generator=gen) * scale).to(torch.bfloat16)


def _check(out, ref, what):
    o = out.float().cpu().numpy()
    d = np.abs(o - ref)
    assert np.isfinite(o).all(), what
    assert d.max() <= MAX_ABS and d.mean() <= MEAN_ABS, (what, d.max(), d.mean())


def _ws_bytes(args):
    nbytes = ctypes.c_int64()
    _lib.check(_lib.load().qik_attn_workspace_size(ctypes.byref(args), ctypes.byref(nbytes)), "ws size")
    return nbytes.value


def _plan(n_items, nmb):
    """(ngroups, pieces) of the split plan on this device: two workgroups per CU."""
    sx = 2 * torch.cuda.get_device_properties(0).multi_processor_count // 8
    grid, ngroups, ns = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int32()
    _lib.check(_lib.load().qik_attn_work_map(n_items, nmb, sx, 1, None, None, None, 0, ctypes.byref(grid),
                                             ctypes.byref(ngroups), ctypes.byref(ns)), "work map")
    return ngroups.value, ns.value


CTL_BYTES = _lib.WS_CTL_BYTES


def _ctl_bytes(ngroups):
    return CTL_BYTES


def _cus():
    return torch.cuda.get_device_properties(0).multi_processor_count


def _uses_workspace(n):
    """The launch of n row blocks merges pieces through the workspace: above the
    CU count, or at most half of it."""
    return n > _cus() or 2 * n <= _cus()


def _n_groups(args):
    """Row blocks of one launch on this device that merge through the workspace,
    checked against the workspace size; 0 for the two-group form without it."""
    nmb = -(-args.SQ // 128)
    n = args.B * args.H * nmb
    if not _uses_workspace(n):
        assert _ws_bytes(args) == 0
        return 0
    if n <= _cus():
        # one two-group workgroup per CU: the plan of cus / 8 slots per XCD
        sx = _cus() // 8
        grid, ngroups, ns = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int32()
        _lib.check(_lib.load().qik_attn_work_map(n, nmb, sx, 1, None, None, None, 0, ctypes.byref(grid),
                                                 ctypes.byref(ngroups), ctypes.byref(ns)), "work map")
        ngroups, ns = ngroups.value, ns.value
        assert ngroups == n and ns == 2
    else:
        ngroups, ns = _plan(n, nmb)
    slot = 128 * args.D * 4 + 256 * 8
    assert _ws_bytes(args) == _ctl_bytes(ngroups) + ngroups * ns * slot
    return ngroups


def _workload(name):
    """A benchmark workload, or ``t2i_512_b2``: the 512px layer with two batches
    (432 row blocks, more than the CUs: the queue and the workspace merge)."""
    if name == "t2i_512_b2":
        return dataclasses.replace(wls.workload("t2i_512"), name=name, B=2)
    if name.endswith("_h3"):
        return dataclasses.replace(wls.workload(name[:-3]), name=name, H=3)
    return wls.workload(name)


def _prefill(name, seed):
    wl = _workload(name)
    inp = wls.make_inputs(wl, seed=seed, device=DEV, gen_device="cuda")
    return wl, inp


def _run(wl, inp, split):
    return qik.block_causal_flash_attention(inp["query"], inp["key"], inp["value"], inp["prefix_lengths"], None,
                                            cache_k=inp["cache_k"], cache_v=inp["cache_v"],
                                            cache_v_scale=inp["cache_v_scale"], uniform_full=wl.uniform,
                                            split_tail=split)


def test_workspace_size_matches_the_device_plan():
    """24 heads x 4352 rows: the row blocks left after whole rounds are split."""
    wl = wls.workload("t2i_1024")
    q = torch.empty(1, wl.SQ, wl.H, wl.D, dtype=torch.bfloat16, device=DEV)
    L = torch.zeros(wl.SQ, dtype=torch.int32, device=DEV)
    a = make_args(q, q, q, L, None, q, None, None, None, False)
    assert _n_groups(a) > 0


@pytest.mark.parametrize("name,workspace", [("t2i_512", False), ("t2i_512_b2", True), ("multiref_cfg", True),
                                            ("t2i_1024_h3", True), ("edit_768_h3", True)])
def test_split_vs_unsplit_vs_oracle(name, workspace):
    _flush(f"case split {name}")
    wl, inp = _prefill(name, seed=11)
    a = _run(wl, inp, True)
    b = _run(wl, inp, False)
    torch.cuda.synchronize()
    args = make_args(inp["query"], inp["key"], inp["value"], inp["prefix_lengths"], None, a,
                     inp["cache_k"], inp["cache_v"], inp["cache_v_scale"], wl.uniform)
    assert (_n_groups(args) > 0) == workspace
    d = (a.float() - b.float()).abs()
    # both within the oracle bar below; between them only the accumulation order differs
    assert d.max().item() <= 2 * MAX_ABS and d.mean().item() <= 5e-4, (d.max().item(), d.mean().item())
    heads = list(range(wl.H)) if wl.B == 1 and (wl.P == 0 or wl.H <= 4) else [3, 17]
    slab = {} if wl.P == 0 else dict(cache_k=inp["cache_k"].cpu(), cache_v=inp["cache_v"].cpu(),
                                     cache_v_scale=inp["cache_v_scale"].cpu())
    ref = oa.attention_fp32(inp["query"].cpu(), inp["key"].cpu(), inp["value"].cpu(), wl.lengths(), None,
                            heads=heads, **slab)
    for h in heads:
        _check(a[:, :, h], ref[:, :, h], f"{name} h{h} split")
        _check(b[:, :, h], ref[:, :, h], f"{name} h{h} unsplit")


@pytest.mark.parametrize("H", [4, 32])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [64, 128])
def test_split_dtypes_and_head_dims(dtype, D, H):
    """128 text + 1024 image rows over 1152 keys: 18 KV tiles per image row block, so
    every image row block of this one-round launch is split and merged (both pieces
    non-empty), in both element types and both head dims; 4 heads (36 row blocks)
    take two-group workgroups with every row block split over two CUs, 32 heads
    (288) the queue; both merge through the workspace."""
    _flush(f"case split dtype={dtype} D={D} H={H}")
    g = torch.Generator().manual_seed(30 + D + H)
    S = 1152
    q, k, v = ((torch.randn(1, S, H, D, generator=g)).to(dtype) for _ in range(3))
    L = np.arange(S, dtype=np.int32)
    L[128:] = S - 1
    Ld = torch.from_numpy(L).to(DEV)
    out = qik.block_causal_flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), Ld, None)
    args = make_args(q.to(DEV), k.to(DEV), v.to(DEV), Ld, None, out, None, None, None, False)
    assert (_n_groups(args) > 0) == _uses_workspace(H * 9)
    assert out.dtype == dtype
    _check(out, oa.attention_fp32(q, k, v, L), f"{dtype} D={D}")
    again = qik.block_causal_flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), Ld, None)
    assert torch.equal(out, again)


@pytest.mark.parametrize("H", [3, 48])
def test_split_decode_against_fp8_slab(H):
    """Decode of 640 target rows against a 512-row fp8 slab + 640 fresh keys (18 tiles,
    the first 8 from the slab): the split row blocks mix slab and fresh tiles (3 heads:
    the two-group form; 48 heads, 480 row blocks: the workspace merge)."""
    _flush(f"case split fp8 slab decode H={H}")
    g = torch.Generator().manual_seed(40 + H)
    B, P, SN, D = 2, 512, 640, 128
    pk, pv = ((torch.randn(B, P, H, D, generator=g)).to(torch.bfloat16) for _ in range(2))
    q, k, v = ((torch.randn(B, SN, H, D, generator=g)).to(torch.bfloat16) for _ in range(3))
    cache = qik.ContiguousKVCache(1, B, P + 64, H, D, v_fp8=True, device=DEV)
    cache.get_layer(0).store(pk.to(DEV), pv.to(DEV))
    kc, vc, sc = cache.get_layer(0).views()
    L = torch.full((SN,), P + SN - 1, dtype=torch.int32, device=DEV)
    out = qik.block_causal_flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), L, None, cache_k=kc, cache_v=vc,
                                           cache_v_scale=sc, uniform_full=True)
    args = make_args(q.to(DEV), k.to(DEV), v.to(DEV), None, None, out, kc, vc, sc, True)
    assert (_n_groups(args) > 0) == _uses_workspace(B * H * 5)
    ref = oa.attention_fp32(q, k, v, L.cpu().numpy(), None, kc.cpu(), vc.cpu(), sc.cpu())
    _check(out, ref, "fp8 slab decode")


@pytest.mark.parametrize("name", ["t2i_512", "t2i_512_b2", "t2i_1024_h3"])
def test_split_is_bit_identical_run_to_run(name):
    """Whichever piece arrives last merges, in piece order: the result never changes."""
    _flush(f"case split determinism {name}")
    wl, inp = _prefill(name, seed=12)
    outs = [_run(wl, inp, True) for _ in range(4)]
    for o in outs[1:]:
        assert torch.equal(outs[0], o)


@pytest.mark.parametrize("H", [3, 48])
def test_rows_without_keys_in_one_piece_or_any(H):
    """1024 keys = 16 tiles, two pieces of 8: rows with L < 512 see nothing in piece 1,
    rows with L = -1 nothing at all (zeros); key_valid clears piece 0 for batch 1
    (3 heads: two-group workgroups, every row block split over two CUs; 48 heads:
    the queue and the workspace merge)."""
    _flush(f"case split empty halves H={H}")
    g = torch.Generator().manual_seed(13)
    B, SQ, SN, D = 2, 640, 1024, 128
    q, k, v = (_rand((B, n, H, D), g) for n in (SQ, SN, SN))
    rng = np.random.default_rng(13)
    L = rng.integers(-1, SN, size=SQ).astype(np.int32)
    L[:128] = rng.integers(-1, 511, size=128)       # row block 0: never past piece 0
    L[128:256] = -1                                  # row block 1: empty rows
    L[256:384:2] = SN - 1                            # row block 2: alternating full / short
    L[257:384:2] = 40
    valid = np.ones((B, SN), dtype=bool)
    valid[1, :512] = False                           # batch 1: piece 0 sees no valid key
    valid[0, rng.integers(0, SN, 100)] = False
    kv = torch.from_numpy(valid)
    Ld = torch.from_numpy(L).to(DEV)
    a = qik.block_causal_flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), Ld, kv.to(DEV))
    b = qik.block_causal_flash_attention(q.to(DEV), k.to(DEV), v.to(DEV), Ld, kv.to(DEV), split_tail=False)
    args = make_args(q.to(DEV), k.to(DEV), v.to(DEV), Ld, kv.to(DEV).to(torch.uint8), a, None, None, None, False)
    assert (_n_groups(args) > 0) == _uses_workspace(B * H * 5)
    ref = oa.attention_fp32(q, k, v, L, kv.numpy())
    _check(a, ref, "split")
    _check(b, ref, "unsplit")
    assert (a[:, 128:256].float() == 0).all()


def _direct(inp, wl, ws, nbytes):
    out = torch.empty_like(inp["query"])
    args = make_args(inp["query"], inp["key"], inp["value"], inp["prefix_lengths"], None, out,
                     inp["cache_k"], inp["cache_v"], inp["cache_v_scale"], wl.uniform)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    st = _lib.load().qik_attn_fwd_ws(ctypes.byref(args), None if ws is None else ws.data_ptr(), nbytes, stream)
    return st, out, args


@pytest.mark.parametrize("name", ["t2i_512_b2", "edit_768", "edit_768_h3"])
def test_workspace_control_words_return_to_zero(name):
    """Only the control words must start at zero: the slots may hold anything.  Every
    launch leaves the control words zero again, so the next launch reuses the buffer."""
    _flush(f"case split workspace contents {name}")
    wl, inp = _prefill(name, seed=14)
    want = _run(wl, inp, True)
    _, _, args = _direct(inp, wl, None, 0)
    n = _ws_bytes(args)
    nmb = -(-wl.SQ // 128)
    assert n > 0
    ctl = _ctl_bytes(_plan(wl.B * wl.H * nmb, nmb)[0])
    g = torch.Generator(device=DEV).manual_seed(15)
    ws = torch.randint(0, 256, (n,), generator=g, device=DEV, dtype=torch.int32).to(torch.uint8)
    ws[:ctl] = 0
    for i in range(3):
        st, out, _ = _direct(inp, wl, ws, n)
        assert st == 0
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"launch {i}"
        assert (ws[:ctl] == 0).all(), f"control words left nonzero after launch {i}"


def test_one_workspace_across_shapes():
    """One workspace, never re-zeroed, through shapes whose split plans differ (a small
    ragged batch, the 1152-row layer, the multi-reference slab decode): every launch
    equals a launch on a fresh workspace.  The control words sit in a fixed region,
    so one shape's slot data never lands where the next keeps its counters."""
    _flush("case split workspace across shapes")
    cases = [_prefill("tiny", seed=20), _prefill("t2i_512_b2", seed=21), _prefill("multiref_cfg", seed=22),
             _prefill("t2i_512_b2", seed=23), _prefill("tiny", seed=24), _prefill("t2i_512", seed=25)]
    sizes = [_ws_bytes(_direct(inp, wl, None, 0)[2]) for wl, inp in cases]
    shared = torch.zeros(max(sizes), dtype=torch.uint8, device=DEV)
    for (wl, inp), n in zip(cases, sizes):
        fresh = torch.zeros(n, dtype=torch.uint8, device=DEV)
        st0, want, _ = _direct(inp, wl, fresh, n)
        st1, got, _ = _direct(inp, wl, shared, n)
        assert st0 == 0 and st1 == 0
        torch.cuda.synchronize()
        assert torch.equal(got, want), wl.name
        assert (shared[:CTL_BYTES] == 0).all(), wl.name


def test_workspace_checks_are_host_side():
    wl, inp = _prefill("t2i_512_b2", seed=16)
    _, _, args = _direct(inp, wl, None, 0)
    n = _ws_bytes(args)
    ws = torch.zeros(n + 512, dtype=torch.uint8, device=DEV)
    assert _direct(inp, wl, None, 0)[0] == -12                   # missing
    assert _direct(inp, wl, ws, n - 1)[0] == -12                 # too small
    assert _direct(inp, wl, ws[16:], n)[0] == -12                # not 256-byte aligned
    assert _direct(inp, wl, ws, n)[0] == 0
    torch.cuda.synchronize()


@pytest.mark.parametrize("name", ["t2i_512", "t2i_512_b2", "edit_768_h3"])
def test_split_under_graph_replay(name):
    """Captured once, replayed several times with eager launches (on the cached
    workspace) between replays: every replay equals the eager result."""
    _flush(f"case split graph {name}")
    wl, inp = _prefill(name, seed=17)
    want = _run(wl, inp, True)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        _run(wl, inp, True)  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = _run(wl, inp, True)
    for i in range(4):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {i}"
        eager = _run(wl, inp, True)   # eager launches share nothing with the graph's workspace
        torch.cuda.synchronize()
        assert torch.equal(eager, want)
