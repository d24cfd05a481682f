"""GPU parity of qik_attn_fwd_noalloc, the attention entry point that allocates nothing.

Its workspace is a static device array inside the library (one per device),
whose control words the call clears with a fill kernel.  Checked through the
C ABI against qik_attn_fwd_ws (same kernel and work plan, so bit-identical)
on two calls in a row, the second with a smaller input (the array then holds
the first call's slots), and against the CPU oracle at the attention bar.
Launches of more than half and at most one row block per CU take the
two-group form without a workspace: there the entry point does not touch the
array (the tiny layout, with fewer row blocks, splits them over two CUs and
uses it).
"""

import ctypes
import dataclasses

import numpy as np
import pytest
import torch

from oracle import attention as oa

import qwen_image_kernel_amd.workloads as wls
from qwen_image_kernel_amd import _lib
from qwen_image_kernel_amd.attention import make_args

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MEAN_ABS = 2e-3


def _workload(name):
    """A benchmark workload, or ``t2i_512_b2``: the 512px layer with two batches
    (432 row blocks: split through the workspace)."""
    if name == "t2i_512_b2":
        return dataclasses.replace(wls.workload("t2i_512"), name=name, B=2)
    return wls.workload(name)


def _args(wl, inp, out):
    L = None if wl.uniform else inp["prefix_lengths"]
    return make_args(inp["query"], inp["key"], inp["value"], L, None, out, inp["cache_k"], inp["cache_v"],
                     inp["cache_v_scale"], wl.uniform)


def _ws_call(lib, wl, inp, stream):
    out = torch.empty_like(inp["query"])
    a = _args(wl, inp, out)
    nb = ctypes.c_int64()
    _lib.check(lib.qik_attn_workspace_size(ctypes.byref(a), ctypes.byref(nb)), "qik_attn_workspace_size")
    assert 0 <= nb.value <= _lib.ATTN_SCRATCH_BYTES
    ws = torch.zeros(max(nb.value, 1), dtype=torch.uint8, device="cuda")
    _lib.check(lib.qik_attn_fwd_ws(ctypes.byref(a), ws.data_ptr(), nb.value, stream), "qik_attn_fwd_ws")
    torch.cuda.synchronize()
    return out


def _noalloc_call(lib, wl, inp, stream):
    out = torch.full_like(inp["query"], float("nan"))
    a = _args(wl, inp, out)
    _lib.check(lib.qik_attn_fwd_noalloc(ctypes.byref(a), stream), "qik_attn_fwd_noalloc")
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("first,second", [("edit_768", "tiny"), ("t2i_1024", "t2i_512_b2"), ("t2i_512_b2", "t2i_512")])
def test_noalloc_matches_workspace_launch(first, second):
    lib = _lib.load()
    torch.cuda.set_device(0)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for i, name in enumerate((first, second)):
        print(f"noalloc case {name} (call {i + 1} of 2)", flush=True)
        wl = _workload(name)
        inp = wls.make_inputs(wl, seed=900 + i, device="cuda", gen_device="cuda")
        want = _ws_call(lib, wl, inp, stream)
        got = _noalloc_call(lib, wl, inp, stream)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), name
        if wl.SQ * wl.KV * wl.H <= 2e8:
            # the CPU oracle at the attention bar, where it finishes in seconds
            ref = oa.attention_fp32(inp["query"].cpu(), inp["key"].cpu(), inp["value"].cpu(),
                                    wl.lengths(), None,
                                    None if inp["cache_k"] is None else inp["cache_k"].cpu(),
                                    None if inp["cache_v"] is None else inp["cache_v"].cpu(),
                                    None if inp["cache_v_scale"] is None else inp["cache_v_scale"].cpu())
            d = np.abs(got.float().cpu().numpy() - ref)
            assert d.max() <= MAX_ABS and d.mean() <= MEAN_ABS, (name, d.max(), d.mean())


def test_noalloc_repeated_calls_are_bit_identical():
    """The control words are cleared per call and left zero by the launch: three calls agree."""
    lib = _lib.load()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    wl = _workload("t2i_512_b2")
    inp = wls.make_inputs(wl, seed=911, device="cuda", gen_device="cuda")
    outs = [_noalloc_call(lib, wl, inp, stream) for _ in range(3)]
    for o in outs[1:]:
        assert torch.equal(o.view(torch.int16), outs[0].view(torch.int16))
