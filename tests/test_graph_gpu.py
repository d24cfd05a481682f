"""A layer's device steps captured in one HIP graph and replayed.

QK-RMSNorm+RoPE of the prefix and target tokens (qik_rms_rope), the slab
store of the prefix with fp8 V (qik_slab_store_ws), and the target rows'
attention against [slab, fresh] (qik_attn_fwd_ws), the decode flow of
processors.py:97-112, are captured once on a side stream after an eager
warm-up on that stream (which creates the workspaces), then replayed several
times with eager runs of the same steps between replays.  Every replay must
equal the eager result bit for bit: the steps are deterministic, none records
a memset, and every workspace comes back in the state the next launch expects.
"""

import pytest
import torch

import qwen_image_kernel_amd as qik

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _inputs(seed=41):
    g = torch.Generator(device=DEV).manual_seed(seed)
    B, P, SN, H, D = 1, 320, 256, 4, 128
    q, k, v = (torch.randn(B, SN, H, D, generator=g, device=DEV).to(torch.bfloat16) for _ in range(3))
    kp, vp = (torch.randn(B, P, H, D, generator=g, device=DEV).to(torch.bfloat16) for _ in range(2))
    w = torch.randn(D, generator=g, device=DEV) * 0.2 + 1.0
    S = P + SN
    inv = 1.0 / (10000 ** (torch.arange(0, D, 2, device=DEV).float() / D))
    ang = torch.outer(torch.arange(S, device=DEV).float(), inv)
    freqs = torch.polar(torch.ones_like(ang), ang)
    cache = qik.ContiguousKVCache(1, B, P + 16, H, D, v_fp8=True, device=DEV)
    return dict(q=q, k=k, v=v, kp=kp, vp=vp, w=w, freqs=freqs, cache=cache, P=P, SN=SN)


def _layer(x):
    """RMSNorm+RoPE of the prefix keys and the target q/k, slab store, decode attention."""
    P, SN = x["P"], x["SN"]
    kp = qik.fused_rms_norm_rope(x["kp"], x["w"], x["freqs"][:P], 1e-6)
    q = qik.fused_rms_norm_rope(x["q"], x["w"], x["freqs"][P:], 1e-6)
    k = qik.fused_rms_norm_rope(x["k"], x["w"], x["freqs"][P:], 1e-6)
    layer = x["cache"].get_layer(0)
    layer.store(kp, x["vp"])
    k8, v8, sc = layer.views()
    L = torch.full((SN,), P + SN - 1, dtype=torch.int32, device=DEV)
    out = qik.block_causal_flash_attention(q, k, x["v"], L, None, cache_k=k8, cache_v=v8, cache_v_scale=sc,
                                           uniform_full=True)
    return out, kp, q, k, sc


def test_layer_steps_under_graph_replay():
    print("case layer graph", flush=True)
    x = _inputs()
    want = [t.clone() for t in _layer(x)]
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        _layer(x)  # warm-up on the capture stream: its workspaces exist before capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        got = _layer(x)
    for i in range(4):
        for t in got:
            t.zero_()
        x["cache"].k_buf.zero_()
        graph.replay()
        torch.cuda.synchronize()
        for name, a, b in zip(("out", "k_prefix", "q", "k", "v_scale"), got, want):
            assert torch.equal(a, b), f"replay {i}: {name}"
        eager = _layer(x)  # eager steps on the default stream between replays
        torch.cuda.synchronize()
        assert torch.equal(eager[0], want[0]), f"eager after replay {i}"


def test_fp8_linear_under_graph_replay():
    """FP8Linear (quantiser + GEMM, and the K-split GEMM with its workspace)
    captured in a graph: every replay equals the eager result, with eager
    calls of the same module between replays."""
    print("case fp8 linear graph", flush=True)
    torch.manual_seed(7)
    mods = [qik.FP8Linear.from_linear(torch.nn.Linear(K, N, bias=True, dtype=torch.bfloat16, device=DEV))
            for K, N in ((3072, 3072), (12288, 3072))]
    xs = [torch.randn(256, m.in_features, device=DEV, dtype=torch.bfloat16) for m in mods]
    want = [m(x).clone() for m, x in zip(mods, xs)]
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for m, x in zip(mods, xs):
            m(x)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        got = [m(x) for m, x in zip(mods, xs)]
    for i in range(4):
        for t in got:
            t.zero_()
        graph.replay()
        torch.cuda.synchronize()
        for j, (a, b) in enumerate(zip(got, want)):
            assert torch.equal(a, b), f"replay {i}: linear {j}"
        eager = [m(x) for m, x in zip(mods, xs)]
        torch.cuda.synchronize()
        for a, b in zip(eager, want):
            assert torch.equal(a, b), f"eager after replay {i}"
