"""GPU parity of the steps beside the attention call.

* ``fused_rms_norm_rope`` (qik_rms_rope) against the fp32 restatement
  oracle/rms_rope.py bit for bit, and against the stock composition within the
  reference's bar (tests/test_fused.py:21-47, 4e-2);
* ``ContiguousKVCache.store`` (qik_slab_store) against the torch ops of
  kv_cache.py:30-45 run on the same device and against the oracle's
  quantisation, bit for bit;
* ``QwenImage21KernelProcessor`` driven like the reference drives its
  processor (processors.py:50-126), with a stand-in ``attn`` object, against
  the stock composition: torch RMSNorm + RoPE, fp32 explicit-mask attention.
"""

import ctypes

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import fp8 as of
from oracle import lengths as ol
from oracle import rms_rope as orr

import qwen_image_kernel_amd as qik
from qwen_image_kernel_amd import _lib

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _flush(msg):
    print(msg, flush=True)


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.int16).cpu().numpy()


# ---------------------------------------------------------------------------
# RMSNorm + RoPE


def _rope_case(B, S, H, D, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(B, S, H, D, generator=g) * 0.7).to(dtype)
    w = torch.randn(D, generator=g) * 0.3
    return x, w, orr.rope_freqs(S, D)


def _rope_oracle(x, w, freqs, eps, dtype="bf16"):
    return orr.rms_norm_rope(x.float().numpy(), w.numpy(), freqs.real.float().numpy(), freqs.imag.float().numpy(),
                             eps, dtype)


@pytest.mark.parametrize("B,S,H,D,dtype", [
    (1, 300, 32, 128, torch.bfloat16),   # tests/test_fused.py:37
    (2, 77, 24, 128, torch.bfloat16),
    (1, 130, 5, 64, torch.bfloat16),
    (1, 65, 3, 128, torch.float16),
    (2, 9, 1, 128, torch.bfloat16),      # one head: a thread's next row is 16 positions on
    (4, 3, 2, 128, torch.bfloat16),      # 16 rows on crosses whole batches (b carry)
    (1, 70, 6, 32, torch.bfloat16),      # the other head dims
    (2, 33, 3, 256, torch.float16),
])
def test_rms_rope_bit_exact_vs_oracle(B, S, H, D, dtype):
    _flush(f"case rms_rope {B}x{S}x{H}x{D} {dtype}")
    x, w, freqs = _rope_case(B, S, H, D, seed=S + D, dtype=dtype)
    out = qik.fused_rms_norm_rope(x.to(DEV), w.to(DEV), freqs.to(DEV), 1e-6)
    want = _rope_oracle(x, w, freqs, 1e-6, "bf16" if dtype == torch.bfloat16 else "fp16")
    np.testing.assert_array_equal(out.float().cpu().numpy(), want)
    ref = orr.stock_rms_norm_rope(x.to(DEV), w.to(DEV), freqs.to(DEV), 1e-6)
    assert (out.float() - ref.float()).abs().max().item() < 4e-2


def test_rms_rope_reads_fused_qkv_views_in_place():
    """q/k as strided slices of a fused QKV output (processors.py:65-70)."""
    _flush("case rms_rope strided")
    B, S, H, D = 2, 96, 6, 128
    g = torch.Generator().manual_seed(11)
    qkv = (torch.randn(B, S, 3 * H * D, generator=g) * 0.5).to(torch.bfloat16).to(DEV)
    q, k, v = qkv.unflatten(-1, (3 * H, D)).chunk(3, dim=-2)
    assert not q.is_contiguous()
    w = (torch.randn(D, generator=g) * 0.3).to(DEV)
    freqs = orr.rope_freqs(S, D).to(DEV)
    for t in (q, k):
        got = qik.fused_rms_norm_rope(t, w, freqs, 1e-6)
        want = qik.fused_rms_norm_rope(t.contiguous(), w, freqs, 1e-6)
        np.testing.assert_array_equal(_bits(got), _bits(want))


def test_rms_rope_rejects_bad_freqs():
    x = torch.zeros(1, 8, 2, 128, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError):
        qik.fused_rms_norm_rope(x, torch.ones(128, device=DEV), orr.rope_freqs(7, 128).to(DEV), 1e-6)


# ---------------------------------------------------------------------------
# slab store


def _torch_store(k, v, v_fp8):
    """kv_cache.py:36-42 on the device, as the reference runs it."""
    kt = k.transpose(1, 2).contiguous()
    if not v_fp8:
        return kt, v.transpose(1, 2).contiguous(), None
    vt = v.transpose(1, 2).float()
    scale = vt.abs().amax(dim=(2, 3)).float() / 448.0
    scale = scale.clamp_min(1e-12)
    vq = (vt / scale[:, :, None, None]).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return kt, vq, scale


@pytest.mark.parametrize("B,P,H,D,v_fp8", [(1, 2560, 24, 128, True), (2, 333, 5, 128, True),
                                           (1, 100, 3, 64, True), (2, 257, 4, 128, False),
                                           (2, 150, 3, 32, True), (1, 90, 2, 256, True), (1, 65, 2, 256, False)])
def test_slab_store_bit_exact_vs_torch_ops(B, P, H, D, v_fp8):
    _flush(f"case slab store B={B} P={P} H={H} D={D} fp8={v_fp8}")
    g = torch.Generator().manual_seed(P + H)
    k = torch.randn(B, P, H, D, generator=g).to(torch.bfloat16).to(DEV)
    v = (torch.randn(B, P, H, D, generator=g) * 3).to(torch.bfloat16).to(DEV)
    cache = qik.ContiguousKVCache(3, B, P + 272, H, D, v_fp8=v_fp8, device=DEV)
    cache.get_layer(2).store(k, v)
    kv, vv, sc = cache.get_layer(2).views()
    kt, vt, st = _torch_store(k, v, v_fp8)
    np.testing.assert_array_equal(_bits(kv.transpose(1, 2)), _bits(kt))
    if v_fp8:
        np.testing.assert_array_equal(vv.transpose(1, 2).contiguous().view(torch.uint8).cpu().numpy(),
                                      vt.view(torch.uint8).cpu().numpy())
        np.testing.assert_array_equal(sc.cpu().numpy(), st.cpu().numpy())
        codes, scale = of.quantize_per_head(v.float().cpu().numpy())
        np.testing.assert_array_equal(sc.cpu().numpy(), scale)
        np.testing.assert_array_equal(vv.transpose(1, 2).contiguous().view(torch.uint8).cpu().numpy(), codes)
    else:
        np.testing.assert_array_equal(_bits(vv.transpose(1, 2)), _bits(vt))
    assert cache.lengths[2].item() == P and cache._host_lengths[2] == P
    # the other layers are untouched
    assert cache.lengths[0].item() == 0


@pytest.mark.parametrize("B,P,H,D", [(1, 2560, 24, 128), (2, 333, 5, 128), (1, 100, 3, 64), (3, 31, 2, 128)])
def test_slab_store_two_and_three_launch_forms_agree(B, P, H, D):
    """qik_slab_store_ws (workspace of chunk scales, two launches) against
    qik_slab_store (atomic scale, three launches): the same bytes, with a reused
    workspace holding the previous call's (or garbage) values."""
    _flush(f"case slab store forms B={B} P={P} H={H} D={D}")
    lib = _lib.load()
    g = torch.Generator().manual_seed(900 + P)
    k = torch.randn(B, P, H, D, generator=g).to(torch.bfloat16).to(DEV)
    v = (torch.randn(B, P, H, D, generator=g) * 5).to(torch.bfloat16).to(DEV)
    caches = [qik.ContiguousKVCache(1, B, P + 16, H, D, v_fp8=True, device=DEV) for _ in range(2)]
    stream = torch.cuda.current_stream().cuda_stream
    a3, keep3 = caches[0].get_layer(0).store_args(k, v, P)
    assert lib.qik_slab_store(ctypes.byref(a3), stream) == 0
    a2, keep2 = caches[1].get_layer(0).store_args(k, v, P)
    n = ctypes.c_int64()
    assert lib.qik_slab_store_workspace_size(ctypes.byref(a2), ctypes.byref(n)) == 0
    ws = torch.full((n.value // 4,), 1e30, dtype=torch.float32, device=DEV)     # garbage in the workspace
    for _ in range(2):
        assert lib.qik_slab_store_ws(ctypes.byref(a2), ws.data_ptr(), n.value, stream) == 0
    torch.cuda.synchronize()
    for buf in ("k_buf", "v_buf", "v_scale"):
        x, y = getattr(caches[0], buf), getattr(caches[1], buf)
        if buf == "k_buf":
            x, y = x[..., :P, :], y[..., :P, :]
        elif buf == "v_buf":
            x, y = x[..., :P, :].contiguous().view(torch.uint8), y[..., :P, :].contiguous().view(torch.uint8)
        np.testing.assert_array_equal(_bits(x) if buf == "k_buf" else x.cpu().numpy(),
                                      _bits(y) if buf == "k_buf" else y.cpu().numpy(), err_msg=buf)
    del keep3, keep2


def test_slab_store_every_bf16_value_under_many_scales():
    """The quantiser divides through the scale's reciprocal and one fma
    correction; against torch's IEEE division (the reference's v / scale,
    kv_cache.py:38-40) on the same device and against the oracle: every finite
    bf16 value with |v| <= amax in each of 24 heads whose planted amax spans
    1e-30 .. 1e30 (powers of two, 448, 1e-12-floor heads included)."""
    _flush("case slab store every bf16 value")
    B, P, H, D = 1, 512, 24, 128
    allv = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    vals = (allv.astype(np.uint32) << 16).view(np.float32)
    vals = vals[np.isfinite(vals)]
    rng = np.random.default_rng(17)
    amaxes = [1.0, 448.0, 2.0 ** -20, 2.0 ** 20, 3.0, 1e-30, 1e30, 1e-13, 5e-10, 0.1, 7.0, 1000.0]
    amaxes += list(10.0 ** rng.uniform(-30, 30, H - len(amaxes)))
    v = np.zeros((B, P, H, D), np.float32)
    for h, am in enumerate(amaxes):
        am = np.float32(torch.tensor(am).to(torch.bfloat16).float().item())
        sel = vals[np.abs(vals) <= am]
        head = np.resize(sel, P * D)
        head[0] = am                                   # the amax itself
        v[0, :, h, :] = head.reshape(P, D)
    vb = torch.from_numpy(v).to(torch.bfloat16)
    k = torch.zeros(B, P, H, D, dtype=torch.bfloat16)
    cache = qik.ContiguousKVCache(1, B, P, H, D, v_fp8=True, device=DEV)
    cache.get_layer(0).store(k.to(DEV), vb.to(DEV))
    _, vv, sc = cache.get_layer(0).views()
    got = vv.transpose(1, 2).contiguous().view(torch.uint8).cpu().numpy()
    kt, vt, st = _torch_store(k.to(DEV), vb.to(DEV), True)
    np.testing.assert_array_equal(sc.cpu().numpy(), st.cpu().numpy())
    np.testing.assert_array_equal(got, vt.view(torch.uint8).cpu().numpy())
    codes, scale = of.quantize_per_head(vb.float().numpy())
    np.testing.assert_array_equal(got, codes)


@pytest.mark.parametrize("D", [128, 64])
def test_slab_store_fp16_source_every_value(D):
    """An fp8 slab in an fp16 model: the reference quantises whatever dtype V
    has (kv_cache.py:36-42 takes v.float() first).  Every finite fp16 value,
    shuffled, in heads whose planted amax runs from the largest fp16 (65504)
    down to the smallest subnormal (2^-24), plus an all-zero head; codes and
    scales against the oracle and torch's ops on the device, K bit-exact, and
    the three-launch form against the workspace form."""
    _flush(f"case slab store fp16 source D={D}")
    B, P, H = 2, 160, 5
    allv = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16).view(np.float16)
    vals = allv[np.isfinite(allv)].astype(np.float32)
    rng = np.random.default_rng(23 + D)
    amaxes = [65504.0, 1.0, 448.0, 2.0 ** -14, 2.0 ** -24, 0.0, 3.0, 1e-3, 1000.0, 0.1]
    v = np.zeros((B, P, H, D), np.float32)
    for i, am in enumerate(amaxes):
        b, h = divmod(i, H)
        am = np.float32(np.float16(am))
        sel = vals[np.abs(vals) <= am]
        head = np.resize(rng.permutation(sel), P * D)
        head[0] = am
        v[b, :, h, :] = head.reshape(P, D)
    vh = torch.from_numpy(v).to(torch.float16).to(DEV)
    k = torch.from_numpy(v[:, ::-1].copy()).to(torch.float16).to(DEV)
    caches = [qik.ContiguousKVCache(1, B, P + 8, H, D, v_fp8=True, device=DEV, dtype=torch.float16)
              for _ in range(2)]
    caches[0].get_layer(0).store(k, vh)                        # workspace form
    lib = _lib.load()
    a3, keep3 = caches[1].get_layer(0).store_args(k, vh, P)
    assert lib.qik_slab_store(ctypes.byref(a3), torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    kt, vt, st = _torch_store(k, vh, True)
    codes, scale = of.quantize_per_head(v)
    for c in caches:                                           # slab layout [B, H, P, D]
        got = c.v_buf[0, :, :, :P].contiguous().view(torch.uint8).cpu().numpy()
        sc = c.v_scale[0].cpu().numpy()
        np.testing.assert_array_equal(got, codes)
        np.testing.assert_array_equal(got, vt.view(torch.uint8).cpu().numpy())
        np.testing.assert_array_equal(sc, scale)
        np.testing.assert_array_equal(sc, st.cpu().numpy())
        np.testing.assert_array_equal(_bits(c.k_buf[0, :, :, :P]), _bits(kt))
    assert scale[1, 0] == np.float32(1e-12)                    # the all-zero head
    del keep3


def test_slab_store_rounding_edges():
    """Quotients on e4m3fn ties and in the subnormal range, an all-zero head
    (scale 1e-12) and the extremes +-amax (codes +-448)."""
    _flush("case slab store edges")
    B, P, H, D = 1, 64, 3, 128
    table = of.e4m3fn_decode_table()
    finite = table[np.isfinite(table)]
    pos = np.unique(np.abs(finite))
    mids = ((pos[:-1].astype(np.float64) + pos[1:]) / 2).astype(np.float32)   # exact ties
    vals = np.concatenate([pos, mids, -pos, -mids, pos[:8] * 0.75])
    v = np.zeros((B, P, H, D), np.float32)
    flat = np.resize(vals, P * D).reshape(P, D)
    flat[0, 0] = 448.0                          # amax: scale = 448 * fp32(1/448)
    v[0, :, 0, :] = flat
    v[0, :, 1, :] = -flat * 2.0 ** -20          # tiny magnitudes, same pattern
    # head 2 stays all zero
    vb = torch.from_numpy(v).to(torch.bfloat16)
    k = torch.zeros(B, P, H, D, dtype=torch.bfloat16)
    cache = qik.ContiguousKVCache(1, B, P, H, D, v_fp8=True, device=DEV)
    cache.get_layer(0).store(k.to(DEV), vb.to(DEV))
    _, vv, sc = cache.get_layer(0).views()
    codes, scale = of.quantize_per_head(vb.float().numpy())
    np.testing.assert_array_equal(sc.cpu().numpy(), scale)
    np.testing.assert_array_equal(vv.transpose(1, 2).contiguous().view(torch.uint8).cpu().numpy(), codes)
    assert sc[0, 2].item() == np.float32(1e-12)
    kt, vt, st = _torch_store(k.to(DEV), vb.to(DEV), True)
    np.testing.assert_array_equal(vv.transpose(1, 2).contiguous().view(torch.uint8).cpu().numpy(),
                                  vt.view(torch.uint8).cpu().numpy())


# ---------------------------------------------------------------------------
# processor


class _Norm:
    def __init__(self, D, g):
        self.weight = (1.0 + 0.2 * torch.randn(D, generator=g)).to(DEV)
        self.eps = 1e-6


class _Lin(torch.nn.Module):
    def __init__(self, i, o, g):
        super().__init__()
        self.in_features, self.out_features = i, o
        self.weight = (torch.randn(o, i, generator=g) * i ** -0.5).to(torch.bfloat16).to(DEV)
        self.bias = (torch.randn(o, generator=g) * 0.02).to(torch.bfloat16).to(DEV)

    def forward(self, x):
        return torch.nn.functional.linear(x, self.weight, self.bias)


class FakeAttn:
    """The attributes the processor reads from diffusers' Attention module."""

    def __init__(self, dim, H, D, seed, fused=False, out_proj=False):
        g = torch.Generator().manual_seed(seed)
        self.heads = H
        if fused:
            self.fused_qkv = _Lin(dim, 3 * H * D, g)
        else:
            self.to_q, self.to_k, self.to_v = (_Lin(dim, H * D, g) for _ in range(3))
        self.norm_q, self.norm_k = _Norm(D, g), _Norm(D, g)
        self.to_out = [_Lin(H * D, dim, g) if out_proj else torch.nn.Identity(), torch.nn.Identity()]

    def qkv(self, x):
        H = self.heads
        if hasattr(self, "fused_qkv"):
            D = self.fused_qkv.out_features // (3 * H)
            return self.fused_qkv(x).unflatten(-1, (3 * H, D)).chunk(3, dim=-2)
        D = self.to_q.out_features // H
        return tuple(m(x).unflatten(-1, (H, D)) for m in (self.to_q, self.to_k, self.to_v))


def _stock_qkv(attn, x, freqs):
    q, k, v = attn.qkv(x)
    q = orr.stock_rms_norm_rope(q, attn.norm_q.weight, freqs, attn.norm_q.eps)
    k = orr.stock_rms_norm_rope(k, attn.norm_k.weight, freqs, attn.norm_k.eps)
    return q, k, v


def _hidden(B, S, dim, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(B, S, dim, generator=g).to(torch.bfloat16).to(DEV)


def _close(out, ref, what):
    d = np.abs(out.float().cpu().numpy() - ref)
    assert np.isfinite(out.float().cpu().numpy()).all(), what
    assert d.max() <= 2e-2 and d.mean() <= 2e-3, (what, d.max(), d.mean())


@pytest.mark.parametrize("fused", [False, True])
def test_processor_prefill_with_segments(fused):
    _flush(f"case processor prefill fused={fused}")
    B, H, D, dim = 2, 4, 128, 256
    segs, S = ol.make_segments([("text", 40), ("img", 150), ("text", 20), ("img", 90)])
    attn = FakeAttn(dim, H, D, seed=1, fused=fused)
    x = _hidden(B, S, dim, 2)
    freqs = orr.rope_freqs(S, D).to(DEV)
    kv_valid = torch.ones(B, S, dtype=torch.bool, device=DEV)
    kv_valid[1, 30:40] = False                    # padded text keys of the second sample
    out = qik.QwenImage21KernelProcessor()(attn, x, rotary_emb=freqs, segments=segs, key_valid=kv_valid)
    q, k, v = _stock_qkv(attn, x, freqs)
    L = ol.build_prefix_lengths(segs, segs[-1][1], S)
    ref = oa.attention_fp32(q, k, v, L, kv_valid.cpu()).reshape(B, S, H * D)
    _close(out, ref, "prefill")


def test_processor_extract_then_decode_against_the_slab():
    """Prefill writes the prefix into an fp8 slab (kv_cache_mode="extract"), then the
    target rows decode against the slab views without concatenation."""
    _flush("case processor extract + decode")
    B, H, D, dim = 1, 4, 128, 256
    segs, P = ol.make_segments([("text", 32), ("img", 224)])
    T = 160
    attn = FakeAttn(dim, H, D, seed=3, fused=True)
    cache = qik.ContiguousKVCache(2, B, P + 272, H, D, v_fp8=True, device=DEV)
    layer = cache.get_layer(1)
    proc = qik.QwenImage21KernelProcessor()

    xp = _hidden(B, P + T, dim, 4)
    freqs_all = orr.rope_freqs(P + T, D).to(DEV)
    proc(attn, xp, rotary_emb=freqs_all, layer_cache=layer, kv_cache_mode="extract",
         cache_write_slice=slice(0, P), segments=segs)
    # the slab holds the processor's post-RoPE K and the fp8 quantisation of V
    qa, ka, va = attn.qkv(xp)
    k_rope = qik.fused_rms_norm_rope(ka, attn.norm_k.weight, freqs_all, attn.norm_k.eps)
    kc, vc, sc = layer.views()
    np.testing.assert_array_equal(_bits(kc), _bits(k_rope[:, :P]))
    codes, scale = of.quantize_per_head(va[:, :P].float().cpu().numpy())
    np.testing.assert_array_equal(sc.cpu().numpy(), scale)
    np.testing.assert_array_equal(vc.transpose(1, 2).contiguous().view(torch.uint8).cpu().numpy(), codes)

    # decode step: target rows only, RoPE of the target positions
    xt = _hidden(B, T, dim, 5)
    freqs_t = orr.rope_freqs(T, D, offset=P).to(DEV)
    out = proc(attn, xt, rotary_emb=freqs_t, layer_cache=layer)
    q, k, v = _stock_qkv(attn, xt, freqs_t)
    L = np.full(T, P + T - 1, dtype=np.int32)
    ref = oa.attention_fp32(q, k, v, L, None, kc.cpu(), vc.cpu(), sc.cpu()).reshape(B, T, H * D)
    _close(out, ref, "decode fp8 slab")

    # the same step with a key mask over [prefix, target] (attention_mask [B, 1, KV])
    mask = torch.ones(B, 1, P + T, dtype=torch.bool, device=DEV)
    mask[:, :, 5:20] = False
    out_m = proc(attn, xt, attention_mask=mask, rotary_emb=freqs_t, layer_cache=layer)
    ref_m = oa.attention_fp32(q, k, v, L, mask.reshape(B, -1).cpu(), kc.cpu(), vc.cpu(), sc.cpu())
    _close(out_m, ref_m.reshape(B, T, H * D), "decode masked")


class _StockCache:
    """A cache with only get() (bf16 V, no views / scale), processors.py:100-102."""

    def __init__(self, k, v):
        self.k, self.v = k, v

    def get(self):
        return self.k, self.v


def test_processor_decode_with_get_only_cache_and_no_cache():
    _flush("case processor get-only cache / no cache")
    B, H, D, dim, P, T = 2, 3, 128, 192, 200, 96
    attn = FakeAttn(dim, H, D, seed=6)
    g = torch.Generator().manual_seed(7)
    ck = torch.randn(B, P, H, D, generator=g).to(torch.bfloat16).to(DEV)
    cv = torch.randn(B, P, H, D, generator=g).to(torch.bfloat16).to(DEV)
    xt = _hidden(B, T, dim, 8)
    freqs = orr.rope_freqs(T, D, offset=P).to(DEV)
    proc = qik.QwenImage21KernelProcessor()
    out = proc(attn, xt, rotary_emb=freqs, layer_cache=_StockCache(ck, cv))
    q, k, v = _stock_qkv(attn, xt, freqs)
    ref = oa.attention_fp32(q, k, v, np.full(T, P + T - 1, np.int32), None, ck.cpu(), cv.cpu())
    _close(out, ref.reshape(B, T, H * D), "get-only cache")
    # no cache, no segments: full attention over the sequence
    out2 = proc(attn, xt, rotary_emb=freqs)
    ref2 = oa.attention_fp32(q, k, v, np.full(T, T - 1, np.int32))
    _close(out2, ref2.reshape(B, T, H * D), "no cache")


def test_processor_applies_output_projection():
    _flush("case processor to_out")
    B, H, D, dim = 1, 2, 128, 128
    segs, S = ol.make_segments([("text", 16), ("img", 64)])
    attn = FakeAttn(dim, H, D, seed=9, out_proj=True)
    x = _hidden(B, S, dim, 10)
    freqs = orr.rope_freqs(S, D).to(DEV)
    proc = qik.QwenImage21KernelProcessor()
    out = proc(attn, x, rotary_emb=freqs, segments=segs)
    proj = attn.to_out[0]
    attn.to_out[0] = torch.nn.Identity()
    inner = proc(attn, x, rotary_emb=freqs, segments=segs)
    attn.to_out[0] = proj
    assert out.shape == (B, S, dim)
    np.testing.assert_array_equal(_bits(out), _bits(proj(inner)))
