"""Attention oracles on the CPU.  Test infrastructure only.

* ``reference_block_causal_attention`` -- fp32 explicit-mask softmax attention with
  the signature of triton_attention.py:266-293, plus fp8 slab V.
* ``attention_fp64``  -- float64 brute force for tiny inputs (pins the fp32 oracle).
* ``flash_emulation`` -- the Triton kernel's tile loop with its rounding points
  (triton_attention.py:121-168), in numpy, for tiny inputs.
* ``sdpa_explicit_mask_cpu`` -- the CPU baseline: torch explicit-mask SDPA in fp32.
"""

from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

from . import fp8 as _fp8
from . import schedule as _sched

LOG2E = 1.4426950408889634


def _np(t) -> np.ndarray:
    if isinstance(t, torch.Tensor):
        t = t.detach().cpu()
        if t.dtype in (torch.bfloat16, torch.float16):
            t = t.float()
        if t.dtype == torch.float8_e4m3fn:
            return t.view(torch.uint8).numpy()
        return t.numpy()
    return np.asarray(t)


def dequant_cache_v(cache_v, cache_v_scale) -> np.ndarray:
    """[B, P, H, D] fp8 codes (torch float8_e4m3fn or uint8) + [B, H] scale -> fp32 values on bf16."""
    codes = _np(cache_v).astype(np.uint8)                    # [B, P, H, D]
    sc = _np(cache_v_scale).astype(np.float32)               # [B, H]
    return _fp8.dequant_bf16(codes, sc[:, None, :, None])


def _kv_all(key, value, cache_k, cache_v, cache_v_scale):
    k = _np(key).astype(np.float32)
    v = _np(value).astype(np.float32)
    if cache_k is not None and cache_k.shape[1] > 0:
        ck = _np(cache_k).astype(np.float32)
        cv = dequant_cache_v(cache_v, cache_v_scale) if cache_v_scale is not None else _np(cache_v).astype(np.float32)
        k = np.concatenate([ck, k], axis=1)
        v = np.concatenate([cv, v], axis=1)
    return k, v


def attention_fp32(query, key, value, prefix_lengths, key_valid=None, cache_k=None, cache_v=None,
                   cache_v_scale=None, heads=None, batches=None) -> np.ndarray:
    """fp32 softmax(Q K^T * D**-0.5 masked) V, returned as float32 [B, SQ, H, D].

    Restates reference_block_causal_attention (triton_attention.py:266-293):
    allowed = (kv <= L[q]) & key_valid[b, kv]; masked scores are -inf; torch fp32
    softmax and matmuls on the CPU, one (b, h) at a time to bound memory.
    Difference: a row with no allowed key returns zeros (the reference yields
    NaN there; the kernel writes zeros, triton_attention.py:166).
    ``heads`` / ``batches`` restrict the computation (other entries stay 0).
    """
    q = _np(query).astype(np.float32)
    k, v = _kv_all(key, value, cache_k, cache_v, cache_v_scale)
    B, SQ, H, D = q.shape
    KV = k.shape[1]
    L = _np(prefix_lengths).astype(np.int64)[:SQ]
    allowed = torch.from_numpy(np.arange(KV)[None, :] <= L[:, None])
    kvm = None if key_valid is None else torch.from_numpy(_np(key_valid).astype(bool))
    out = np.zeros((B, SQ, H, D), dtype=np.float32)
    scale = D ** -0.5
    for b in (range(B) if batches is None else batches):
        al = allowed if kvm is None else (allowed & kvm[b][None, :KV])
        any_row = al.any(dim=1, keepdim=True)
        # with every key allowed (uniform lengths) the mask and the empty-row
        # guard change nothing and are skipped
        full = bool(al.all())
        for h in (range(H) if heads is None else heads):
            qt = torch.from_numpy(np.ascontiguousarray(q[b, :, h]))
            kt = torch.from_numpy(np.ascontiguousarray(k[b, :, h]))
            vt = torch.from_numpy(np.ascontiguousarray(v[b, :, h]))
            s = (qt @ kt.T) * scale
            if not full:
                s = s.masked_fill(~al, float("-inf"))
            p = torch.softmax(s, dim=-1)
            if not full:
                p = torch.where(any_row, p, torch.zeros_like(p))
            out[b, :, h] = (p @ vt).numpy()
    return out


def reference_block_causal_attention(query, key, value, prefix_lengths, key_valid, cache_k=None,
                                     cache_v=None, cache_v_scale=None):
    """Same signature and result dtype as triton_attention.py:266 (plus ``cache_v_scale``)."""
    out = attention_fp32(query, key, value, prefix_lengths, key_valid, cache_k, cache_v, cache_v_scale)
    return torch.from_numpy(out).to(query.dtype)


def attention_fp64(query, key, value, prefix_lengths, key_valid=None, cache_k=None, cache_v=None,
                   cache_v_scale=None) -> np.ndarray:
    """Float64 brute force, row by row, from the definition of softmax attention.

    For tiny inputs only.  Inputs are taken at their stored values (bf16 / the
    dequantised fp8 V), so only the arithmetic precision differs from the fp32 oracle.
    """
    q = _np(query).astype(np.float64)
    k, v = _kv_all(key, value, cache_k, cache_v, cache_v_scale)
    k = k.astype(np.float64)
    v = v.astype(np.float64)
    B, SQ, H, D = q.shape
    KV = k.shape[1]
    L = _np(prefix_lengths).astype(np.int64)
    kvm = None if key_valid is None else _np(key_valid).astype(bool)
    out = np.zeros((B, SQ, H, D), dtype=np.float64)
    for b in range(B):
        for h in range(H):
            for r in range(SQ):
                keys = [j for j in range(KV) if j <= L[r] and (kvm is None or kvm[b, j])]
                if not keys:
                    continue
                s = np.array([float(np.dot(q[b, r, h], k[b, j, h])) for j in keys]) / math.sqrt(D)
                w = np.exp(s - s.max())
                w /= w.sum()
                out[b, r, h] = (w[:, None] * v[b, keys, h]).sum(axis=0)
    return out


def flash_emulation(query, key, value, prefix_lengths, key_valid=None, cache_k=None, cache_v=None,
                    cache_v_scale=None, BM=128, BN=64, uniform=False, out_dtype="bf16") -> np.ndarray:
    """The Triton kernel's loop and rounding points in numpy (triton_attention.py:70-168).

    Per row block: reference tile schedule (:95-121), S = (Q.K^T) * qk_scale with
    qk_scale = fp32(fp32(D**-0.5) * fp32(log2 e)) (:93, :143), masked to -inf (:144),
    exp2 online softmax with l accumulated from fp32 p and P rounded to bf16 for the
    PV product (:146-163), fp8 slab V dequantised as bf16(fp32(v) * scale) (:157-159),
    out = l > 0 ? acc / l : 0 rounded to bf16 (:166-168).  Tiny inputs only.
    """
    q = _np(query).astype(np.float32)
    kn = _np(key).astype(np.float32)
    vn = _np(value).astype(np.float32)
    B, SQ, H, D = q.shape
    SN = kn.shape[1]
    has_cache = cache_k is not None and cache_k.shape[1] > 0
    P = cache_k.shape[1] if has_cache else 0
    if has_cache:
        kc = _np(cache_k).astype(np.float32)
        vc = dequant_cache_v(cache_v, cache_v_scale) if cache_v_scale is not None else _np(cache_v).astype(np.float32)
    KV = P + SN
    L = np.full(SQ, KV - 1) if uniform else _np(prefix_lengths).astype(np.int64)[:SQ]
    kvm = None if key_valid is None else _np(key_valid).astype(bool)
    qk_scale = np.float32(np.float32(D ** -0.5) * np.float32(LOG2E))
    tiles = _sched.visited_tiles(L, SQ, P, SN, BM, BN, has_cache, uniform, rule="reference")
    out = np.zeros((B, SQ, H, D), dtype=np.float32)
    segs = _sched.segments(P, SN, BN, has_cache)
    for b in range(B):
        for h in range(H):
            for mblk in range(len(tiles)):
                r0, r1 = mblk * BM, min(SQ, (mblk + 1) * BM)
                Lr = L[r0:r1]
                qt = q[b, r0:r1, h]
                m_i = np.full(r1 - r0, -np.inf, dtype=np.float32)
                l_i = np.zeros(r1 - r0, dtype=np.float32)
                acc = np.zeros((r1 - r0, D), dtype=np.float32)
                for ph, t in tiles[mblk]:
                    seg_len, start, _ = segs[ph]
                    loc = np.arange(t * BN, (t + 1) * BN)
                    in_seg = loc < seg_len
                    locc = np.minimum(loc, seg_len - 1)
                    if has_cache and ph == 0:
                        kt, vt = kc[b, locc, h], vc[b, locc, h]
                    else:
                        kt, vt = kn[b, locc, h], vn[b, locc, h]
                    kt = np.where(in_seg[:, None], kt, 0.0).astype(np.float32)
                    vt = np.where(in_seg[:, None], vt, 0.0).astype(np.float32)
                    kv_abs = start + loc
                    allowed = in_seg[None, :] & (kv_abs[None, :] <= Lr[:, None])
                    if kvm is not None:
                        allowed &= kvm[b, np.minimum(kv_abs, KV - 1)][None, :] & in_seg[None, :]
                    s = (qt @ kt.T).astype(np.float32) * qk_scale
                    s = np.where(allowed, s, -np.inf).astype(np.float32)
                    m_new = np.maximum(m_i, s.max(axis=1))
                    m_safe = np.where(m_new == -np.inf, np.float32(0), m_new).astype(np.float32)
                    with np.errstate(invalid="ignore"):
                        p = np.exp2(s - m_safe[:, None]).astype(np.float32)
                    p = np.where(allowed, p, 0.0).astype(np.float32)
                    alpha = np.where(m_new == -np.inf, 0.0, np.exp2(m_i - m_safe)).astype(np.float32)
                    l_i = (l_i * alpha + p.sum(axis=1)).astype(np.float32)
                    m_i = m_new
                    acc = (acc * alpha[:, None] + _fp8.bf16_round(p) @ vt).astype(np.float32)
                with np.errstate(invalid="ignore", divide="ignore"):
                    o = np.where(l_i[:, None] > 0, acc / l_i[:, None], 0.0).astype(np.float32)
                out[b, r0:r1, h] = o
    return _fp8.bf16_round(out) if out_dtype == "bf16" else out


def sdpa_explicit_mask_cpu(query, key, value, prefix_lengths, key_valid=None, cache_k=None, cache_v=None,
                           cache_v_scale=None, heads=None, batches=None) -> torch.Tensor:
    """CPU baseline: torch F.scaled_dot_product_attention in fp32 with a bool [SQ, KV] mask.

    One (b, h) at a time; fp8 slab V is dequantised first.  Returns fp32 [B, SQ, H, D].
    """
    q = torch.from_numpy(_np(query).astype(np.float32))
    k, v = _kv_all(key, value, cache_k, cache_v, cache_v_scale)
    k = torch.from_numpy(k)
    v = torch.from_numpy(v)
    B, SQ, H, D = q.shape
    KV = k.shape[1]
    L = torch.from_numpy(_np(prefix_lengths).astype(np.int64)[:SQ])
    mask = torch.arange(KV)[None, :] <= L[:, None]
    out = torch.zeros(B, SQ, H, D)
    for b in (range(B) if batches is None else batches):
        mb = mask if key_valid is None else mask & torch.as_tensor(_np(key_valid)[b].astype(bool))[None, :KV]
        for h in (range(H) if heads is None else heads):
            out[b, :, h] = F.scaled_dot_product_attention(
                q[b, :, h][None, None].contiguous(), k[b, :, h][None, None].contiguous(),
                v[b, :, h][None, None].contiguous(), attn_mask=mb[None, None])[0, 0]
    return out


class CpuSdpaBaseline:
    """The CPU baseline prepared once, then timed per (b, h).

    ``prepare`` (untimed) moves the inputs to fp32 host tensors, dequantises an
    fp8 slab V and concatenates [slab, fresh] keys; ``run(b, h)`` is one
    explicit-mask F.scaled_dot_product_attention call with a bool [SQ, KV] mask.
    """

    def __init__(self, query, key, value, prefix_lengths, cache_k=None, cache_v=None, cache_v_scale=None):
        self.q = torch.from_numpy(np.ascontiguousarray(_np(query).astype(np.float32)))
        k, v = _kv_all(key, value, cache_k, cache_v, cache_v_scale)
        self.k = torch.from_numpy(np.ascontiguousarray(k))
        self.v = torch.from_numpy(np.ascontiguousarray(v))
        SQ, KV = self.q.shape[1], self.k.shape[1]
        L = torch.from_numpy(_np(prefix_lengths).astype(np.int64)[:SQ])
        self.mask = (torch.arange(KV)[None, :] <= L[:, None])[None, None]
        self.pairs = int(self.mask.sum())

    def run(self, b: int, h: int) -> torch.Tensor:
        return F.scaled_dot_product_attention(
            self.q[b, :, h][None, None].contiguous(), self.k[b, :, h][None, None].contiguous(),
            self.v[b, :, h][None, None].contiguous(), attn_mask=self.mask)[0, 0]
