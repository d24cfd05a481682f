"""Attention processor for Qwen-Image 2.1 on the MI355X path.

``QwenImage21KernelProcessor`` has the call signature and semantics of the
reference processor (qwen_image_kernel/processors.py:39-126), with every device
step of the attention layer between the projections on this package's HIP
kernels:

* Q/K: per-head RMSNorm + RoPE, ``fused_rms_norm_rope`` (qik_rms_rope);
* prefix extraction: ``layer_cache.store`` (qik_slab_store on a HIP slab);
* attention: ``block_causal_flash_attention`` (qik_attn_fwd_ws) -- prefill over the
  joint sequence with per-row causal lengths from the segment list, decode of
  the target rows against the slab views (no torch.cat), or full attention
  without a cache;
* the causal lengths: ``build_prefix_lengths`` (qik_build_prefix_lengths).

The projections (``to_q/k/v`` or ``fused_qkv``, ``to_out``) are the caller's
modules, called as the reference calls them.
"""

from __future__ import annotations

import torch

from .attention import block_causal_flash_attention, build_prefix_lengths
from .fused import fused_rms_norm_rope
from .kv_cache import _LayerView

__all__ = ["QwenImage21KernelProcessor", "_build_prefix_lengths"]


def _build_prefix_lengths(segments, prefix_len: int, seq_len: int, device) -> torch.Tensor:
    """Per-row inclusive kv limit L (processors.py:22-36): row q attends iff kv <= L[q].

    text run (s, e) -> L[s:e] = s..e-1 (causal); image run (s, e) -> L[s:e] = e-1;
    rows >= prefix_len -> seq_len - 1.  One device launch.
    """
    return build_prefix_lengths(segments, prefix_len, seq_len, device)


class QwenImage21KernelProcessor:
    """Drop-in for ``QwenImage21AttnProcessor`` (same call signature)."""

    _attention_backend = None
    _parallel_config = None

    def __call__(
        self,
        attn,
        hidden_states: torch.Tensor,
        attention_mask=None,
        rotary_emb=None,
        layer_cache=None,
        kv_cache_mode: str | None = None,
        cache_write_slice=None,
        segments=None,
        key_valid=None,
    ) -> torch.Tensor:
        B, S, _ = hidden_states.shape
        H = attn.heads
        fused_qkv = getattr(attn, "fused_qkv", None)
        if fused_qkv is not None:
            # one GEMM for Q, K, V; the q/k/v slices are strided views that the
            # kernels below read in place
            D = fused_qkv.out_features // (3 * H)
            qkv = fused_qkv(hidden_states)
            query, key, value = qkv.unflatten(-1, (3 * H, D)).chunk(3, dim=-2)
        else:
            D = attn.to_q.out_features // H
            query = attn.to_q(hidden_states).unflatten(-1, (H, D))
            key = attn.to_k(hidden_states).unflatten(-1, (H, D))
            value = attn.to_v(hidden_states).unflatten(-1, (H, D))

        # QK-RMSNorm + RoPE (processors.py:77-79)
        query = fused_rms_norm_rope(query, attn.norm_q.weight, rotary_emb, attn.norm_q.eps)
        key = fused_rms_norm_rope(key, attn.norm_k.weight, rotary_emb, attn.norm_k.eps)

        if kv_cache_mode == "extract" and layer_cache is not None and cache_write_slice is not None:
            k_pre, v_pre = key[:, cache_write_slice], value[:, cache_write_slice]
            if not isinstance(layer_cache, _LayerView):
                # a cache that keeps the tensors it is given (the stock get()-only
                # cache) gets copies, as processors.py:83-84 hands it, so that it
                # does not pin the whole K/V (or fused QKV output) of the layer
                k_pre, v_pre = k_pre.clone(), v_pre.clone()
            # ContiguousKVCache copies into its slab: the slices are read in place
            layer_cache.store(k_pre, v_pre)

        if segments is not None:
            # prefill over the full joint sequence (processors.py:86-94)
            assert key_valid is None or key_valid.dim() == 2
            prefix_end = segments[-1][1] if segments else 0
            L = _build_prefix_lengths(segments, prefix_end, S, query.device)
            out = block_causal_flash_attention(query, key, value, L, key_valid, cache_k=None, cache_v=None)
        else:
            kv_mask = attention_mask
            if kv_mask is not None:
                kv_mask = kv_mask.reshape(kv_mask.shape[0], -1)
            if layer_cache is not None:
                # decode: target rows against [prefix slab, fresh target keys] (:95-112)
                if hasattr(layer_cache, "views"):
                    cache_k, cache_v, v_scale = layer_cache.views()
                else:
                    cache_k, cache_v = layer_cache.get()
                    v_scale = None
                kv_total = cache_k.shape[1] + key.shape[1]
                L = torch.full((key.shape[1],), kv_total - 1, dtype=torch.int32, device=query.device)
                out = block_causal_flash_attention(
                    query, key, value, L, kv_mask, cache_k=cache_k, cache_v=cache_v,
                    cache_v_scale=v_scale, uniform_full=kv_mask is None,
                )
            else:
                # no cache: full attention over the whole sequence (:113-122)
                L = torch.full((key.shape[1],), key.shape[1] - 1, dtype=torch.int32, device=query.device)
                out = block_causal_flash_attention(query, key, value, L, kv_mask, uniform_full=kv_mask is None)

        out = out.flatten(2, 3).type_as(query)
        out = attn.to_out[0](out)
        return attn.to_out[1](out)
