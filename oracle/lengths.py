"""Causal-length array and the masks it stands for.  Test infrastructure only."""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F


def make_segments(seq_layout):
    """[('text', n) | ('img', n), ...] -> ([(start, end, is_text)], total).

    Restates make_segments of tests/test_attention.py:56-62.
    """
    segs, pos = [], 0
    for kind, n in seq_layout:
        segs.append((pos, pos + n, kind == "text"))
        pos += n
    return segs, pos


def build_prefix_lengths(segments, prefix_len: int, seq_len: int) -> np.ndarray:
    """L: row q attends kv iff kv <= L[q]  (processors.py:22-36).

    L = arange(seq_len); every non-text run (s, e) sets L[s:e] = e-1 in order;
    then L[prefix_len:] = seq_len-1.  numpy slicing has Python slice semantics,
    as the reference's torch slice assignments do.

    Pinned by: brute-force equality of (kv <= L[q]) with ``segment_mask``.
    """
    L = np.arange(seq_len, dtype=np.int32)
    for start, end, is_text in segments:
        if not is_text:
            L[start:end] = end - 1
    L[prefix_len:] = seq_len - 1
    return L


def segment_mask(segments, seq_len: int, prefix_len: int) -> np.ndarray:
    """Brute-force allowed[q, kv] from the mask's definition (triton_attention.py:5-14).

    Prefix rows: allowed = (q >= kv) or (q and kv in the same image run).
    Rows at or after prefix_len (the target) attend every key.
    """
    allowed = np.zeros((seq_len, seq_len), dtype=bool)
    q = np.arange(seq_len)[:, None]
    kv = np.arange(seq_len)[None, :]
    allowed |= q >= kv
    for start, end, is_text in segments:
        if not is_text:
            allowed[start:end, start:end] = True
    allowed[prefix_len:, :] = True
    return allowed


def mask_from_lengths(L: np.ndarray, kv_total: int, key_valid: np.ndarray | None = None) -> np.ndarray:
    """allowed[b?, q, kv] = kv <= L[q] (and key_valid[b, kv]); shape [SQ, KV] or [B, SQ, KV]."""
    allowed = np.arange(kv_total)[None, :] <= np.asarray(L)[:, None]
    if key_valid is not None:
        allowed = allowed[None, :, :] & np.asarray(key_valid, dtype=bool)[:, None, :]
    return allowed


def stock_multipass_sdpa(query, key, value, segments, prefix_len, key_valid=None):
    """The stock processor's prefill as per-segment SDPA calls, in fp32 on the CPU.

    Restates stock_reference of tests/test_attention.py:17-53: each text run
    attends [0, start) fully plus a causal triangle of itself, each image run
    attends [0, end) fully, the target attends every key; key_valid gates keys.
    Inputs [B, S, H, D]; returns fp32 [B, S, H, D].  An independent statement of
    the mask that L collapses (it never looks at L).
    """
    q = query.float().cpu()
    k = key.float().cpu()
    v = value.float().cpu()
    kvm = None if key_valid is None else key_valid.cpu().bool()
    outs = []
    for start, end, is_text in segments:
        seg_mask = None
        if is_text:
            n = end - start
            seg_mask = torch.cat(
                [torch.ones(n, start, dtype=torch.bool), torch.tril(torch.ones(n, n, dtype=torch.bool))], dim=1
            )[None, None]
        if kvm is not None:
            kk = kvm[:, None, None, :end]
            seg_mask = kk if seg_mask is None else (seg_mask & kk)
        outs.append(
            F.scaled_dot_product_attention(
                q[:, start:end].transpose(1, 2).contiguous(),
                k[:, :end].transpose(1, 2).contiguous(),
                v[:, :end].transpose(1, 2).contiguous(),
                attn_mask=seg_mask,
            ).transpose(1, 2)
        )
    outs.append(
        F.scaled_dot_product_attention(
            q[:, prefix_len:].transpose(1, 2).contiguous(),
            k.transpose(1, 2).contiguous(),
            v.transpose(1, 2).contiguous(),
            attn_mask=kvm[:, None, None, :] if kvm is not None else None,
        ).transpose(1, 2)
    )
    return torch.cat(outs, dim=1)
