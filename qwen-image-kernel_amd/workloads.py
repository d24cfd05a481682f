"""Attention shapes of Qwen-Image 2.1 (head_dim 128) and seeded synthetic inputs.

Five shapes, from the CPU-checkable tiny case up to the multi-reference edit:

* ``tiny``         B1 H4,  64 causal text + one 256-token image block, fresh K/V (N=320)
* ``t2i_512``      B1 H24, 128 text + 1024 image tokens (32x32 latent patches), fresh K/V
* ``t2i_1024``     B1 H24, 256 text + 4096 image tokens (64x64), fresh K/V, 32 layers
* ``edit_768``     B1 H24, decode: 4096 target queries against a slab prefix of
                   256 text + 2304 condition tokens (48x48; bf16 K, fp8 V) + 4096 fresh keys
* ``multiref_cfg`` B2 H24 (cond/uncond), 256 text + 3 x 1024 condition blocks in the slab
                   + 4096 fresh target tokens, all 7424 rows queried, ragged L
* ``ref_decode_1024`` B1 H32, the shape of the reference's one published kernel number
                   (RESULTS.md:27, tools/sweep_attention2.py:95): 4096 target queries against
                   a 256-token text slab (bf16 K and V) + 4096 fresh keys, uniform L

Inputs are N(0, 1) in fp32 from a seeded ``torch.Generator`` cast to bf16; the
slab V is quantised to fp8 per (b, h) by ``ContiguousKVCache.store``.  The
unmasked FLOP count is 4*D per allowed (query, key) pair, summed over (b, h).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

from .kv_cache import ContiguousKVCache

SLAB_PAD = 272  # extra slab capacity beyond the prefix, so the slab head stride != P*D


@dataclass
class Workload:
    name: str
    B: int
    H: int
    D: int
    SQ: int            # query rows
    P: int             # slab prefix keys (0 = no cache)
    SN: int            # fresh keys
    segments: list     # [(start, end, is_text)] over the prefix part of the query rows
    prefix_len: int    # rows >= prefix_len attend every key
    uniform: bool      # every row attends all P+SN keys
    v_fp8: bool        # slab V stored as fp8e4m3fn
    layers: int = 1
    L: np.ndarray = field(default=None, repr=False)

    @property
    def KV(self) -> int:
        return self.P + self.SN

    def lengths(self) -> np.ndarray:
        """Per-row causal length L (int32 [SQ]); the same array the processor builds."""
        if self.L is None:
            if self.uniform:
                L = np.full(self.SQ, self.KV - 1, dtype=np.int32)
            else:
                L = np.arange(self.SQ, dtype=np.int32)
                for s, e, is_text in self.segments:
                    if not is_text:
                        L[s:e] = e - 1
                L[self.prefix_len:] = self.SQ - 1
            self.L = L
        return self.L

    def unmasked_pairs(self) -> int:
        """Allowed (query, key) pairs of one (b, h)."""
        L = self.lengths().astype(np.int64)
        return int(np.minimum(L + 1, self.KV).clip(min=0).sum())

    def flops(self) -> int:
        """Unmasked QK^T + PV FLOPs of one layer: 4 * D * B * H * sum_q (L[q] + 1)."""
        return 4 * self.D * self.B * self.H * self.unmasked_pairs()

    def min_bytes(self) -> int:
        """Compulsory HBM bytes of one layer: Q, O, fresh K/V, slab K (+ V fp8 or bf16), L, scales."""
        vb = 1 if self.v_fp8 else 2
        per_bh = self.D * (2 * self.SQ * 2 + 2 * self.SN * 2 + self.P * (2 + vb))
        return self.B * self.H * per_bh + (0 if self.uniform else 4 * self.SQ) + (4 * self.B * self.H if self.v_fp8 else 0)


def _layout(runs):
    segs, pos = [], 0
    for kind, n in runs:
        segs.append((pos, pos + n, kind == "text"))
        pos += n
    return segs, pos


def workload(name: str) -> Workload:
    if name == "tiny":
        segs, n = _layout([("text", 64), ("img", 256)])
        return Workload(name, 1, 4, 128, n, 0, n, segs, n, False, False)
    if name == "t2i_512":
        segs, n = _layout([("text", 128), ("img", 1024)])
        return Workload(name, 1, 24, 128, n, 0, n, segs, n, False, False)
    if name == "t2i_1024":
        segs, n = _layout([("text", 256), ("img", 4096)])
        return Workload(name, 1, 24, 128, n, 0, n, segs, n, False, False, layers=32)
    if name == "edit_768":
        return Workload(name, 1, 24, 128, 4096, 256 + 48 * 48, 4096, [], 0, True, True)
    if name == "multiref_cfg":
        segs, p = _layout([("text", 256), ("img", 1024), ("img", 1024), ("img", 1024)])
        return Workload(name, 2, 24, 128, p + 4096, p, 4096, segs, p, False, True)
    if name == "ref_decode_1024":
        return Workload(name, 1, 32, 128, 4096, 256, 4096, [], 0, True, False)
    raise KeyError(f"unknown workload {name!r}")


NAMES = ("tiny", "t2i_512", "t2i_1024", "edit_768", "multiref_cfg")


def _randn(shape, gen: torch.Generator, device) -> torch.Tensor:
    return torch.randn(*shape, generator=gen, dtype=torch.float32, device=gen.device).to(
        device=device, dtype=torch.bfloat16)


def make_inputs(wl: Workload, seed: int, device="cuda", gen_device: str = "cpu") -> dict:
    """Seeded synthetic inputs for one layer of ``wl``.

    Draw order: query, fresh key, fresh value, then (with a slab) prefix key and
    prefix value, each N(0, 1) fp32 from ``torch.Generator(gen_device).manual_seed(seed)``
    cast to bf16.  The prefix is written through ``ContiguousKVCache.store`` into
    a one-layer slab of capacity P + 272, and the kernel reads its ``views()``.
    """
    gen = torch.Generator(device=gen_device)
    gen.manual_seed(seed)
    B, H, D = wl.B, wl.H, wl.D
    q = _randn((B, wl.SQ, H, D), gen, device)
    k = _randn((B, wl.SN, H, D), gen, device)
    v = _randn((B, wl.SN, H, D), gen, device)
    out = {"query": q, "key": k, "value": v,
           "prefix_lengths": torch.from_numpy(wl.lengths()).to(device)}
    if wl.P > 0:
        ck = _randn((B, wl.P, H, D), gen, device)
        cv = _randn((B, wl.P, H, D), gen, device)
        cache = ContiguousKVCache(1, B, wl.P + SLAB_PAD, H, D, v_fp8=wl.v_fp8, device=device)
        cache.get_layer(0).store(ck, cv)
        kc, vc, sc = cache.get_layer(0).views()
        out.update(cache=cache, cache_k=kc, cache_v=vc, cache_v_scale=sc, prefix_k=ck, prefix_v=cv)
    else:
        out.update(cache=None, cache_k=None, cache_v=None, cache_v_scale=None)
    return out
