"""Contiguous prefix-KV slab, same attributes and layout as the reference.

``ContiguousKVCache`` / ``_LayerView`` keep the API of
``qwen_image_kernel/kv_cache.py:23-95``: one preallocated slab for all layers,
K ``[L, B, H, P_max, D]`` in the model dtype, V the same or fp8e4m3fn with one
fp32 scale per (layer, b, h), and ``lengths [L]`` int64 on the device.  Each
head's prefix tokens are dense (256 B rows of bf16 K, 128 B rows of fp8 V), and
``views()`` returns ``[B, P, H, D]`` strided views that the attention kernel
reads in place.

``store`` on a HIP device is one call of ``qik_slab_store_ws`` (include/qik_ops.h):
the transposed copy of K (and of a bf16 V) and, for an fp8 slab, the per-(b, h)
amax, scale and e4m3fn codes of V, bit-identical to the torch ops of
kv_cache.py:36-42 run on the same device, in two launches with a small
workspace that the cache keeps per (device, stream).  A slab on the CPU (the
reference's own CPU-runnable case) runs those torch ops.

Difference from the reference: the prefix length of each layer is also kept on
the host, so ``get()``/``views()`` do not synchronise the device
(the reference reads ``int(lengths[layer])``, kv_cache.py:49, 56).
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .attention import _kernel_layout

FP8_E4M3_MAX = 448.0


class _LayerView:
    """Per-layer store/get interface compatible with the stock cache."""

    def __init__(self, cache: "ContiguousKVCache", layer: int):
        self._c = cache
        self._layer = layer

    def store(self, k: torch.Tensor, v: torch.Tensor) -> None:
        """k, v: [B, P, H, D] post-RoPE; V is quantised per (b, h) when the slab is fp8.

        Quantisation (kv_cache.py:36-42): scale = max(amax|v| / 448, 1e-12) in
        fp32, code = e4m3fn(clamp(v / scale, +-448)) with a true fp32 division
        and round-to-nearest-even.
        """
        c = self._c
        P = k.shape[1]
        if P > c.capacity:
            raise ValueError(f"prefix of {P} tokens exceeds the slab capacity {c.capacity}")
        if c.k_buf.is_cuda and P > 0 and k.shape[0] > 0 and k.shape[2] > 0:
            # the store's first launch also writes lengths[layer] = P
            self._store_device(k, v, P)
        else:
            if c.k_buf.is_cuda:
                self._store_device(k, v, P)
            else:
                self._store_torch(k, v, P)
            # a fill kernel: assigning a Python int to one element is a
            # host-to-device copy, which a stream under graph capture rejects
            c.lengths[self._layer:self._layer + 1].fill_(P)
        c._host_lengths[self._layer] = P

    def _store_device(self, k: torch.Tensor, v: torch.Tensor, P: int) -> None:
        c = self._c
        kd = c.k_buf
        # inputs the kernels cannot read in place (a base off 16 bytes, odd
        # strides) go through contiguous copies; other dtypes or devices are
        # converted (into fresh tensors) by store_args
        if k.dim() == 4 and k.device == kd.device and k.dtype == kd.dtype:
            k = _kernel_layout(k)
        if v.dim() == 4 and v.device == kd.device and v.dtype == kd.dtype:
            v = _kernel_layout(v)
        a, keep, nbytes = self._cached_store_args(k, v, P)
        lib = _lib.load()
        idx = kd.device.index
        if idx != torch.cuda.current_device():
            with torch.cuda.device(kd.device):
                self._launch_store(lib, a, nbytes, idx)
        else:
            self._launch_store(lib, a, nbytes, idx)
        del keep

    def _launch_store(self, lib, a, nbytes: int, idx: int) -> None:
        handle = torch._C._cuda_getCurrentRawStream(idx)
        ws = self._c._workspace(idx, handle, nbytes)
        _lib.check(lib.qik_slab_store_ws(ctypes.byref(a), ws, nbytes, ctypes.c_void_p(handle)), "qik_slab_store_ws")

    def _cached_store_args(self, k: torch.Tensor, v: torch.Tensor, P: int):
        """store_args with the struct and its workspace size kept per geometry (layer, shapes, strides)."""
        c = self._c
        gkey = (self._layer, P, tuple(k.shape), k.stride(), v.stride(), k.dtype, v.dtype, k.device, v.device)
        hit = c._args_cache.get(gkey)
        if hit is None:
            a, keep = self.store_args(k, v, P)
            nbytes = ctypes.c_int64(0)
            with torch.cuda.device(c.k_buf.device):
                _lib.check(_lib.load().qik_slab_store_workspace_size(ctypes.byref(a), ctypes.byref(nbytes)),
                           "qik_slab_store_workspace_size")
            if len(c._args_cache) >= 4 * max(c.num_layers, 1):
                c._args_cache.clear()
            # only inputs already in the slab's dtype, device and a unit D stride are
            # launched from the cached struct; others are converted per call
            if keep[0] is k and keep[1] is v:
                c._args_cache[gkey] = (_lib.QikSlabStoreArgs.from_buffer_copy(a), nbytes.value)
            return a, keep, nbytes.value
        a = _lib.QikSlabStoreArgs.from_buffer_copy(hit[0])
        a.k = k.data_ptr()
        a.v = v.data_ptr()
        return a, (k, v), hit[1]

    def store_args(self, k: torch.Tensor, v: torch.Tensor, P: int):
        """(qik_slab_store argument struct, tensors it points into) for a device slab."""
        c = self._c
        if k.shape != v.shape or k.dim() != 4 or tuple(k.shape[2:]) != tuple(c.k_buf.shape[2:3] + c.k_buf.shape[4:]):
            raise ValueError(f"k, v must be [B, P, H, D] matching the slab, got {tuple(k.shape)}, {tuple(v.shape)}")
        if k.shape[0] != c.batch_size:
            raise ValueError(f"batch {k.shape[0]} != slab batch {c.batch_size}")
        k = k.to(device=c.k_buf.device, dtype=c.k_buf.dtype)
        v = v.to(device=c.k_buf.device, dtype=c.k_buf.dtype)
        if k.stride(-1) != 1:
            k = k.contiguous()
        if v.stride(-1) != 1:
            v = v.contiguous()
        kd = c.k_buf[self._layer]
        vd = c.v_buf[self._layer]
        a = _lib.QikSlabStoreArgs()
        a.abi_version = _lib.ABI_VERSION
        a.dtype = _lib.DTYPE_BF16 if c.k_buf.dtype == torch.bfloat16 else _lib.DTYPE_FP16
        a.v_fp8 = 1 if c.v_fp8 else 0
        a.k = k.data_ptr()
        a.v = v.data_ptr()
        a.k_dst = kd.data_ptr()
        a.v_dst = vd.data_ptr()
        a.v_scale = c.v_scale[self._layer].data_ptr() if c.v_fp8 else None
        a.B, a.P, a.H, a.D = k.shape[0], P, k.shape[2], k.shape[3]
        a.stride_k = _lib._i64x3(k.stride(0), k.stride(1), k.stride(2))
        a.stride_v = _lib._i64x3(v.stride(0), v.stride(1), v.stride(2))
        a.stride_k_dst = _lib._i64x3(kd.stride(0), kd.stride(1), kd.stride(2))
        a.stride_v_dst = _lib._i64x3(vd.stride(0), vd.stride(1), vd.stride(2))
        a.length_dst = c.lengths.data_ptr() + c.lengths.element_size() * self._layer
        return a, (k, v)

    def _store_torch(self, k: torch.Tensor, v: torch.Tensor, P: int) -> None:
        c = self._c
        c.k_buf[self._layer, :, :, :P, :].copy_(k.transpose(1, 2))
        if c.v_fp8:
            vt = v.transpose(1, 2).float()
            scale = vt.abs().amax(dim=(2, 3)).float() / FP8_E4M3_MAX
            scale = scale.clamp_min(1e-12)
            vq = (vt / scale[:, :, None, None]).clamp(-FP8_E4M3_MAX, FP8_E4M3_MAX).to(torch.float8_e4m3fn)
            c.v_buf[self._layer, :, :, :P, :].copy_(vq)
            c.v_scale[self._layer].copy_(scale)
        else:
            c.v_buf[self._layer, :, :, :P, :].copy_(v.transpose(1, 2))

    def get(self):
        """(k, v) as [B, P, H, D] strided views."""
        P = self._c._host_lengths[self._layer]
        k = self._c.k_buf[self._layer, :, :, :P, :].transpose(1, 2)
        v = self._c.v_buf[self._layer, :, :, :P, :].transpose(1, 2)
        return k, v

    def views(self):
        """(k, v, v_scale_or_None) for block_causal_flash_attention."""
        P = self._c._host_lengths[self._layer]
        k = self._c.k_buf[self._layer, :, :, :P, :].transpose(1, 2)
        v = self._c.v_buf[self._layer, :, :, :P, :].transpose(1, 2)
        scale = self._c.v_scale[self._layer] if self._c.v_fp8 else None
        return k, v, scale


class ContiguousKVCache:
    """Single-slab prefix KV cache: one allocation per buffer for all layers.

    K layout: [L, B, H, P_max, D] (dtype).  V layout: same (dtype) or fp8e4m3fn
    with per-head fp32 scales [L, B, H].  Per prefix token across 32 layers at
    H*D = 3072: K+V bf16 = 384 KB, K bf16 + V fp8 = 288 KB.
    """

    def __init__(
        self,
        num_layers: int,
        batch: int,
        prefix_max: int,
        num_heads: int,
        head_dim: int,
        v_fp8: bool = False,
        device: torch.device | str = "cuda",
        dtype: torch.dtype = torch.bfloat16,
    ):
        if torch.device(device).type != "cpu" and dtype not in (torch.bfloat16, torch.float16):
            # the device store and the attention kernel read 2-byte K/V
            # elements; a CPU slab (stored by torch's ops, as the reference's
            # cache does) takes any dtype
            raise ValueError(f"a device slab's dtype must be bfloat16 or float16, got {dtype}")
        self.v_fp8 = v_fp8
        self.num_layers = num_layers
        self.capacity = prefix_max
        self.batch_size = batch
        self.k_buf = torch.empty(num_layers, batch, num_heads, prefix_max, head_dim, dtype=dtype, device=device)
        v_dtype = torch.float8_e4m3fn if v_fp8 else dtype
        self.v_buf = torch.empty(num_layers, batch, num_heads, prefix_max, head_dim, dtype=v_dtype, device=device)
        self.v_scale = torch.empty(num_layers, batch, num_heads, dtype=torch.float32, device=device)
        self.lengths = torch.zeros(num_layers, dtype=torch.int64, device=device)
        self._host_lengths = [0] * num_layers
        self._ws: dict = {}   # (device index, stream) -> store workspace (fp8 slab)
        self._args_cache: dict = {}  # store geometry -> (argument struct, workspace bytes)
        self.layers = [_LayerView(self, i) for i in range(num_layers)]

    def _workspace(self, device_index: int, stream: int, nbytes: int):
        """Device pointer of this cache's store workspace for `stream` (None when none is needed).

        Its contents never need clearing: every store writes what it reads.
        Stores on different streams get different workspaces.
        """
        if nbytes <= 0:
            return None
        key = (device_index, stream)
        ws = self._ws.get(key)
        if ws is None or ws.numel() < nbytes:
            if ws is None and len(self._ws) >= 16:
                self._ws.pop(next(iter(self._ws)))
            ws = torch.empty(nbytes, dtype=torch.uint8, device=torch.device("cuda", device_index))
            self._ws[key] = ws
        return ws.data_ptr()

    def get_layer(self, i: int) -> _LayerView:
        return self.layers[i]
