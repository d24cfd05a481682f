"""Block-causal flash attention entry point, same signature as the reference.

``block_causal_flash_attention`` keeps the argument list, defaults, asserts and
output allocation of ``qwen_image_kernel/triton_attention.py:171-260`` and hands
the call to the gfx950 HIP kernel through the C ABI (``qik_attn_fwd_ws``, with
a workspace kept per device and stream).  The launch is asynchronous on the
current stream of the query's device, like the Triton launch it replaces.

Also here: ``build_prefix_lengths`` (the per-row causal-length array of
``processors.py:22-36``, built on the device in one launch) and
``tile_schedule`` (the host mirror of the kernel's KV-tile schedule).
"""

from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib

__all__ = [
    "block_causal_flash_attention",
    "build_prefix_lengths",
    "tile_schedule",
    "block_shape",
    "make_args",
]

_DTYPES = {torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_FP16}


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _bsh(t: torch.Tensor) -> tuple[int, int, int]:
    return (t.stride(0), t.stride(1), t.stride(2))


def _check_rows(name: str, t: torch.Tensor) -> None:
    if t.dim() != 4:
        raise ValueError(f"{name} must be [B, S, H, D], got shape {tuple(t.shape)}")
    if t.shape[-1] > 1 and t.stride(-1) != 1:
        raise ValueError(f"{name} must have unit stride along D (got stride {t.stride(-1)})")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor (the kernel runs on the GPU)")


def _kernel_layout(t: torch.Tensor, base: int = 16) -> torch.Tensor:
    """``t`` itself when the kernel can read it in place: base address a
    multiple of ``base`` bytes, b/s/h strides multiples of 8 elements (the
    copies move 16-byte chunks) and rows that do not overlap.  Otherwise a
    contiguous copy on the same device, so that every layout the reference's
    kernel takes (it reads any strides) gives a result here too, at the price
    of one read and one write of ``t``."""
    B, S, H, D = t.shape
    sb, ss, sh, _ = t.stride()
    if (t.data_ptr() % base == 0 and (B == 1 or sb % 8 == 0) and (H == 1 or sh % 8 == 0)
            and (S == 1 or (ss % 8 == 0 and ss >= D))):
        return t
    return t.clone(memory_format=torch.contiguous_format)


def make_args(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    prefix_lengths: torch.Tensor | None,
    kv_bytes: torch.Tensor | None,
    out: torch.Tensor,
    cache_k: torch.Tensor | None,
    cache_v: torch.Tensor | None,
    cache_v_scale: torch.Tensor | None,
    uniform: bool,
    debug_tiles: torch.Tensor | None = None,
) -> _lib.QikAttnArgs:
    """Fill the C argument struct from tensors (no device work)."""
    B, SQ, H, D = query.shape
    P = 0 if cache_k is None else cache_k.shape[1]
    a = _lib.QikAttnArgs()
    a.abi_version = _lib.ABI_VERSION
    a.dtype = _DTYPES[query.dtype]
    flags = 0
    if P > 0:
        flags |= _lib.HAS_CACHE
    if kv_bytes is not None:
        flags |= _lib.HAS_KEY_VALID
    if uniform:
        flags |= _lib.UNIFORM_L
    if cache_v_scale is not None:
        flags |= _lib.V_CACHE_FP8
    a.flags = flags
    a.q = _ptr(query)
    a.k_new = _ptr(key)
    a.v_new = _ptr(value)
    a.out = _ptr(out)
    a.prefix_lengths = _ptr(prefix_lengths)
    a.key_valid = _ptr(kv_bytes)
    a.debug_tiles = _ptr(debug_tiles)
    a.B, a.SQ, a.SN, a.P, a.H, a.D = B, SQ, key.shape[1], P, H, D
    a.stride_q = _lib._i64x3(*_bsh(query))
    a.stride_k_new = _lib._i64x3(*_bsh(key))
    a.stride_v_new = _lib._i64x3(*_bsh(value))
    a.stride_out = _lib._i64x3(*_bsh(out))
    if P > 0:
        a.k_cache = _ptr(cache_k)
        a.v_cache = _ptr(cache_v)
        a.stride_k_cache = _lib._i64x3(*_bsh(cache_k))
        a.stride_v_cache = _lib._i64x3(*_bsh(cache_v))
        a.v_scale = _ptr(cache_v_scale)
    a.stride_valid_b = kv_bytes.stride(0) if kv_bytes is not None else 0
    # fp32 D**-0.5, as the Triton launch passes query.shape[-1] ** -0.5 (triton_attention.py:240)
    a.sm_scale = float(D) ** -0.5
    return a


def block_causal_flash_attention(
    query: torch.Tensor,  # [B, SQ, H, D]
    key: torch.Tensor,  # [B, SN, H, D]  fresh keys
    value: torch.Tensor,  # [B, SN, H, D]
    prefix_lengths: torch.Tensor,  # [SQ] int32
    key_valid: torch.Tensor | None,  # [B, KV_TOTAL] bool or None
    cache_k: torch.Tensor | None = None,  # [B, P, H, D]
    cache_v: torch.Tensor | None = None,
    cache_v_scale: torch.Tensor | None = None,  # [B, H] fp32, only with fp8 cache V
    uniform_full: bool = False,  # caller guarantee: L == KV_TOTAL-1 for every row
    *,
    debug_tiles: torch.Tensor | None = None,
    split_tail: bool = True,
) -> torch.Tensor:
    """Exact block-causal attention via per-row prefix lengths.

    Row q attends key kv iff kv <= prefix_lengths[q] (and key_valid[b, kv] when
    given).  With ``cache_k``/``cache_v`` the keys/values are the virtual
    concatenation [cache, key] and ``prefix_lengths``/``key_valid`` index that
    absolute space; nothing is concatenated.  Rows with L = -1 produce zeros.
    With ``cache_v_scale`` the cache V is fp8e4m3fn dequantised per (b, h) as
    bf16(fp32(v) * scale).  Semantics: triton_attention.py:171-260.

    ``debug_tiles`` (keyword only, not in the reference) receives the number of
    KV tiles visited per (b, h, row block), int32 [B*H*cdiv(SQ, BM)].

    ``split_tail`` (keyword only, not in the reference): True (default) runs
    ``qik_attn_fwd_ws`` (resident workgroups pulling row blocks from per-XCD
    queues, the last partial round's row blocks split in two over their KV
    tiles) with a zeroed workspace kept per (device, stream); False runs
    ``qik_attn_fwd``, one workgroup per row block.
    """
    assert query.dtype in (torch.bfloat16, torch.float16), "fp16/bf16 only"
    B, SQ, H, D = query.shape
    if cache_k is not None:
        P = cache_k.shape[1]
        SN = key.shape[1]
        assert cache_k.shape[2] == H and key.shape[2] == H
        assert cache_k.dtype == key.dtype
    else:
        P = 0
        SN = key.shape[1]
    KV_TOTAL = P + SN
    assert key.dtype == query.dtype and value.dtype == query.dtype, "q/k/v dtypes must match"
    for name, t in (("query", query), ("key", key), ("value", value)):
        _check_rows(name, t)
    if P > 0:
        assert cache_v is not None and cache_v.shape[:3] == cache_k.shape[:3]
        _check_rows("cache_k", cache_k)
        _check_rows("cache_v", cache_v)
    dev = query.device
    for name, t in (("key", key), ("value", value)) + ((("cache_k", cache_k), ("cache_v", cache_v)) if P > 0 else ()):
        if t.device != dev:
            raise ValueError(f"{name} is on {t.device}, query on {dev}")

    out = torch.empty_like(query)
    if out.stride(-1) != 1:
        out = torch.empty(query.shape, dtype=query.dtype, device=dev)
    if out.numel() == 0:
        # no query rows (or heads): the reference's grid is empty and it
        # returns the empty output without a launch
        return out

    kv_bytes = None
    if key_valid is not None:
        _check_aux("key_valid", key_valid, dev)
        kv_bytes = key_valid.to(torch.uint8).contiguous()
        assert kv_bytes.dim() == 2 and kv_bytes.shape[1] >= KV_TOTAL, "key_valid must be [B, KV_TOTAL]"
        if kv_bytes.shape[0] not in (1, B):
            raise ValueError(f"key_valid batch dim must be 1 or B={B}, got {kv_bytes.shape[0]}")
        if kv_bytes.shape[0] == 1 and B > 1:
            kv_bytes = kv_bytes.expand(B, -1)

    v_fp8 = cache_v_scale is not None
    scale = None
    if v_fp8:
        assert cache_v is not None and cache_v.dtype == torch.float8_e4m3fn
        _check_aux("cache_v_scale", cache_v_scale, dev)
        scale = cache_v_scale
        if scale.dtype != torch.float32 or not scale.is_contiguous():
            scale = scale.float().contiguous()
        assert scale.numel() == B * H, "cache_v_scale must be [B, H]"
    elif P > 0:
        assert cache_v.dtype == query.dtype, "bf16/fp16 cache V must match the query dtype"

    uniform = uniform_full and key_valid is None

    L = None
    if not uniform:
        _check_aux("prefix_lengths", prefix_lengths, dev)
        L = prefix_lengths
        if L.dtype != torch.int32 or not L.is_contiguous():
            L = L.to(torch.int32).contiguous()
        assert L.numel() >= SQ, "prefix_lengths must be [SQ]"

    if debug_tiles is not None:
        _check_aux("debug_tiles", debug_tiles, dev)
        need = B * H * -(-SQ // block_shape()[0])
        if debug_tiles.dtype != torch.int32 or not debug_tiles.is_contiguous() or debug_tiles.numel() < need:
            raise ValueError(f"debug_tiles must be a contiguous int32 tensor of at least {need} elements")

    # with P == 0 the slab (and its fp8 scale) is never read (HAS_CACHE = P > 0, :250)
    if P == 0:
        cache_k = cache_v = scale = None
    st = _run(query, key, value, L, kv_bytes, out, cache_k, cache_v, scale, uniform, debug_tiles, split_tail, dev)
    if st == _ERR_ALIGN:
        # nothing was launched: a layout the kernel cannot read in place goes
        # through contiguous copies (the reference's kernel reads any strides)
        query, key, value = _kernel_layout(query), _kernel_layout(key), _kernel_layout(value)
        if cache_k is not None:
            cache_k = _kernel_layout(cache_k)
            cache_v = _kernel_layout(cache_v, 8 if cache_v.dtype == torch.float8_e4m3fn else 16)
        st = _run(query, key, value, L, kv_bytes, out, cache_k, cache_v, scale, uniform, debug_tiles, split_tail,
                  dev)
    _lib.check(st, "qik_attn_fwd_ws" if split_tail else "qik_attn_fwd")
    return out


_ERR_ALIGN = -8  # QIK_ERR_ALIGN


def _run(query, key, value, L, kv_bytes, out, cache_k, cache_v, scale, uniform, debug_tiles, split_tail, dev) -> int:
    """Argument struct (cached per geometry) and launch; the library's status."""
    args, ws_bytes = _cached_args(query, key, value, L, kv_bytes, out, cache_k, cache_v, scale, uniform,
                                  debug_tiles, split_tail)
    if args is None:
        return ws_bytes
    if dev.index is not None and dev.index != torch.cuda.current_device():
        with torch.cuda.device(dev):
            return _launch(args, dev, split_tail, ws_bytes)
    return _launch(args, dev, split_tail, ws_bytes)


def _check_aux(name: str, t: torch.Tensor, dev: torch.device) -> None:
    """The side inputs go to the kernel as raw device addresses: they must live on the query's device."""
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{name} must be a tensor on {dev}")
    if t.device != dev:
        raise ValueError(f"{name} is on {t.device}; it must be on the query's device {dev}")


# Argument structs by call geometry: everything of qik_attn_args except the
# data pointers, plus the workspace size the launch needs.  Building the
# struct and asking the library for the size cost more host time than a
# small launch takes on the device, so both are done once per geometry.
_ARGS_CACHE: dict = {}
_ARGS_CACHE_MAX = 256


def _geometry(query, key, value, L, kv_bytes, out, cache_k, cache_v, scale, uniform, debug, split_tail):
    return (
        query.device, query.dtype, tuple(query.shape), query.stride(), key.shape[1], key.stride(), value.stride(),
        out.stride(),
        None if cache_k is None else (cache_k.shape[1], cache_k.stride(), cache_v.stride(), cache_v.dtype),
        L is None, uniform, None if kv_bytes is None else kv_bytes.stride(0), scale is None, debug is None,
        split_tail,
    )


def _cached_args(query, key, value, L, kv_bytes, out, cache_k, cache_v, scale, uniform, debug, split_tail):
    gkey = _geometry(query, key, value, L, kv_bytes, out, cache_k, cache_v, scale, uniform, debug, split_tail)
    hit = _ARGS_CACHE.get(gkey)
    if hit is None:
        a = make_args(query, key, value, L, kv_bytes, out, cache_k, cache_v, scale, uniform, debug)
        lib = _lib.load()
        st = lib.qik_attn_validate(ctypes.byref(a))
        if st != 0:
            return None, st   # (None, status): not cached, nothing launched
        ws_bytes = 0
        if split_tail:
            nbytes = ctypes.c_int64(0)
            with torch.cuda.device(query.device):
                _lib.check(lib.qik_attn_workspace_size(ctypes.byref(a), ctypes.byref(nbytes)),
                           "qik_attn_workspace_size")
            ws_bytes = nbytes.value
        if len(_ARGS_CACHE) >= _ARGS_CACHE_MAX:
            _ARGS_CACHE.clear()
        _ARGS_CACHE[gkey] = (_lib.QikAttnArgs.from_buffer_copy(a), ws_bytes)
        return a, ws_bytes
    a = _lib.QikAttnArgs.from_buffer_copy(hit[0])
    a.q = query.data_ptr()
    a.k_new = key.data_ptr()
    a.v_new = value.data_ptr()
    a.out = out.data_ptr()
    a.prefix_lengths = None if L is None else L.data_ptr()
    a.key_valid = None if kv_bytes is None else kv_bytes.data_ptr()
    a.debug_tiles = None if debug is None else debug.data_ptr()
    if cache_k is not None:
        a.k_cache = cache_k.data_ptr()
        a.v_cache = cache_v.data_ptr()
        a.v_scale = None if scale is None else scale.data_ptr()
    return a, hit[1]


# (device index, stream handle) -> workspace of one stream, control words zero.
# Bounded: a program that cycles through many streams drops the oldest.
_WORKSPACES: dict = {}
_WORKSPACES_MAX = 16


def _workspace(dev: torch.device, stream: int, nbytes: int) -> torch.Tensor:
    """A workspace for qik_attn_fwd_ws whose control words are zero.

    Every launch leaves the control words (the first ``WS_CTL_BYTES``) zero
    again, so one workspace per (device, stream) is kept and reused; launches
    on one stream never overlap.  Under graph capture a fresh workspace is
    taken from the graph's pool instead, and only its control words are
    cleared (by a captured fill kernel), so a replay never shares the cached
    one with eager launches; the partial-state slots behind them are always
    written before they are read.
    """
    if torch.cuda.is_current_stream_capturing():
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        ws[: min(nbytes, _lib.WS_CTL_BYTES)].zero_()
        return ws
    key = (dev.index, stream)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        if ws is None and len(_WORKSPACES) >= _WORKSPACES_MAX:
            _WORKSPACES.pop(next(iter(_WORKSPACES)))
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        ws[: min(nbytes, _lib.WS_CTL_BYTES)].zero_()
        _WORKSPACES[key] = ws
    return ws


def _current_stream(dev: torch.device) -> int:
    """Raw handle of the current stream of ``dev`` (the current device)."""
    return torch._C._cuda_getCurrentRawStream(dev.index if dev.index is not None else torch.cuda.current_device())


def _launch(args: _lib.QikAttnArgs, dev: torch.device, split_tail: bool, ws_bytes: int) -> int:
    """Enqueue the kernel on the current stream of ``dev`` (the current device); the status."""
    lib = _lib.load()
    handle = _current_stream(dev)
    stream = ctypes.c_void_p(handle)
    if not split_tail:
        return lib.qik_attn_fwd(ctypes.byref(args), stream)
    ws = None if ws_bytes == 0 else _workspace(dev if dev.index is not None else
                                               torch.device("cuda", torch.cuda.current_device()),
                                               handle, ws_bytes)
    return lib.qik_attn_fwd_ws(ctypes.byref(args), None if ws is None else ws.data_ptr(), ws_bytes, stream)


def _norm_slice(start: int, stop: int | None, n: int) -> tuple[int, int]:
    s, e, _ = slice(start, stop).indices(n)
    return s, max(s, e)


def build_prefix_lengths(
    segments: list[tuple[int, int, bool]], prefix_len: int, seq_len: int, device: torch.device
) -> torch.Tensor:
    """Per-row inclusive kv limit L: row q attends iff kv <= L[q] (processors.py:22-36).

    text run (s, e)      -> L[s:e] = s..e-1  (causal)
    image run (s, e)     -> L[s:e] = e-1     (bidirectional block + full prefix)
    target rows [P, S)   -> L = S-1          (full attention)

    The fill value of an image run is ``end - 1`` even when ``end`` exceeds
    ``seq_len``, and ``prefix_len`` follows Python slice semantics, as the
    reference's slice assignments do.  Negative segment bounds raise ValueError
    (the reference would write negative lengths).  The array is filled on
    ``device`` by one HIP launch.
    """
    device = torch.device(device)
    if device.type != "cuda":
        raise ValueError("build_prefix_lengths builds L on the GPU; pass a device tensor's device")
    L = torch.empty(seq_len, dtype=torch.int32, device=device)
    rows = []
    for s, e, is_text in segments:
        if s < 0 or e < 0:
            raise ValueError(f"segment ({s}, {e}) has a negative bound")
        if e > s:  # an empty or reversed slice assigns nothing
            rows.append((s, e, 1 if is_text else 0))
    segs = np.zeros((max(len(rows), 1), 3), dtype=np.int32)
    for i, r in enumerate(rows):
        segs[i] = r
    pe, _ = _norm_slice(prefix_len, None, seq_len)
    lib = _lib.load()
    with torch.cuda.device(device):
        stream = torch.cuda.current_stream(device).cuda_stream
        st = lib.qik_build_prefix_lengths(
            segs.ctypes.data, len(rows), pe, seq_len, L.data_ptr(), ctypes.c_void_p(stream)
        )
    _lib.check(st, "qik_build_prefix_lengths")
    return L


def block_shape() -> tuple[int, int]:
    """(BM, BN): query rows per workgroup and keys per KV tile of the kernel."""
    bm, bn = ctypes.c_int32(), ctypes.c_int32()
    _lib.check(_lib.load().qik_attn_block_shape(ctypes.byref(bm), ctypes.byref(bn)), "qik_attn_block_shape")
    return bm.value, bn.value


def tile_schedule(
    SQ: int, P: int, SN: int, prefix_lengths: np.ndarray | torch.Tensor | None, uniform: bool
) -> np.ndarray:
    """KV tiles the kernel visits per row block (host computation, no device).

    Returns int32 [cdiv(SQ, BM)]; the same numbers the kernel writes into
    ``debug_tiles`` for every (b, h).
    """
    bm, _ = block_shape()
    flags = (_lib.HAS_CACHE if P > 0 else 0) | (_lib.UNIFORM_L if uniform else 0)
    Lh = None
    if not uniform:
        if isinstance(prefix_lengths, torch.Tensor):
            prefix_lengths = prefix_lengths.detach().cpu().numpy()
        Lh = np.ascontiguousarray(prefix_lengths, dtype=np.int32)
        assert Lh.size >= SQ
    out = np.zeros(max(-(-SQ // bm), 1), dtype=np.int32)
    st = _lib.load().qik_attn_tile_schedule(
        SQ, P, SN, flags, None if Lh is None else Lh.ctypes.data, out.ctypes.data
    )
    _lib.check(st, "qik_attn_tile_schedule")
    return out[: -(-SQ // bm)]
