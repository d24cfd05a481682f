"""W8A8 fp8 linear layers, same API as ``qwen_image_kernel/fp8.py``.

``FP8Linear`` keeps the reference module's constructor, buffers (``weight``
fp8e4m3fn ``[out, in]``, ``weight_scale`` fp32 ``[1]``, ``bias`` bf16 or
None), ``forward`` and ``from_linear`` (fp8.py:63-101); ``compute_scale``,
``quantize_tensorwise``, ``quantize_weight_tensorwise``, ``convert_linears_fp8``
and ``fp8_state_dict`` keep their signatures and results (fp8.py:24-60,
104-128).  The device work runs in the gfx950 HIP kernels behind
include/qik_fp8.h, asynchronously on the current stream:

* ``quantize_tensorwise`` / ``quantize_weight_tensorwise``: ``qik_fp8_quantize``
  (two launches: per-block maxima, then the scale and the codes), in place of
  the reference's torch amax + Triton cast kernel (fp8.py:24-53) and torch
  division chain (fp8.py:56-60);
* the GEMM: ``qik_fp8_gemm`` on the fp8 matrix cores, in place of
  ``torch._scaled_mm`` with tensorwise scales (fp8.py:87-88);
* the bf16 path of layers with fewer than 256 inputs (fp8.py:79-84): the
  weight is dequantised by ``qik_fp8_dequant`` and multiplied by
  ``torch.nn.functional.linear``, as in the reference.

A weight that lives on the CPU is quantised on the CPU by the library's host
routine ``qik_fp8_quantize_weight_host``, bit-identical to the reference's
torch ops run on the CPU (where both divisions are true fp32 divisions), so the
offline conversion runs on a machine without a GPU as the reference's does
(quantize_offline.py:15-25).  A weight on a HIP device gets the scale torch
forms there (the amax times the fp32 reciprocal of 448).

``FP8Linear`` keeps a small per-module cache of prepared launch arguments.  It
holds no tensor (weak references only), is dropped by ``.to()``/``.cuda()``/
``.half()`` and by copying or pickling the module, so the module moves,
copies and frees its buffers exactly as the reference's does.
"""

from __future__ import annotations

import ctypes
import weakref

import torch
import torch.nn as nn

from . import _lib

__all__ = [
    "FP8_E4M3_MAX",
    "compute_scale",
    "quantize_tensorwise",
    "quantize_weight_tensorwise",
    "fp8_linear",
    "FP8Linear",
    "convert_linears_fp8",
    "fp8_state_dict",
]

FP8_E4M3_MAX = 448.0

_IN_DTYPES = {torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_FP16, torch.float32: _lib.DTYPE_FP32}
_OUT_DTYPES = {torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_FP16}
# element types qik_fp8_dequant writes
_DEQUANT_DTYPES = _IN_DTYPES

# workspace of the quantiser, one per (device, stream): zero-filled once when
# created, and every call leaves it that way (include/qik_fp8.h)
_QUANT_WS: dict = {}
_GEMM_WS: dict = {}   # (device index, stream) -> fp32 workspace of the K-split GEMMs


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _quant_workspace(dev: torch.device, stream: int, nbytes: int) -> torch.Tensor:
    """Partial-maximum workspace of the quantiser on this stream.  Under graph
    capture a fresh one from the graph's pool, so that replays of different
    graphs (or a replay beside eager work) never share one."""
    if torch.cuda.is_current_stream_capturing():
        # torch.zeros records a fill kernel, not a memset node
        return torch.zeros(max(nbytes // 4, 1024), dtype=torch.int32, device=dev)
    key = (dev.index, stream)
    ws = _QUANT_WS.get(key)
    if ws is None or ws.numel() * 4 < nbytes:
        if len(_QUANT_WS) >= 64:
            _QUANT_WS.clear()
        ws = _QUANT_WS[key] = torch.zeros(max(nbytes // 4, 1024), dtype=torch.int32, device=dev)
    return ws


def _gemm_workspace(dev: torch.device, stream: int, nbytes: int) -> torch.Tensor | None:
    """A workspace of at least nbytes for qik_fp8_gemm_ws on this stream
    (None when the call needs none).  One per (device, stream), grown as
    needed: calls on one stream run in order, so they can share it.  Under
    graph capture a fresh one from the graph's pool (the split-K sums of two
    graphs replayed on different streams must not share memory)."""
    if nbytes <= 0:
        return None
    if torch.cuda.is_current_stream_capturing():
        return torch.empty((nbytes + 3) // 4, dtype=torch.float32, device=dev)
    key = (dev.index, stream)
    ws = _GEMM_WS.get(key)
    if ws is None or ws.numel() * 4 < nbytes:
        if len(_GEMM_WS) >= 64:
            _GEMM_WS.clear()
        ws = _GEMM_WS[key] = torch.empty((nbytes + 3) // 4, dtype=torch.float32, device=dev)
    return ws


def quant_args(flat: torch.Tensor, out: torch.Tensor, scale: torch.Tensor, mode: int) -> _lib.QikFp8QuantArgs:
    """The qik_fp8_quantize argument struct for a contiguous device tensor (no device work)."""
    a = _lib.QikFp8QuantArgs()
    a.abi_version = _lib.ABI_VERSION
    a.dtype = _IN_DTYPES[flat.dtype]
    a.mode = mode
    a.x = flat.data_ptr()
    a.out = out.data_ptr()
    a.scale = scale.data_ptr()
    a.n = flat.numel()
    return a


def _quantize(x: torch.Tensor, mode: int) -> tuple[torch.Tensor, torch.Tensor]:
    """codes (x's shape, fp8e4m3fn) and scale ([1] fp32) of a device tensor."""
    if not x.is_cuda:
        raise ValueError("the fp8 quantiser runs on a HIP device; move the tensor there first")
    if x.dtype not in _IN_DTYPES:
        raise ValueError(f"quantiser input must be bf16, fp16 or fp32, got {x.dtype}")
    if x.numel() == 0:
        raise ValueError("cannot quantise an empty tensor (its amax is undefined)")
    flat = x.reshape(-1)
    if not flat.is_contiguous() or flat.data_ptr() % 16 != 0:
        flat = flat.clone(memory_format=torch.contiguous_format)
    dev = x.device
    out = torch.empty(flat.shape, dtype=torch.float8_e4m3fn, device=dev)
    scale = torch.empty(1, dtype=torch.float32, device=dev)
    a = quant_args(flat, out, scale, mode)
    lib = _lib.load()
    with torch.cuda.device(dev):
        need = ctypes.c_int64(0)
        _lib.check(lib.qik_fp8_quant_workspace_size(ctypes.byref(a), ctypes.byref(need)), "qik_fp8_quant_workspace_size")
        s = _stream(dev)
        ws = _quant_workspace(dev, s, need.value)
        _lib.check(lib.qik_fp8_quantize(ctypes.byref(a), ws.data_ptr(), ws.numel() * 4, s), "qik_fp8_quantize")
    return out.view(x.shape), scale


def compute_scale(x: torch.Tensor) -> torch.Tensor:
    """Dynamic per-tensor fp8 activation scale (fp32 0-d tensor, on the device): max(amax/448, 1e-12)."""
    return _quantize(x, _lib.FP8_ACTIVATION)[1].reshape(())


def quantize_tensorwise(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """[M, K] -> (fp8 codes e4m3(x * (1/scale)), scale [1]) (fp8.py:43-53)."""
    return _quantize(x, _lib.FP8_ACTIVATION)


def quantize_weight_tensorwise(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """[N, K] -> (fp8 codes e4m3(clamp(w / scale, +-448)), scale [1]) (fp8.py:56-60).

    On a HIP device: the device quantiser.  A CPU tensor is quantised on the
    CPU by the library's host routine, with the results torch's CPU ops give
    (the reference's offline conversion runs there, quantize_offline.py:15-25)."""
    if w.is_cuda:
        return _quantize(w, _lib.FP8_WEIGHT)
    if w.device.type != "cpu":
        raise ValueError(f"quantize_weight_tensorwise takes a HIP or CPU tensor, got {w.device}")
    if w.dtype not in _IN_DTYPES:
        raise ValueError(f"quantiser input must be bf16, fp16 or fp32, got {w.dtype}")
    if w.numel() == 0:
        raise ValueError("cannot quantise an empty tensor (its amax is undefined)")
    wc = w.contiguous()
    codes = torch.empty(w.shape, dtype=torch.float8_e4m3fn)
    scale = torch.empty(1, dtype=torch.float32)
    _lib.check(_lib.load().qik_fp8_quantize_weight_host(wc.data_ptr(), _IN_DTYPES[wc.dtype], wc.numel(),
                                                        codes.data_ptr(), scale.data_ptr(),
                                                        torch.get_num_threads()),
               "qik_fp8_quantize_weight_host")
    return codes, scale


def _dequant_weight(w: torch.Tensor, scale: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """fp32(w) * scale (fp8.py:81) in `dtype` when that is bf16, fp16 or fp32
    (rounded once, or the fp32 product itself); for any other dtype the fp32
    product, which the caller converts as the reference's ``w.to(x.dtype)``
    does."""
    if not w.is_cuda:
        raise ValueError("FP8Linear runs on a HIP device; move the module there first")
    kdt = dtype if dtype in _DEQUANT_DTYPES else torch.float32
    wc = w.contiguous()
    out = torch.empty(wc.shape, dtype=kdt, device=w.device)
    sc = scale.to(device=w.device, dtype=torch.float32).contiguous()
    lib = _lib.load()
    with torch.cuda.device(w.device):
        _lib.check(
            lib.qik_fp8_dequant(wc.data_ptr(), sc.data_ptr(), out.data_ptr(), wc.numel(), _DEQUANT_DTYPES[kdt],
                                _stream(w.device)),
            "qik_fp8_dequant",
        )
    return out


def _gemm_args(xq, w, s_a, s_w, bias, out) -> _lib.QikFp8GemmArgs:
    a = _lib.QikFp8GemmArgs()
    a.abi_version = _lib.ABI_VERSION
    a.out_dtype = _OUT_DTYPES[out.dtype]
    a.a = xq.data_ptr()
    a.w = w.data_ptr()
    a.scale_a = s_a.data_ptr()
    a.scale_w = s_w.data_ptr()
    a.bias = bias.data_ptr() if bias is not None else None
    a.out = out.data_ptr()
    a.M, a.K = xq.shape
    a.N = w.shape[0]
    a.lda = xq.stride(0)
    a.ldw = w.stride(0)
    a.ldc = out.stride(0)
    return a


def fp8_linear(
    xq: torch.Tensor,             # [M, K] fp8e4m3fn
    w: torch.Tensor,              # [N, K] fp8e4m3fn
    scale_a: torch.Tensor,        # [1] fp32
    scale_w: torch.Tensor,        # [1] fp32
    bias: torch.Tensor | None = None,   # [N] in out_dtype
    out_dtype: torch.dtype = torch.bfloat16,
) -> torch.Tensor:
    """round((xq . w^T) * (scale_a * scale_w) + bias): what
    ``torch._scaled_mm(xq, w.t(), scale_a=..., scale_b=..., bias=..., out_dtype=...)``
    computes with tensorwise scales (fp8.py:87-88)."""
    if xq.dim() != 2 or w.dim() != 2 or xq.shape[1] != w.shape[1]:
        raise ValueError(f"shapes {tuple(xq.shape)} and {tuple(w.shape)} do not multiply as A . W^T")
    if xq.dtype != torch.float8_e4m3fn or w.dtype != torch.float8_e4m3fn:
        raise ValueError("fp8_linear takes float8_e4m3fn operands")
    if out_dtype not in _OUT_DTYPES:
        raise ValueError(f"out_dtype must be bf16 or fp16, got {out_dtype}")
    dev = xq.device
    for name, t in (("w", w), ("scale_a", scale_a), ("scale_w", scale_w), ("bias", bias)):
        if t is not None and (not t.is_cuda or t.device != dev):
            raise ValueError(f"{name} must be on {dev}")
    if xq.stride(1) != 1:
        xq = xq.contiguous()
    if w.stride(1) != 1:
        w = w.contiguous()
    sa = scale_a.reshape(1).to(torch.float32).contiguous()
    sw = scale_w.reshape(1).to(torch.float32).contiguous()
    b = None
    if bias is not None:
        if bias.numel() != w.shape[0]:
            raise ValueError(f"bias must have {w.shape[0]} elements, got {bias.numel()}")
        b = bias.reshape(-1).to(out_dtype).contiguous()
    out = torch.empty((xq.shape[0], w.shape[0]), dtype=out_dtype, device=dev)
    if xq.shape[0] == 0:
        return out
    a = _gemm_args(xq, w, sa, sw, b, out)
    lib = _lib.load()
    with torch.cuda.device(dev):
        need = ctypes.c_int64(0)
        _lib.check(lib.qik_fp8_gemm_workspace_size(ctypes.byref(a), ctypes.byref(need)), "qik_fp8_gemm")
        stream = _stream(dev)
        ws = _gemm_workspace(dev, stream, need.value)
        _lib.check(lib.qik_fp8_gemm_ws(ctypes.byref(a), None if ws is None else ws.data_ptr(), need.value, stream),
                   "qik_fp8_gemm")
    return out


class _LinearCall:
    """What one FP8Linear.forward input geometry needs at call time: the
    argument structs of the quantise + GEMM pair, and weak references to the
    weight, scale and bias they were made for (with those tensors' versions),
    so that the entry is used only while the module still holds exactly them
    and never keeps them alive."""

    __slots__ = ("fast", "index", "xq_shape", "out_shape", "result_shape", "ws_bytes", "gws_bytes", "qargs", "gargs",
                 "refs", "versions")

    def matches(self, weight, wscale, bias) -> bool:
        r = self.refs
        if r[0]() is not weight or r[1]() is not wscale:
            return False
        if (r[2] is None) != (bias is None) or (bias is not None and r[2]() is not bias):
            return False
        return self.versions == (weight._version, wscale._version, None if bias is None else bias._version)


def _prepare_linear(x, weight, wscale, bias, out_features) -> _LinearCall:
    """Checks and argument templates of the quantise + GEMM pair for one input
    geometry.  Inputs the fast path does not take (non-contiguous x, a host
    tensor, an empty batch, operands that need converting) run the general
    path, which checks them per call."""
    c = _LinearCall()
    c.index = x.device.index
    c.refs = (weakref.ref(weight), weakref.ref(wscale), None if bias is None else weakref.ref(bias))
    c.versions = (weight._version, wscale._version, None if bias is None else bias._version)
    K = x.shape[-1]
    M = x.numel() // K if K > 0 else 0
    c.xq_shape = (M, K)
    c.out_shape = (M, out_features)
    c.result_shape = (*x.shape[:-1], out_features)
    c.fast = bool(
        x.is_cuda and x.is_contiguous() and M > 0 and x.dtype in _IN_DTYPES
        and weight.is_cuda and weight.device == x.device and weight.dtype == torch.float8_e4m3fn
        and weight.dim() == 2 and weight.shape[1] == K and weight.shape[0] == out_features and weight.stride(1) == 1
        and wscale.is_cuda and wscale.device == x.device and wscale.dtype == torch.float32 and wscale.numel() == 1
        and (bias is None or (bias.is_cuda and bias.device == x.device and bias.dtype == torch.bfloat16
                              and bias.is_contiguous() and bias.numel() == out_features)))
    if not c.fast:
        return c
    lib = _lib.load()
    xq = torch.empty(c.xq_shape, dtype=torch.float8_e4m3fn, device=x.device)
    s_a = torch.empty(1, dtype=torch.float32, device=x.device)
    out = torch.empty(c.out_shape, dtype=torch.bfloat16, device=x.device)
    c.qargs = quant_args(x.reshape(-1), xq, s_a, _lib.FP8_ACTIVATION)
    need = ctypes.c_int64(0)
    _lib.check(lib.qik_fp8_quant_workspace_size(ctypes.byref(c.qargs), ctypes.byref(need)),
               "qik_fp8_quant_workspace_size")
    c.ws_bytes = need.value
    c.gargs = _gemm_args(xq, weight, s_a, wscale, bias, out)
    need = ctypes.c_int64(0)
    _lib.check(lib.qik_fp8_gemm_workspace_size(ctypes.byref(c.gargs), ctypes.byref(need)), "qik_fp8_gemm")
    c.gws_bytes = need.value
    return c


class FP8Linear(nn.Module):
    """Drop-in replacement for nn.Linear with fp8 weights and dynamic
    per-tensor activation quantisation (fp8.py:63-90)."""

    def __init__(self, in_features: int, out_features: int, bias: bool = False):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.register_buffer("weight", torch.zeros(out_features, in_features, dtype=torch.float8_e4m3fn))
        self.register_buffer("weight_scale", torch.ones(1, dtype=torch.float32))
        if bias:
            self.register_buffer("bias", torch.zeros(out_features, dtype=torch.bfloat16))
        else:
            self.bias = None

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.in_features < 256:
            # layers with few inputs (img_in, K = 64) run in bf16 on the
            # dequantised weight, as the reference does (fp8.py:79-84)
            w = _dequant_weight(self.weight, self.weight_scale, x.dtype)
            out = torch.nn.functional.linear(x, w.to(x.dtype), self.bias)
            return out.to(x.dtype)
        weight, wscale, bias = self.weight, self.weight_scale, self.bias
        key = (x.shape, x.stride(), x.dtype, x.device)
        calls = self.__dict__.get("_calls")
        if calls is None:
            calls = self.__dict__["_calls"] = {}
        ent = calls.get(key)
        if ent is None or not ent.matches(weight, wscale, bias):
            ent = _prepare_linear(x, weight, wscale, bias, self.out_features)
            if len(calls) >= 8:
                calls.clear()
            calls[key] = ent
        idx = ent.index
        if ent.fast and x.data_ptr() % 16 == 0 and idx == torch.cuda.current_device():
            # quantise x and multiply: the argument structs of both launches
            # are prepared per input geometry, only the data pointers change
            lib = _lib.load()
            stream = torch._C._cuda_getCurrentRawStream(idx)
            ws = _QUANT_WS.get((idx, stream))
            if ws is None or ws.numel() * 4 < ent.ws_bytes or torch.cuda.is_current_stream_capturing():
                ws = _quant_workspace(x.device, stream, ent.ws_bytes)
            xq = torch.empty(ent.xq_shape, dtype=torch.float8_e4m3fn, device=x.device)
            s_a = torch.empty(1, dtype=torch.float32, device=x.device)
            out = torch.empty(ent.out_shape, dtype=torch.bfloat16, device=x.device)
            qa = _lib.QikFp8QuantArgs.from_buffer_copy(ent.qargs)
            qa.x = x.data_ptr()
            qa.out = xq.data_ptr()
            qa.scale = s_a.data_ptr()
            _lib.check(lib.qik_fp8_quantize(ctypes.byref(qa), ws.data_ptr(), ws.numel() * 4, stream),
                       "qik_fp8_quantize")
            ga = _lib.QikFp8GemmArgs.from_buffer_copy(ent.gargs)
            ga.a = xq.data_ptr()
            ga.scale_a = s_a.data_ptr()
            ga.out = out.data_ptr()
            gws = _gemm_workspace(x.device, stream, ent.gws_bytes)
            _lib.check(lib.qik_fp8_gemm_ws(ctypes.byref(ga), None if gws is None else gws.data_ptr(), ent.gws_bytes,
                                           stream), "qik_fp8_gemm")
        else:
            x2 = x.reshape(-1, x.shape[-1])
            xq, s_a = quantize_tensorwise(x2)
            out = fp8_linear(xq, weight, s_a, wscale, bias, torch.bfloat16)
        out = out.view(ent.result_shape)
        return out.to(x.dtype) if out.dtype != x.dtype else out

    def _apply(self, fn, recurse=True):
        # .to() / .cuda() / .half() replace the buffers: drop the launch cache
        self.__dict__.pop("_calls", None)
        return super()._apply(fn, recurse)

    def __getstate__(self):
        # copies and pickles carry the buffers, not the launch cache (ctypes
        # structs of device addresses)
        state = super().__getstate__()
        state.pop("_calls", None)
        return state

    @staticmethod
    def from_linear(linear: nn.Linear) -> "FP8Linear":
        """Convert a loaded bf16 nn.Linear (weights on the CPU or a HIP device)."""
        mod = FP8Linear(linear.in_features, linear.out_features, bias=linear.bias is not None)
        wq, s = quantize_weight_tensorwise(linear.weight.data.float())
        mod.weight = wq.to(linear.weight.device)
        mod.weight_scale = s.to(linear.weight.device)
        if linear.bias is not None:
            mod.bias = linear.bias.data.to(torch.bfloat16).clone()
        return mod.to(linear.weight.device)


def convert_linears_fp8(module: nn.Module, skip_patterns: tuple[str, ...] = (), prefix: str = "") -> list[str]:
    """Replace every nn.Linear below `module` with FP8Linear in place (fp8.py:104-122);
    returns the converted names, skipping names that contain a skip pattern."""
    converted = []
    for name, child in list(module.named_children()):
        full = f"{prefix}.{name}" if prefix else name
        if any(p in full for p in skip_patterns):
            continue
        if isinstance(child, nn.Linear):
            setattr(module, name, FP8Linear.from_linear(child))
            converted.append(full)
        else:
            converted.extend(convert_linears_fp8(child, skip_patterns, full))
    return converted


def fp8_state_dict(model: nn.Module) -> dict[str, torch.Tensor]:
    """The state dict of a converted model: fp8 `weight` + `weight_scale` for
    converted linears, every other tensor in its own dtype (fp8.py:125-128)."""
    return dict(model.state_dict().items())
