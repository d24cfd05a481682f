"""ctypes binding of the C ABI declared in include/qik_attn.h and include/qik_ops.h.

The shared library is built in-tree (``lib/libqik_attn.so`` next to this file)
by ``build.py``.  There is no fallback: if the library is missing or fails to
load, every entry point raises.

torch is imported before the library is opened on purpose.  torch ships its own
HIP runtime (soname ``libamdhip64.so.7``); loading torch first makes the
dynamic linker bind this library to that same runtime instance, so the
``hipStream_t`` handles torch hands out are valid here.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (load order: torch's HIP runtime first)

LIB_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib")
LIB_PATH = os.path.join(LIB_DIR, "libqik_attn.so")

ABI_VERSION = 2

DTYPE_BF16 = 0
DTYPE_FP16 = 1
DTYPE_FP32 = 2  # quantiser input only (include/qik_fp8.h)

FP8_ACTIVATION = 0
FP8_WEIGHT = 1

# leading bytes of a qik_attn_fwd_ws workspace that hold its control words
WS_CTL_BYTES = 32768

HAS_CACHE = 1
HAS_KEY_VALID = 2
UNIFORM_L = 4
V_CACHE_FP8 = 8

STATUS_NAMES = {
    0: "QIK_OK",
    -1: "QIK_ERR_NULL_ARG",
    -2: "QIK_ERR_ABI_VERSION",
    -3: "QIK_ERR_DTYPE",
    -4: "QIK_ERR_HEAD_DIM",
    -5: "QIK_ERR_SHAPE",
    -6: "QIK_ERR_CACHE",
    -7: "QIK_ERR_FP8_SCALE",
    -8: "QIK_ERR_ALIGN",
    -9: "QIK_ERR_LAUNCH",
    -10: "QIK_ERR_SEGMENTS",
    -11: "QIK_ERR_DEVICE",
    -12: "QIK_ERR_WORKSPACE",
    -13: "QIK_ERR_SCRATCH",
}

# bytes of the static device array behind qik_attn_fwd_noalloc
ATTN_SCRATCH_BYTES = 72 * 1024 * 1024

_i64x3 = ctypes.c_int64 * 3


class QikAttnArgs(ctypes.Structure):
    """Mirror of ``struct qik_attn_args`` (include/qik_attn.h)."""

    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("flags", ctypes.c_int32),
        ("reserved0", ctypes.c_int32),
        ("q", ctypes.c_void_p),
        ("k_new", ctypes.c_void_p),
        ("v_new", ctypes.c_void_p),
        ("k_cache", ctypes.c_void_p),
        ("v_cache", ctypes.c_void_p),
        ("v_scale", ctypes.c_void_p),
        ("prefix_lengths", ctypes.c_void_p),
        ("key_valid", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("debug_tiles", ctypes.c_void_p),
        ("B", ctypes.c_int64),
        ("SQ", ctypes.c_int64),
        ("SN", ctypes.c_int64),
        ("P", ctypes.c_int64),
        ("H", ctypes.c_int64),
        ("D", ctypes.c_int64),
        ("stride_q", _i64x3),
        ("stride_k_new", _i64x3),
        ("stride_v_new", _i64x3),
        ("stride_k_cache", _i64x3),
        ("stride_v_cache", _i64x3),
        ("stride_out", _i64x3),
        ("stride_valid_b", ctypes.c_int64),
        ("sm_scale", ctypes.c_float),
        ("reserved1", ctypes.c_int32),
    ]


class QikRmsRopeArgs(ctypes.Structure):
    """Mirror of ``struct qik_rms_rope_args`` (include/qik_ops.h)."""

    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("x", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("weight", ctypes.c_void_p),
        ("cos", ctypes.c_void_p),
        ("sin", ctypes.c_void_p),
        ("B", ctypes.c_int64),
        ("S", ctypes.c_int64),
        ("H", ctypes.c_int64),
        ("D", ctypes.c_int64),
        ("stride_x", _i64x3),
        ("stride_out", _i64x3),
        ("eps", ctypes.c_float),
        ("reserved0", ctypes.c_int32),
    ]


class QikSlabStoreArgs(ctypes.Structure):
    """Mirror of ``struct qik_slab_store_args`` (include/qik_ops.h)."""

    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("v_fp8", ctypes.c_int32),
        ("reserved0", ctypes.c_int32),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("k_dst", ctypes.c_void_p),
        ("v_dst", ctypes.c_void_p),
        ("v_scale", ctypes.c_void_p),
        ("B", ctypes.c_int64),
        ("P", ctypes.c_int64),
        ("H", ctypes.c_int64),
        ("D", ctypes.c_int64),
        ("stride_k", _i64x3),
        ("stride_v", _i64x3),
        ("stride_k_dst", _i64x3),
        ("stride_v_dst", _i64x3),
        ("length_dst", ctypes.c_void_p),
    ]


class QikFp8QuantArgs(ctypes.Structure):
    """Mirror of ``struct qik_fp8_quant_args`` (include/qik_fp8.h)."""

    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("mode", ctypes.c_int32),
        ("reserved0", ctypes.c_int32),
        ("x", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("scale", ctypes.c_void_p),
        ("n", ctypes.c_int64),
    ]


class QikFp8GemmArgs(ctypes.Structure):
    """Mirror of ``struct qik_fp8_gemm_args`` (include/qik_fp8.h)."""

    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("out_dtype", ctypes.c_int32),
        ("reserved0", ctypes.c_int32),
        ("reserved1", ctypes.c_int32),
        ("a", ctypes.c_void_p),
        ("w", ctypes.c_void_p),
        ("scale_a", ctypes.c_void_p),
        ("scale_w", ctypes.c_void_p),
        ("bias", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("M", ctypes.c_int64),
        ("N", ctypes.c_int64),
        ("K", ctypes.c_int64),
        ("lda", ctypes.c_int64),
        ("ldw", ctypes.c_int64),
        ("ldc", ctypes.c_int64),
    ]


# (name, restype, argtypes) of every exported entry point
EXPORTS = (
    ("qik_abi_version", ctypes.c_int, ()),
    ("qik_strerror", ctypes.c_char_p, (ctypes.c_int,)),
    ("qik_attn_block_shape", ctypes.c_int, (ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int32))),
    ("qik_attn_validate", ctypes.c_int, (ctypes.POINTER(QikAttnArgs),)),
    ("qik_attn_fwd", ctypes.c_int, (ctypes.POINTER(QikAttnArgs), ctypes.c_void_p)),
    ("qik_attn_workspace_size", ctypes.c_int, (ctypes.POINTER(QikAttnArgs), ctypes.POINTER(ctypes.c_int64))),
    (
        "qik_attn_fwd_ws",
        ctypes.c_int,
        (ctypes.POINTER(QikAttnArgs), ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p),
    ),
    ("qik_attn_fwd_noalloc", ctypes.c_int, (ctypes.POINTER(QikAttnArgs), ctypes.c_void_p)),
    (
        "qik_attn_work_map",
        ctypes.c_int,
        (ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p,
         ctypes.c_void_p, ctypes.c_int64, ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int64),
         ctypes.POINTER(ctypes.c_int32)),
    ),
    (
        "qik_attn_work_map_xcds",
        ctypes.c_int,
        (ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p,
         ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.POINTER(ctypes.c_int64),
         ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int32)),
    ),
    (
        "qik_attn_tile_schedule",
        ctypes.c_int,
        (ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p),
    ),
    (
        "qik_build_prefix_lengths",
        ctypes.c_int,
        (ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p),
    ),
    ("qik_rms_rope", ctypes.c_int, (ctypes.POINTER(QikRmsRopeArgs), ctypes.c_void_p)),
    ("qik_slab_store", ctypes.c_int, (ctypes.POINTER(QikSlabStoreArgs), ctypes.c_void_p)),
    ("qik_slab_store_workspace_size", ctypes.c_int, (ctypes.POINTER(QikSlabStoreArgs), ctypes.POINTER(ctypes.c_int64))),
    ("qik_slab_store_ws", ctypes.c_int,
     (ctypes.POINTER(QikSlabStoreArgs), ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p)),
    ("qik_fp8_quant_workspace_size", ctypes.c_int,
     (ctypes.POINTER(QikFp8QuantArgs), ctypes.POINTER(ctypes.c_int64))),
    ("qik_fp8_quantize", ctypes.c_int,
     (ctypes.POINTER(QikFp8QuantArgs), ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p)),
    ("qik_fp8_gemm_validate", ctypes.c_int, (ctypes.POINTER(QikFp8GemmArgs),)),
    ("qik_fp8_gemm", ctypes.c_int, (ctypes.POINTER(QikFp8GemmArgs), ctypes.c_void_p)),
    ("qik_fp8_gemm_workspace_size", ctypes.c_int,
     (ctypes.POINTER(QikFp8GemmArgs), ctypes.POINTER(ctypes.c_int64))),
    ("qik_fp8_gemm_ws", ctypes.c_int,
     (ctypes.POINTER(QikFp8GemmArgs), ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p)),
    ("qik_fp8_gemm_plan", ctypes.c_int,
     (ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int32, ctypes.POINTER(ctypes.c_int32),
      ctypes.POINTER(ctypes.c_int64))),
    ("qik_fp8_dequant", ctypes.c_int,
     (ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p)),
    ("qik_fp8_quantize_weight_host", ctypes.c_int,
     (ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32)),
)

_lock = threading.Lock()
_lib = None


def load() -> ctypes.CDLL:
    """Open the in-tree library once; raise if it is absent or incompatible."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"qwen_image_kernel_amd: HIP library not built ({LIB_PATH} missing); "
                "run __graft_entry__.build() or python -m qwen_image_kernel_amd.build"
            )
        lib = ctypes.CDLL(LIB_PATH)
        for name, restype, argtypes in EXPORTS:
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = list(argtypes)
        ver = lib.qik_abi_version()
        if ver != ABI_VERSION:
            raise RuntimeError(f"qwen_image_kernel_amd: library ABI {ver} != binding ABI {ABI_VERSION}")
        _lib = lib
    return _lib


def strerror(status: int) -> str:
    msg = load().qik_strerror(int(status))
    return msg.decode() if msg else "unknown"


def check(status: int, what: str) -> None:
    """Raise RuntimeError for a nonzero status (the reference raises on launch errors)."""
    if status != 0:
        name = STATUS_NAMES.get(int(status), str(status))
        raise RuntimeError(f"{what} failed: {name}: {strerror(status)}")
