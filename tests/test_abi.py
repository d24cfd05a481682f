"""C ABI: exports, struct layout, host-side validation and the schedule mirror (CPU only).

No test here launches a kernel: qik_attn_validate and qik_attn_tile_schedule
are host-only, and qik_attn_fwd is only called with arguments it rejects (or
with no work) before any device call.
"""

import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

from oracle import schedule as osch

import qwen_image_kernel_amd.workloads as wls
from qwen_image_kernel_amd import _lib, attention

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "qik_attn.h")
HEADERS = [HEADER, os.path.join(ROOT, "include", "qik_ops.h"), os.path.join(ROOT, "include", "qik_fp8.h")]


def header_functions():
    names = set()
    for h in HEADERS:
        names |= set(re.findall(r"^[A-Za-z_][\w\s\*]*?\b(qik_\w+)\s*\(", open(h).read(), flags=re.M))
    return sorted(names)


def test_header_constants_match_the_binding():
    text = open(HEADER).read()
    assert re.search(r"#define QIK_ABI_VERSION (\d+)", text).group(1) == str(_lib.ABI_VERSION)
    assert re.search(r"#define QIK_ATTN_WS_CTL_BYTES (\d+)", text).group(1) == str(_lib.WS_CTL_BYTES)


def test_library_loads_and_exports_every_declared_symbol():
    lib = _lib.load()
    names = header_functions()
    assert len(names) >= 7
    for n in names:
        assert hasattr(lib, n), n
    assert {n for n, _, _ in _lib.EXPORTS} == set(names)
    assert lib.qik_abi_version() == _lib.ABI_VERSION


@pytest.mark.parametrize("cname,pytype", [("qik_attn_args", _lib.QikAttnArgs),
                                           ("qik_rms_rope_args", _lib.QikRmsRopeArgs),
                                           ("qik_slab_store_args", _lib.QikSlabStoreArgs),
                                           ("qik_fp8_quant_args", _lib.QikFp8QuantArgs),
                                           ("qik_fp8_gemm_args", _lib.QikFp8GemmArgs)])
def test_struct_layout_matches_c_header(tmp_path, cname, pytype):
    fields = [f for f, _ in pytype._fields_]
    src = ["#include <stdio.h>", "#include <stddef.h>", '#include "qik_ops.h"', '#include "qik_fp8.h"',
           "int main(void) {",
           f'printf("sizeof %zu\\n", sizeof({cname}));']
    for f in fields:
        src.append(f'printf("{f} %zu\\n", offsetof({cname}, {f}));')
    src.append("return 0; }")
    c = tmp_path / "layout.c"
    c.write_text("\n".join(src))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", f"-I{os.path.dirname(HEADER)}", str(c), "-o", str(exe)], check=True)
    got = dict(line.split() for line in subprocess.run([str(exe)], capture_output=True, text=True,
                                                        check=True).stdout.splitlines())
    assert int(got["sizeof"]) == ctypes.sizeof(pytype)
    for f in fields:
        assert int(got[f]) == getattr(pytype, f).offset, f


def _valid_args(**kw):
    a = _lib.QikAttnArgs()
    a.abi_version = _lib.ABI_VERSION
    a.dtype = _lib.DTYPE_BF16
    a.flags = 0
    B, SQ, SN, H, D = 1, 300, 300, 4, 128
    a.B, a.SQ, a.SN, a.P, a.H, a.D = B, SQ, SN, 0, H, D
    fake = 0x10000
    a.q, a.k_new, a.v_new, a.out, a.prefix_lengths = fake, fake, fake, fake, fake
    st = (SQ * H * D, H * D, D)
    for f in ("stride_q", "stride_k_new", "stride_v_new", "stride_out"):
        setattr(a, f, _lib._i64x3(*st))
    a.sm_scale = D ** -0.5
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def _validate(a):
    return _lib.load().qik_attn_validate(ctypes.byref(a))


def test_validate_accepts_reference_call_patterns():
    assert _validate(_valid_args()) == 0
    # decode: slab views [B, P, H, D] with strides (H*Pmax*D, D, Pmax*D) and fp8 V
    a = _valid_args(P=256, flags=_lib.HAS_CACHE | _lib.V_CACHE_FP8 | _lib.UNIFORM_L)
    a.k_cache = a.v_cache = a.v_scale = 0x20000
    a.stride_k_cache = a.stride_v_cache = _lib._i64x3(4 * 528 * 128, 128, 528 * 128)
    a.prefix_lengths = None
    assert _validate(a) == 0
    # fresh V as a strided view of a fused QKV output: stride_s = 3*H*D
    a = _valid_args()
    a.stride_v_new = _lib._i64x3(300 * 3 * 4 * 128, 3 * 4 * 128, 128)
    assert _validate(a) == 0


@pytest.mark.parametrize(
    "mutate,code",
    [
        (lambda a: setattr(a, "abi_version", 99), -2),
        (lambda a: setattr(a, "reserved0", 1), -2),
        (lambda a: setattr(a, "dtype", 7), -3),              # triton_attention.py:190
        (lambda a: setattr(a, "D", 96), -4),
        (lambda a: setattr(a, "D", 16), -4),
        (lambda a: setattr(a, "D", 512), -4),
        (lambda a: setattr(a, "SQ", -1), -5),
        (lambda a: setattr(a, "flags", 64), -5),
        (lambda a: setattr(a, "P", 16), -6),                 # P > 0 without HAS_CACHE (:192-196)
        (lambda a: setattr(a, "flags", _lib.HAS_CACHE), -6),  # HAS_CACHE with P == 0
        (lambda a: setattr(a, "flags", _lib.V_CACHE_FP8), -7),  # fp8 V without a cache (:213-216)
        (lambda a: setattr(a, "v_scale", 0x30000), -7),      # a scale without fp8 V
        (lambda a: setattr(a, "flags", _lib.HAS_KEY_VALID), -1),
        (lambda a: setattr(a, "q", None), -1),
        (lambda a: setattr(a, "prefix_lengths", None), -1),
        (lambda a: setattr(a, "q", 0x10008), -8),
        (lambda a: setattr(a, "stride_k_new", _lib._i64x3(300 * 512, 516, 128)), -8),
    ],
)
def test_validate_error_codes(mutate, code):
    a = _valid_args()
    mutate(a)
    assert _validate(a) == code
    # the launches and the workspace query validate first and return the same
    # code without a device call
    lib = _lib.load()
    assert lib.qik_attn_fwd(ctypes.byref(a), None) == code
    assert lib.qik_attn_fwd_ws(ctypes.byref(a), None, 0, None) == code
    nbytes = ctypes.c_int64(-1)
    assert lib.qik_attn_workspace_size(ctypes.byref(a), ctypes.byref(nbytes)) == code
    assert nbytes.value == 0
    assert _lib.STATUS_NAMES[code] and _lib.strerror(code) != "unknown qik status"


def test_fp8_requires_bf16():
    a = _valid_args(P=64, dtype=_lib.DTYPE_FP16, flags=_lib.HAS_CACHE | _lib.V_CACHE_FP8)
    a.k_cache = a.v_cache = a.v_scale = 0x20000
    a.stride_k_cache = a.stride_v_cache = _lib._i64x3(4 * 64 * 128, 128, 64 * 128)
    assert _validate(a) == -7


def test_fwd_without_work_is_a_no_op():
    a = _valid_args(SQ=0)
    lib = _lib.load()
    assert lib.qik_attn_fwd(ctypes.byref(a), None) == 0
    nbytes = ctypes.c_int64(-1)
    assert lib.qik_attn_workspace_size(ctypes.byref(a), ctypes.byref(nbytes)) == 0
    assert nbytes.value == 0
    assert lib.qik_attn_fwd_ws(ctypes.byref(a), None, 0, None) == 0
    assert lib.qik_attn_workspace_size(ctypes.byref(a), None) == -1


def test_segment_validation_is_host_side():
    lib = _lib.load()
    bad = np.array([[5, 3, 0]], dtype=np.int32)
    assert lib.qik_build_prefix_lengths(bad.ctypes.data, 1, 0, 10, None, None) == -10
    neg = np.array([[-1, 3, 0]], dtype=np.int32)
    assert lib.qik_build_prefix_lengths(neg.ctypes.data, 1, 0, 10, None, None) == -10
    ok = np.array([[0, 3, 0]], dtype=np.int32)
    assert lib.qik_build_prefix_lengths(ok.ctypes.data, 1, 11, 10, None, None) == -10   # prefix_end > seq_len
    assert lib.qik_build_prefix_lengths(ok.ctypes.data, 1, 0, 0, None, None) == 0       # nothing to fill


@pytest.mark.parametrize("name", wls.NAMES)
def test_schedule_mirror_equals_oracle_exact_rule(name):
    wl = wls.workload(name)
    bm, bn = attention.block_shape()
    got = attention.tile_schedule(wl.SQ, wl.P, wl.SN, wl.lengths(), wl.uniform)
    want = osch.exact_rule(wl.lengths(), wl.SQ, wl.P, wl.SN, bm, bn, wl.P > 0, wl.uniform)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("seed", range(30))
def test_schedule_mirror_random(seed):
    rng = np.random.default_rng(seed)
    SQ = int(rng.integers(1, 700))
    P = int(rng.integers(0, 2)) * int(rng.integers(1, 500))
    SN = int(rng.integers(1, 700))
    L = rng.integers(-1, P + SN + 3, size=SQ).astype(np.int32)
    bm, bn = attention.block_shape()
    for uniform in (False, True):
        got = attention.tile_schedule(SQ, P, SN, L, uniform)
        want = osch.exact_rule(L, SQ, P, SN, bm, bn, P > 0, uniform)
        np.testing.assert_array_equal(got, want)


def test_wrapper_keeps_reference_asserts_on_cpu():
    import torch
    q = torch.zeros(1, 8, 2, 128)
    with pytest.raises(AssertionError, match="fp16/bf16 only"):
        attention.block_causal_flash_attention(q, q, q, torch.zeros(8, dtype=torch.int32), None)
    qb = q.to(torch.bfloat16)
    ck = torch.zeros(1, 4, 3, 128, dtype=torch.bfloat16)
    with pytest.raises(AssertionError):
        attention.block_causal_flash_attention(qb, qb, qb, torch.zeros(8, dtype=torch.int32), None,
                                               cache_k=ck, cache_v=ck)


def _rope_args(**kw):
    a = _lib.QikRmsRopeArgs()
    a.abi_version = _lib.ABI_VERSION
    a.dtype = _lib.DTYPE_BF16
    a.B, a.S, a.H, a.D = 1, 16, 2, 128
    a.x = a.out = a.weight = a.cos = a.sin = 0x10000
    a.stride_x = a.stride_out = _lib._i64x3(16 * 2 * 128, 2 * 128, 128)
    a.eps = 1e-6
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("kw,code", [
    (dict(abi_version=3), -2), (dict(reserved0=1), -2), (dict(dtype=5), -3), (dict(D=96), -4),
    (dict(S=-2), -5), (dict(x=None), -1), (dict(cos=None), -1), (dict(out=0x10004), -8),
    (dict(stride_x=_lib._i64x3(4096, 260, 128)), -8),
])
def test_rms_rope_rejects_before_any_device_call(kw, code):
    assert _lib.load().qik_rms_rope(ctypes.byref(_rope_args(**kw)), None) == code


def test_rms_rope_without_rows_is_a_no_op():
    assert _lib.load().qik_rms_rope(ctypes.byref(_rope_args(S=0, x=None)), None) == 0


def _store_args(**kw):
    a = _lib.QikSlabStoreArgs()
    a.abi_version = _lib.ABI_VERSION
    a.dtype = _lib.DTYPE_BF16
    a.v_fp8 = 1
    a.k = a.v = a.k_dst = a.v_dst = a.v_scale = 0x10000
    a.B, a.P, a.H, a.D = 1, 32, 2, 128
    a.stride_k = a.stride_v = _lib._i64x3(32 * 2 * 128, 2 * 128, 128)
    a.stride_k_dst = a.stride_v_dst = _lib._i64x3(2 * 48 * 128, 48 * 128, 128)
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("kw,code", [
    (dict(abi_version=0), -2), (dict(dtype=9), -3), (dict(D=96), -4), (dict(P=-1), -5),
    (dict(v_scale=None), -7),                     # fp8 V needs the scale output
    (dict(v_fp8=0), -7),                          # a scale output without fp8 V
    (dict(k=None), -1), (dict(v_dst=0x10004), -8), (dict(stride_k=_lib._i64x3(8192, 260, 128)), -8),
    (dict(length_dst=0x10004), -8),               # the length is an int64
])
def test_slab_store_rejects_before_any_device_call(kw, code):
    assert _lib.load().qik_slab_store(ctypes.byref(_store_args(**kw)), None) == code


def test_slab_store_without_rows_is_a_no_op():
    assert _lib.load().qik_slab_store(ctypes.byref(_store_args(P=0, k=None)), None) == 0


@pytest.mark.parametrize("kw,code", [
    (dict(abi_version=0), -2), (dict(dtype=9), -3), (dict(D=96), -4), (dict(P=-1), -5),
    (dict(v_scale=None), -7), (dict(v_fp8=0), -7),
    (dict(k=None), -1), (dict(v_dst=0x10004), -8),
])
def test_slab_store_ws_rejects_like_the_three_launch_store(kw, code):
    lib = _lib.load()
    ws = (ctypes.c_float * (2 * 64))()
    assert lib.qik_slab_store_ws(ctypes.byref(_store_args(**kw)), ctypes.addressof(ws), 2 * 64 * 4, None) == code


def test_slab_store_workspace_checks_and_size():
    """fp8 V: B*H*64 fp32 partial scales, 4-byte aligned; no workspace needed otherwise."""
    lib = _lib.load()
    n = ctypes.c_int64(-1)
    assert lib.qik_slab_store_workspace_size(ctypes.byref(_store_args()), ctypes.byref(n)) == 0
    assert n.value == 1 * 2 * 64 * 4
    assert lib.qik_slab_store_workspace_size(ctypes.byref(_store_args(v_fp8=0, v_scale=None)), ctypes.byref(n)) == 0
    assert n.value == 0
    assert lib.qik_slab_store_workspace_size(ctypes.byref(_store_args()), None) == -1
    buf = (ctypes.c_float * 256)()
    base = ctypes.addressof(buf)
    WS = -12
    assert lib.qik_slab_store_ws(ctypes.byref(_store_args()), None, 512, None) == WS
    assert lib.qik_slab_store_ws(ctypes.byref(_store_args()), base, 511, None) == WS
    assert lib.qik_slab_store_ws(ctypes.byref(_store_args()), base + 2, 512, None) == WS
    # no rows: nothing to do, no workspace looked at
    assert lib.qik_slab_store_ws(ctypes.byref(_store_args(P=0, k=None)), None, 0, None) == 0


def test_side_input_device_check_is_host_side():
    """A side input that is not on the query's device raises ValueError before any launch."""
    import torch

    cpu = torch.zeros(4, dtype=torch.int32)
    with pytest.raises(ValueError, match="prefix_lengths"):
        attention._check_aux("prefix_lengths", cpu, torch.device("cuda", 0))
    with pytest.raises(ValueError, match="key_valid"):
        attention._check_aux("key_valid", cpu.bool(), torch.device("cuda", 0))
    with pytest.raises(ValueError, match="cache_v_scale"):
        attention._check_aux("cache_v_scale", None, torch.device("cuda", 0))
    attention._check_aux("prefix_lengths", cpu, torch.device("cpu"))


def test_scratch_constant_matches_the_binding():
    text = open(HEADER).read()
    m = re.search(r"#define QIK_ATTN_SCRATCH_BYTES \((\d+) \* 1024 \* 1024\)", text)
    assert int(m.group(1)) * 1024 * 1024 == _lib.ATTN_SCRATCH_BYTES


def test_fp8_header_constants_match_the_binding():
    text = open(os.path.join(ROOT, "include", "qik_fp8.h")).read()
    assert re.search(r"#define QIK_DTYPE_FP32 (\d+)", text).group(1) == str(_lib.DTYPE_FP32)
    assert re.search(r"QIK_FP8_ACTIVATION = (\d+)", text).group(1) == str(_lib.FP8_ACTIVATION)
    assert re.search(r"QIK_FP8_WEIGHT = (\d+)", text).group(1) == str(_lib.FP8_WEIGHT)


def _gemm_args(**kw):
    a = _lib.QikFp8GemmArgs()
    a.abi_version = _lib.ABI_VERSION
    a.out_dtype = _lib.DTYPE_BF16
    a.a, a.w, a.scale_a, a.scale_w, a.out = 0x10000, 0x20000, 0x30000, 0x30004, 0x40000
    a.M, a.N, a.K = 1536, 4096, 4096
    a.lda, a.ldw, a.ldc = 4096, 4096, 4096
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize(
    "kw,code",
    [
        ({}, 0),
        ({"bias": 0x50008}, 0),
        ({"M": 1, "N": 16, "K": 16, "lda": 16, "ldw": 16, "ldc": 16}, 0),
        ({"out_dtype": _lib.DTYPE_FP16}, 0),
        ({"abi_version": 9}, -2),
        ({"reserved1": 1}, -2),
        ({"out_dtype": _lib.DTYPE_FP32}, -3),   # fp32 out is not an output type here
        ({"M": 0}, -5),
        ({"N": 4100, "ldc": 4100}, -5),        # N % 16 (the _scaled_mm contract)
        ({"K": 4104}, -5),                     # K % 16
        ({"lda": 4080}, -5),                   # row stride < K
        ({"ldc": 4000}, -5),
        ({"lda": 1 << 24, "ldw": 4096}, -5),   # a tile's rows exceed a 31-bit offset
        ({"w": None}, -1),
        ({"scale_a": None}, -1),
        ({"a": 0x10008}, -8),
        ({"lda": 4104}, -8),
        ({"bias": 0x50004}, -8),
    ],
)
def test_fp8_gemm_validate(kw, code):
    assert _lib.load().qik_fp8_gemm_validate(ctypes.byref(_gemm_args(**kw))) == code


def test_fp8_gemm_workspace_size_and_checks():
    """The workspace variant splits K only for few tiles and a long K: the
    reference test's shape needs none; the text stream's MLP out (256 tokens,
    K = 12288) takes 5 slices of 48 tiles of 128 x 128 (on 256 CUs, the count
    the host assumes when it cannot ask a device) in fp32."""
    lib = _lib.load()
    n = ctypes.c_int64(-1)
    assert lib.qik_fp8_gemm_workspace_size(ctypes.byref(_gemm_args()), ctypes.byref(n)) == 0
    assert n.value == 0
    skinny = dict(M=256, N=3072, K=12288, lda=12288, ldw=12288, ldc=3072)
    assert lib.qik_fp8_gemm_workspace_size(ctypes.byref(_gemm_args(**skinny)), ctypes.byref(n)) == 0
    assert n.value == 5 * 256 * 3072 * 4
    assert lib.qik_fp8_gemm_workspace_size(ctypes.byref(_gemm_args(M=0)), ctypes.byref(n)) == -5
    assert lib.qik_fp8_gemm_workspace_size(ctypes.byref(_gemm_args()), None) == -1
    buf = (ctypes.c_uint8 * 64)()
    base = (ctypes.addressof(buf) + 15) // 16 * 16
    WS = -12
    a = _gemm_args(**skinny)
    assert lib.qik_fp8_gemm_ws(ctypes.byref(a), None, n.value, None) == WS
    assert lib.qik_fp8_gemm_ws(ctypes.byref(a), base, 32, None) == WS
    assert lib.qik_fp8_gemm_ws(ctypes.byref(a), base + 8, n.value, None) == WS
    assert lib.qik_fp8_gemm_ws(ctypes.byref(_gemm_args(M=0)), base, n.value, None) == -5


@pytest.mark.parametrize("mnk,plan,n1", [
    ((1536, 4096, 4096), [192, 128, 128, 128, 0, 1], 4096),    # 256 tiles of 192 x 128, one per CU
    ((4352, 9216, 3072), [256, 256, 256, 128, 1, 1], 7680),    # fused QKV: 256 x 128 columns launched first
    ((4352, 12288, 3072), [256, 256, 256, 128, 1, 1], 11520),  # MLP in: the same
    ((4352, 3072, 12288), [256, 256, 256, 128, 0, 1], 3072),   # MLP out: 204 tiles of 256 x 256
    ((256, 9216, 3072), [256, 128, 128, 128, 0, 1], 0),        # text QKV: 144 tiles of 128 x 128
    ((256, 3072, 12288), [128, 128, 128, 128, 0, 5], 3072),    # text MLP out: K split in 5
    ((1543, 9232, 1104), [256, 256, 256, 128, 0, 1], 8192),    # small tiles first would finish later
    ((100, 1040, 8192), [128, 128, 128, 128, 0, 8], 1040),     # K split in 8
])
def test_fp8_gemm_plan(mnk, plan, n1):
    """The host mirror of the GEMM launch (256 CUs, the count the host assumes
    without a device): tile shapes, the columns of the big tiles, which region
    goes first, the K split."""
    lib = _lib.load()
    got = (ctypes.c_int32 * 6)()
    n = ctypes.c_int64()
    assert lib.qik_fp8_gemm_plan(*mnk, 0, got, ctypes.byref(n)) == 0
    assert list(got) == plan and n.value == n1


def test_fp8_gemm_plan_checks():
    lib = _lib.load()
    got = (ctypes.c_int32 * 6)()
    n = ctypes.c_int64()
    assert lib.qik_fp8_gemm_plan(0, 16, 16, 0, got, ctypes.byref(n)) == -5
    assert lib.qik_fp8_gemm_plan(16, 24, 16, 0, got, ctypes.byref(n)) == -5
    assert lib.qik_fp8_gemm_plan(16, 16, 16, 0, None, None) == -1


def _quant_args(**kw):
    a = _lib.QikFp8QuantArgs()
    a.abi_version = _lib.ABI_VERSION
    a.dtype = _lib.DTYPE_BF16
    a.mode = _lib.FP8_ACTIVATION
    a.x, a.out, a.scale = 0x10000, 0x20000, 0x30000
    a.n = 1536 * 4096
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def test_fp8_quant_workspace_size_and_checks():
    lib = _lib.load()
    n = ctypes.c_int64(-1)
    # one size for every n: 64 control words, 1024 64-bit one-pass slots, 1024 two-pass partial maxima
    for nn in (1536 * 4096, 3, 1 << 36):
        assert lib.qik_fp8_quant_workspace_size(ctypes.byref(_quant_args(n=nn)), ctypes.byref(n)) == 0
        assert n.value == 4 * (64 + 2 * 1024 + 1024)
    for kw, code in [({"n": 0}, -5), ({"dtype": 5}, -3), ({"mode": 2}, -3), ({"x": None}, -1),
                     ({"x": 0x10008}, -8), ({"out": 0x20004}, -8), ({"dtype": _lib.DTYPE_FP32, "out": 0x20004}, 0),
                     ({"reserved0": 1}, -2)]:
        assert lib.qik_fp8_quant_workspace_size(ctypes.byref(_quant_args(**kw)), ctypes.byref(n)) == code, kw
    buf = (ctypes.c_uint32 * 4096)()
    base = ctypes.addressof(buf)
    WS = -12
    assert lib.qik_fp8_quantize(ctypes.byref(_quant_args()), None, 16384, None) == WS
    assert lib.qik_fp8_quantize(ctypes.byref(_quant_args()), base, 12540, None) == WS
    assert lib.qik_fp8_quantize(ctypes.byref(_quant_args()), base + 2, 16384, None) == WS


def test_fp8_dequant_rejects_before_any_launch():
    lib = _lib.load()
    assert lib.qik_fp8_dequant(0x10000, 0x20000, 0x30000, 64, 3, None) == -3       # fp32 is an output type now
    assert lib.qik_fp8_dequant(0x10000, 0x20000, 0x30000, -1, _lib.DTYPE_BF16, None) == -5
    assert lib.qik_fp8_dequant(0x10000, 0x20000, 0x30000, 0, _lib.DTYPE_BF16, None) == 0   # no work
    assert lib.qik_fp8_dequant(None, 0x20000, 0x30000, 64, _lib.DTYPE_BF16, None) == -1
    assert lib.qik_fp8_dequant(0x10004, 0x20000, 0x30000, 64, _lib.DTYPE_BF16, None) == -8
    assert lib.qik_fp8_dequant(0x10000, 0x20000, 0x30008, 64, _lib.DTYPE_BF16, None) == -8


def test_slab_store_fp8_takes_fp16_and_cache_rejects_other_dtypes():
    """An fp8 slab store validates for an fp16 source as for bf16 (the
    reference quantises any dtype, kv_cache.py:36-42); a device cache refuses
    element types its kernels cannot read (4-byte fp32, 1-byte) up front,
    before it allocates anything."""
    import torch
    import qwen_image_kernel_amd as qik
    lib = _lib.load()
    for dt in (_lib.DTYPE_BF16, _lib.DTYPE_FP16):
        n = ctypes.c_int64(-1)
        assert lib.qik_slab_store_workspace_size(ctypes.byref(_store_args(dtype=dt)), ctypes.byref(n)) == 0
        assert n.value == 2 * 64 * 4                  # B*H heads x 64 chunk scales
    for dt in (torch.float32, torch.float8_e4m3fn, torch.int16):
        with pytest.raises(ValueError, match="bfloat16 or float16"):
            qik.ContiguousKVCache(1, 1, 16, 2, 128, device="cuda", dtype=dt)


@pytest.mark.parametrize("v_fp8", [False, True])
def test_cpu_slab_takes_any_float_dtype_like_the_reference(v_fp8):
    """A CPU slab is stored by the reference's torch ops (kv_cache.py:30-45),
    so an fp32 CPU cache works as the reference's does: K copied, V copied or
    quantised per (b, h) with scale max(amax/448, 1e-12)."""
    import torch
    import qwen_image_kernel_amd as qik
    g = torch.Generator().manual_seed(5)
    B, P, H, D = 2, 24, 3, 64
    k = torch.randn(B, P, H, D, generator=g)
    v = torch.randn(B, P, H, D, generator=g) * 3
    cache = qik.ContiguousKVCache(2, B, P + 8, H, D, v_fp8=v_fp8, device="cpu", dtype=torch.float32)
    cache.get_layer(1).store(k, v)
    kk, vv = cache.get_layer(1).get()
    assert kk.dtype == torch.float32 and torch.equal(kk, k)
    assert int(cache.lengths[1]) == P
    if v_fp8:
        vt = v.transpose(1, 2)
        scale = (vt.abs().amax(dim=(2, 3)) / 448.0).clamp_min(1e-12)
        codes = (vt / scale[:, :, None, None]).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
        assert torch.equal(cache.v_scale[1], scale)
        assert torch.equal(vv.transpose(1, 2).view(torch.uint8), codes.view(torch.uint8))
    else:
        assert torch.equal(vv, v)


def test_kernel_layout_rule():
    """The wrappers' layout rule on host tensors: a fused-QKV slice (strides
    multiples of 8, 16-byte base) is passed through in place; an offset base, a
    row stride off a multiple of 8 and overlapping rows get a contiguous copy
    with a 16-byte aligned base and the same values."""
    import torch
    qkv = torch.randn(2, 40, 3 * 4 * 128).to(torch.bfloat16)
    q = qkv.unflatten(-1, (12, 128))[:, :, :4]
    assert attention._kernel_layout(q) is q
    buf = torch.randn(2 * 40 * 4 * 128 + 3).to(torch.bfloat16)
    odd_base = buf[3:].view(2, 40, 4, 128)
    odd_row = torch.randn(2, 40, 4, 132).to(torch.bfloat16)[..., :128]
    overlap = torch.randn(2, 1, 4, 128).to(torch.bfloat16).expand(2, 40, 4, 128)
    for t in (odd_base, odd_row, overlap):
        c = attention._kernel_layout(t)
        assert c is not t and c.is_contiguous() and c.data_ptr() % 16 == 0
        assert torch.equal(c, t)
    fp8 = torch.zeros(1, 16, 2, 128, dtype=torch.float8_e4m3fn)
    assert attention._kernel_layout(fp8, 8) is fp8
