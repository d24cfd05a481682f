"""W8A8 fp8 linear on the GPU: quantiser, GEMM, dequantiser and FP8Linear.

The quantiser must match torch's ops on the same device bit for bit (the
reference computes the scale with torch ops and casts with one correctly
rounded reciprocal, fp8.py:24-60), and the oracle's CPU restatement.  The GEMM
is checked against the fp64 value of the dequantised product (oracle.fp8.scaled_mm,
or an fp32 torch matmul of the dequantised operands at large sizes) to within
one bf16 rounding plus the fp32 accumulation error, and against the unquantised
fp32 product at the reference test's relative-error bar (tests/test_fp8.py:16-30).
"""

import numpy as np
import pytest
import torch

from oracle import fp8 as of

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)


@pytest.fixture(scope="module")
def qik():
    if not torch.cuda.is_available():
        pytest.skip("needs a HIP device")
    import qwen_image_kernel_amd as m
    return m


def torch_act_quant(x):
    """The reference's activation quantisation with torch ops on the device
    (fp8.py:24-26 for the scale; fp8.py:37-40 for the cast: one reciprocal)."""
    s = (x.abs().amax().float() / 448.0).clamp_min(1e-12)
    return (x.float() * (1.0 / s)).to(torch.float8_e4m3fn), s.reshape(1)


def torch_weight_quant(w):
    """fp8.py:56-60 verbatim in torch ops on the device."""
    s = (w.abs().amax().float() / 448.0).clamp_min(1e-12)
    return (w.float() / s).clamp(-448.0, 448.0).to(torch.float8_e4m3fn), s.reshape(1)


def codes(t):
    return t.view(torch.uint8).cpu().numpy()


def _inputs(shape, dtype, seed, kind="normal"):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g)
    if kind == "outlier":
        x.view(-1)[len(x.view(-1)) // 3] = 3e4
    elif kind == "tiny":
        x = x * 1e-20
    elif kind == "zero":
        x = torch.zeros(*shape)
    elif kind == "wide":
        x = x * torch.exp2(torch.randint(-20, 20, shape, generator=g).float())
    return x.to(dtype).to(DEV)


@pytest.mark.parametrize("shape,dtype,kind", [
    ((1536, 4096), torch.bfloat16, "normal"),
    ((4352, 3072), torch.bfloat16, "wide"),
    ((1, 1), torch.bfloat16, "normal"),
    ((7,), torch.bfloat16, "normal"),
    ((1000003,), torch.bfloat16, "outlier"),
    ((333, 257), torch.float16, "normal"),
    ((4096, 64), torch.float32, "wide"),
    ((129, 31), torch.float32, "normal"),
    ((64, 256), torch.bfloat16, "tiny"),
    ((64, 256), torch.bfloat16, "zero"),
])
@pytest.mark.parametrize("which", ["activation", "weight"])
def test_quantiser_bit_exact_vs_torch_ops(qik, shape, dtype, kind, which):
    x = _inputs(shape, dtype, 11 + len(shape) + shape[0], kind)
    if which == "activation":
        got_q, got_s = qik.quantize_tensorwise(x)
        want_q, want_s = torch_act_quant(x)
    else:
        got_q, got_s = qik.quantize_weight_tensorwise(x)
        want_q, want_s = torch_weight_quant(x)
    assert got_q.shape == x.shape and got_q.dtype == torch.float8_e4m3fn
    assert got_s.shape == (1,) and got_s.dtype == torch.float32
    np.testing.assert_array_equal(got_s.cpu().numpy(), want_s.cpu().numpy())
    np.testing.assert_array_equal(codes(got_q), codes(want_q))
    if x.numel() <= 1 << 20:
        oq, osc = (of.quantize_tensorwise if which == "activation" else of.quantize_weight_tensorwise)(
            x.float().cpu().numpy())
        assert np.float32(got_s.item()) == osc
        np.testing.assert_array_equal(codes(got_q), oq)


def test_quantiser_one_pass_and_two_pass_forms_in_turn(qik):
    """Inputs that fit the registers of the resident workgroups take the
    one-pass launch (maxima exchanged through the workspace); larger ones the
    two-pass form.  Alternating them on one stream's workspace checks that
    every call leaves the workspace ready for the next; each call is
    bit-identical to torch's ops.  The two-pass case (72M bf16 elements) is
    past the one-pass capacity of an MI355X (512 workgroups x 256 threads x 52
    vectors of 8)."""
    print("case quantiser one-pass / two-pass alternation", flush=True)
    shapes = [((4352, 3072), torch.bfloat16), ((9000, 8000), torch.bfloat16), ((4352, 12288), torch.bfloat16),
              ((333, 257), torch.float32), ((9000, 8000), torch.bfloat16), ((1, 1), torch.bfloat16),
              ((4352, 3072), torch.bfloat16)]
    for i, (shape, dt) in enumerate(shapes):
        x = _inputs(shape, dt, 70 + i, "wide" if i % 2 else "normal")
        got_q, got_s = qik.quantize_tensorwise(x)
        want_q, want_s = torch_act_quant(x)
        assert torch.equal(got_s, want_s), (shape, got_s, want_s)
        assert torch.equal(got_q.view(torch.uint8), want_q.view(torch.uint8)), shape
        del x, got_q, want_q


@pytest.mark.parametrize("amax", [1.0, 448.0, 3.0, 2.0 ** -20, 2.0 ** 20, 1e-30, 1e30, 1e-13, 5e-10, 7.0, 0.1,
                                  1000.0])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_weight_quantiser_every_value_below_amax(qik, amax, dtype):
    """The weight quantiser divides through the scale's reciprocal and one fma
    correction; against torch's IEEE division (fp8.py:56-60 on the device):
    every finite value of the dtype with |w| <= amax, amax planted."""
    bits = torch.arange(1 << 16, dtype=torch.int32).to(torch.int16)
    vals = bits.view(dtype).float()
    am = torch.tensor(amax).to(dtype).float().item()
    if not np.isfinite(am) or am == 0.0:
        pytest.skip(f"{amax} is not a finite nonzero {dtype}")
    sel = vals[torch.isfinite(vals) & (vals.abs() <= am)]
    w = torch.cat([sel, torch.tensor([am])]).to(dtype).to(DEV)
    got_q, got_s = qik.quantize_weight_tensorwise(w)
    want_q, want_s = torch_weight_quant(w)
    np.testing.assert_array_equal(got_s.cpu().numpy(), want_s.cpu().numpy())
    np.testing.assert_array_equal(codes(got_q), codes(want_q))


def test_quantiser_strided_and_misaligned_input(qik):
    base = _inputs((1537, 4096), torch.bfloat16, 5)
    x = base[1:]               # storage offset of one row: still 16-byte aligned
    y = base[:, 1:4001]        # strided rows: copied first
    z = base.view(-1)[3:1003]  # 6-byte offset: copied to an aligned buffer first
    for t in (x, y, z):
        got_q, got_s = qik.quantize_tensorwise(t)
        want_q, want_s = torch_act_quant(t)
        assert got_s.item() == want_s.item()
        np.testing.assert_array_equal(codes(got_q), codes(want_q))


def test_quantiser_nan_poisons_the_scale(qik):
    x = _inputs((64, 256), torch.bfloat16, 3)
    x[5, 7] = float("nan")
    q, s = qik.quantize_tensorwise(x)
    assert torch.isnan(s).all()
    assert torch.isnan(q.float()).all()


def test_dequant_bit_exact(qik):
    g = torch.Generator().manual_seed(2)
    raw = torch.randint(0, 256, (1000, 64), generator=g, dtype=torch.uint8)
    raw[raw == 0x7F] = 0x7E
    raw[raw == 0xFF] = 0xFE
    w = raw.view(torch.float8_e4m3fn).to(DEV)
    s = torch.tensor([0.0123], device=DEV)
    from qwen_image_kernel_amd.fp8 import _dequant_weight
    for dt in (torch.bfloat16, torch.float16):
        got = _dequant_weight(w, s, dt)
        want = (w.to(torch.bfloat16).float() * s).to(dt)   # fp8.py:81 (then .to(x.dtype))
        np.testing.assert_array_equal(got.view(torch.int16).cpu().numpy(), want.view(torch.int16).cpu().numpy())
    odd = w.reshape(-1)[:1003]
    got = _dequant_weight(odd, s, torch.bfloat16)
    want = (odd.to(torch.bfloat16).float() * s).to(torch.bfloat16)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    # fp32 (and wider) activations take the exact fp32 product (fp8.py:81-82)
    for n in (64000, 1003):
        ww = w.reshape(-1)[:n]
        got = _dequant_weight(ww, s, torch.float32)
        want = ww.to(torch.bfloat16).float() * s
        assert got.dtype == torch.float32 and torch.equal(got.view(torch.int32), want.view(torch.int32))
    assert _dequant_weight(w, s, torch.float64).dtype == torch.float32


def _gemm_operands(M, N, K, seed, lda=None):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g)
    w = torch.randn(N, K, generator=g) * 0.02
    xq, sx = of.quantize_tensorwise(x.numpy())
    wq, sw = of.quantize_weight_tensorwise(w.numpy())
    a = torch.from_numpy(xq).view(torch.float8_e4m3fn)
    if lda is not None:
        buf = torch.zeros(M, lda, dtype=torch.uint8)
        buf[:, :K] = torch.from_numpy(xq)
        a = buf.view(torch.float8_e4m3fn).to(DEV)[:, :K]
    else:
        a = a.to(DEV)
    return a, torch.from_numpy(wq).view(torch.float8_e4m3fn).to(DEV), xq, wq, np.float32(sx), np.float32(sw)


def _half_ulp(v, dtype):
    """half the spacing of `dtype` (bf16 / fp16) at |v| (normal range)."""
    mant = 7 if dtype == torch.bfloat16 else 10
    e = np.floor(np.log2(np.maximum(np.abs(v), 2.0 ** -100)))
    return 2.0 ** (e - mant - 1)


def _check_close(out, ref, abs_sum):
    """out = round(y) with y the kernel's fp32 result; ref the fp64 value.
    |y - ref| <= acc := 2^-14 * sum_k |A[m,k] W[n,k]| * scales + |bias|: the
    fp8 matrix cores sum each block of 64 products in their own way (not an
    IEEE fp32 loop: the kernel matches hipBLASLt's fp8 GEMM bit for bit, not a
    sequential fp32 sum; the largest error seen is about 2^-15 of the sum, at
    one element of 4352 x 3072 x 80, where hipBLASLt gives the same bits),
    then the fp32 accumulation, scale and bias steps.  So |out - ref| <= half an
    output ulp at |ref| + acc, + acc."""
    o = out.double().cpu().numpy()
    acc = 2.0 ** -14 * abs_sum
    bound = _half_ulp(np.abs(ref) + acc, out.dtype) + 2 * acc
    err = np.abs(o - ref)
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err / bound), err.shape)
        raise AssertionError(f"{bad.sum()} of {err.size} outside the bound; worst at {i}: out {o[i]!r} "
                             f"ref {ref[i]!r} err {err[i]:.3g} bound {bound[i]:.3g} acc {acc[i]:.3g}")


def _abs_sum(xq, wq, sx, sw, bias):
    """sum_k |A W| * scales + |bias| per output, the magnitude the rounding errors scale with."""
    av = torch.from_numpy(np.abs(of.decode(xq))).double()
    wv = torch.from_numpy(np.abs(of.decode(wq))).double()
    if torch.cuda.is_available():
        av, wv = av.to(DEV), wv.to(DEV)
    s = (av @ wv.T).cpu().numpy() * float(np.float32(sx * sw))
    return s + (np.abs(bias)[None, :] if bias is not None else 0.0)


@pytest.mark.parametrize("M,N,K", [
    (1536, 4096, 4096),   # 192 x 128 tiles
    (4352, 3072, 3072),   # 256 x 256 tiles
    (300, 272, 4096),     # 64 x 64 tiles, ragged M and N
    (1, 16, 16),
    (17, 48, 80),         # K tail of 16 bytes
    (513, 1040, 1104),    # K = 17 * 64 + 16
    (256, 256, 128),
    (256, 3072, 12288),   # K split in 5 (through the workspace variant)
    (100, 1040, 8192),    # K split in 8, ragged M and N
    (1543, 9232, 1104),   # 256 x 256 tiles on columns [0, 8192), 256 x 128 on the rest
    (803, 8416, 1104),    # 256 x 128 tiles on columns [0, 6400), 128 x 128 on the rest
    (256, 1552, 3072),    # 128 x 128 or 64 x 64 tiles, ragged N
    (4352, 3072, 80),     # 256 x 256 tiles (128 k-bytes per stage): one stage, 80 of its bytes
    (2304, 2560, 144),    # two stages, the second 16 bytes deep
    (2000, 4400, 400),    # ragged M and N, 256 x 256 then 256 x 128 columns, a 16-byte k tail
    (2000, 4400, 12304),  # the same with a long K: 96 stages of 128 bytes and a 16-byte tail
])
@pytest.mark.parametrize("bias", [False, True])
def test_gemm_vs_fp64_oracle(qik, M, N, K, bias):
    a, w, xq, wq, sx, sw = _gemm_operands(M, N, K, 1000 + M + N + K)
    b = torch.randn(N, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16) if bias else None
    out = qik.fp8_linear(a, w, torch.tensor([sx], device=DEV), torch.tensor([sw], device=DEV),
                         b.to(DEV) if bias else None)
    torch.cuda.synchronize()
    bnp = b.float().numpy() if bias else None
    if M * N * K <= 1 << 31:
        ref = of.scaled_mm(xq, wq, sx, sw, bnp)
    else:
        av = torch.from_numpy(of.decode(xq)).to(DEV)
        wv = torch.from_numpy(of.decode(wq)).to(DEV)
        acc = (av.double() @ wv.double().T)
        ab = float(np.float32(sx * sw))
        ref = (acc * ab + (b.to(DEV).double()[None, :] if bias else 0)).cpu().numpy()
    _check_close(out, ref, _abs_sum(xq, wq, sx, sw, bnp))


def test_gemm_fp16_out_and_strided_rows(qik):
    M, N, K = 640, 512, 1024
    a, w, xq, wq, sx, sw = _gemm_operands(M, N, K, 77, lda=1040)
    assert a.stride(0) == 1040
    b = torch.randn(N, generator=torch.Generator().manual_seed(4)).to(torch.float16)
    out = qik.fp8_linear(a, w, torch.tensor([sx], device=DEV), torch.tensor([sw], device=DEV), b.to(DEV),
                         out_dtype=torch.float16)
    assert out.dtype == torch.float16
    bnp = b.float().numpy()
    _check_close(out, of.scaled_mm(xq, wq, sx, sw, bnp), _abs_sum(xq, wq, sx, sw, bnp))


@pytest.mark.parametrize("M,N,K", [
    (640, 512, 1024),     # 64 x 64 tiles
    (1536, 4096, 512),    # 256 x 128 tiles
    (4352, 3072, 256),    # 256 x 256 tiles
    (803, 8416, 320),     # 256 x 128 then 128 x 128 columns
    (4352, 9216, 192),    # 256 x 256 then 256 x 128 columns
    (1536, 4096, 256),    # 192 x 128 tiles
    (1500, 4000, 320),    # ragged M and N
    (256, 3072, 12288),   # K split in 5 (workspace variant)
    (100, 1040, 8192),    # K split in 8, ragged M and N
])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16])
def test_gemm_output_row_stride(qik, M, N, K, out_dtype):
    """An output whose rows are ldc > N elements apart (a column slice of a
    wider buffer) gets the same values as a contiguous one, and the columns
    past N keep what they held: the epilogue's whole-row stores address rows
    by ldc and stop at N."""
    a, w, xq, wq, sx, sw = _gemm_operands(M, N, K, 300 + N)
    sa, sb = torch.tensor([sx], device=DEV), torch.tensor([sw], device=DEV)
    b = torch.randn(N, generator=torch.Generator().manual_seed(6)).to(out_dtype).to(DEV)
    import ctypes
    from qwen_image_kernel_amd import _lib
    from qwen_image_kernel_amd import fp8 as f8
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    want = torch.empty(M, N, dtype=out_dtype, device=DEV)
    args = f8._gemm_args(a, w, sa, sb, b, want)
    need = ctypes.c_int64(0)
    assert lib.qik_fp8_gemm_workspace_size(ctypes.byref(args), ctypes.byref(need)) == 0
    ws = torch.full((max(need.value // 4, 4),), float("nan"), dtype=torch.float32, device=DEV)  # garbage
    assert lib.qik_fp8_gemm_ws(ctypes.byref(args), ws.data_ptr(), need.value, stream) == 0
    wide = torch.full((M, N + 48), -7.0, dtype=out_dtype, device=DEV)
    got = wide[:, :N]
    assert got.stride(0) == N + 48
    args = f8._gemm_args(a, w, sa, sb, b, got)
    assert lib.qik_fp8_gemm_ws(ctypes.byref(args), ws.data_ptr(), need.value, stream) == 0
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    assert (wide[:, N:] == -7.0).all()


@pytest.mark.parametrize("M,K,N,label", [(1536, 4096, 4096, "qkv-like"), (1536, 12288, 4096, "mlp-out-like"),
                                         (4352, 3072, 3072, "H*D=3072 out"), (4352, 3072, 9216, "H*D=3072 fused qkv")])
def test_fp8linear_matches_reference_test_bar(qik, M, K, N, label):
    """tests/test_fp8.py:16-30: FP8Linear.from_linear(nn.Linear * 0.02) within rel-err 0.06 of fp32."""
    torch.manual_seed(0)
    lin = torch.nn.Linear(K, N, bias=False, dtype=torch.bfloat16, device=DEV)
    with torch.no_grad():
        lin.weight.mul_(0.02)
    x = torch.randn(M, K, device=DEV, dtype=torch.bfloat16)
    ref = x.float() @ lin.weight.float().t()
    fq = qik.FP8Linear.from_linear(lin).to(DEV)
    out = fq(x)
    rel = ((out.float() - ref).norm() / ref.norm()).item()
    assert rel < 0.06, (label, rel)
    # and tightly against the same computation on the dequantised operands (fp64)
    xq, s_a = torch_act_quant(x)
    ab = (s_a * fq.weight_scale).double()
    dq = (xq.double() @ fq.weight.double().t()) * ab
    asum = (xq.double().abs() @ fq.weight.double().abs().t()) * ab
    _check_close(out, dq.cpu().numpy(), asum.cpu().numpy())


def test_fp8linear_forward_paths(qik):
    torch.manual_seed(1)
    # bias, 3-d input, fp16 activations
    lin = torch.nn.Linear(512, 768, bias=True, dtype=torch.float16, device=DEV)
    fq = qik.FP8Linear.from_linear(lin)
    assert fq.weight.dtype == torch.float8_e4m3fn and fq.bias.dtype == torch.bfloat16
    x = torch.randn(2, 33, 512, device=DEV, dtype=torch.float16)
    out = fq(x)
    assert out.shape == (2, 33, 768) and out.dtype == torch.float16
    xq, s_a = torch_act_quant(x.reshape(-1, 512))
    ab = (s_a * fq.weight_scale).double()
    want = (xq.double() @ fq.weight.double().t()) * ab + fq.bias.double()
    asum = (xq.double().abs() @ fq.weight.double().abs().t()) * ab + fq.bias.double().abs()
    # the bf16 result converted to fp16 (exact for these magnitudes)
    _check_close(out.reshape(-1, 768).to(torch.bfloat16), want.cpu().numpy(), asum.cpu().numpy())
    # fewer than 256 inputs: the bf16 path on the dequantised weight (fp8.py:79-84)
    small = torch.nn.Linear(64, 3072, bias=True, dtype=torch.bfloat16, device=DEV)
    fs = qik.FP8Linear.from_linear(small)
    x = torch.randn(4, 100, 64, device=DEV, dtype=torch.bfloat16)
    w = (fs.weight.to(torch.bfloat16).float() * fs.weight_scale).to(torch.bfloat16)
    want = torch.nn.functional.linear(x, w, fs.bias)
    assert torch.equal(fs(x), want)
    # the same with fp32 activations: the weight is the fp32 product, unrounded
    fs32 = qik.FP8Linear.from_linear(torch.nn.Linear(64, 512, bias=False, device=DEV))
    x32 = torch.randn(3, 64, device=DEV)
    w32 = fs32.weight.to(torch.bfloat16).float() * fs32.weight_scale
    assert torch.equal(fs32(x32), torch.nn.functional.linear(x32, w32, None))


def test_from_linear_cpu_and_device_weights_follow_torch_there(qik):
    """A CPU weight is quantised on the CPU (torch's CPU ops: true divisions),
    a device weight on the device (torch's device ops: the amax times the
    reciprocal of 448), each bit-identical to the reference's ops where the
    weight lives; the two agree except where the scales differ in the last bit."""
    torch.manual_seed(2)
    lin = torch.nn.Linear(1024, 512, bias=True, dtype=torch.bfloat16)
    fc = qik.FP8Linear.from_linear(lin)
    assert fc.weight.device.type == "cpu"
    s_cpu = (lin.weight.data.float().abs().amax() / 448.0).clamp_min(1e-12)
    w_cpu = (lin.weight.data.float() / s_cpu).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    assert torch.equal(fc.weight.view(torch.uint8), w_cpu.view(torch.uint8))
    fg = qik.FP8Linear.from_linear(lin.to(DEV))
    wq, sw = torch_weight_quant(lin.weight.data.float())
    assert torch.equal(fg.weight.view(torch.uint8), wq.view(torch.uint8)) and torch.equal(fg.weight_scale, sw)
    if torch.equal(fc.weight_scale, fg.weight_scale.cpu()):
        assert torch.equal(fc.weight.view(torch.uint8), fg.weight.view(torch.uint8).cpu())


def test_fp8linear_module_contract_after_a_forward(qik):
    """After a forward the module deep-copies and pickles, and .to('cpu')
    releases its device weight (the reference's runtime moves the DiT off the
    GPU before the VAE decode, runtime.py:643-645)."""
    import copy
    import gc
    import pickle
    torch.manual_seed(3)
    N, K = 4096, 3072
    fq = qik.FP8Linear.from_linear(torch.nn.Linear(K, N, bias=True, dtype=torch.bfloat16, device=DEV))
    x = torch.randn(256, K, device=DEV, dtype=torch.bfloat16)
    want = fq(x)
    assert "_calls" in fq.__dict__
    c = copy.deepcopy(fq)
    assert torch.equal(c(x), want)
    pickle.dumps(fq)
    del c
    gc.collect()
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated(DEV)
    fq.to("cpu")
    gc.collect()
    after = torch.cuda.memory_allocated(DEV)
    assert before - after >= N * K, (before, after)
    assert fq.weight.device.type == "cpu"
    fq.to(DEV)
    assert torch.equal(fq(x), want)


def test_convert_linears_fp8_and_state_dict(qik):
    from qwen_image_kernel_amd import fp8 as f8
    net = torch.nn.Sequential(torch.nn.Linear(256, 256), torch.nn.GELU(),
                              torch.nn.Sequential(torch.nn.Linear(256, 512, bias=False))).to(DEV)
    names = f8.convert_linears_fp8(net, skip_patterns=("2.0",))
    assert names == ["0"]
    assert isinstance(net[0], f8.FP8Linear) and isinstance(net[2][0], torch.nn.Linear)
    sd = f8.fp8_state_dict(net)
    assert sd["0.weight"].dtype == torch.float8_e4m3fn and sd["0.weight_scale"].shape == (1,)
    assert sd["2.0.weight"].dtype == torch.float32


@pytest.mark.parametrize("M,N,K,bias", [(1536, 4096, 4096, False), (4352, 3072, 3072, True),
                                        (300, 272, 4096, True), (513, 1040, 1104, False),
                                        (4352, 9216, 3072, True), (803, 8416, 1104, True),
                                        (256, 3072, 12288, True), (4352, 3072, 80, False),
                                        (2000, 4400, 400, True)])
def test_gemm_matches_torch_scaled_mm(qik, M, N, K, bias):
    """torch._scaled_mm is the call the reference makes (fp8.py:87-88); on this
    device it is hipBLASLt's fp8 GEMM.  The kernel agrees with it on (almost)
    every element, and nowhere by more than one bf16 step."""
    a, w, xq, wq, sx, sw = _gemm_operands(M, N, K, 31 + M + N + K)
    sa, sb = torch.tensor([sx], device=DEV), torch.tensor([sw], device=DEV)
    b = (torch.randn(N, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16).to(DEV) if bias else None)
    try:
        want = torch._scaled_mm(a, w.t(), scale_a=sa, scale_b=sb, bias=b, out_dtype=torch.bfloat16)
    except (RuntimeError, NotImplementedError) as e:
        pytest.skip(f"torch._scaled_mm unavailable here: {e}")
    got = qik.fp8_linear(a, w, sa, sb, b)
    same = (got.view(torch.int16) == want.view(torch.int16)).float().mean().item()
    print(f"M={M} N={N} K={K} bias={bias}: {same:.6f} of the outputs bit-identical to torch._scaled_mm")
    assert same >= 0.99
    d = (got.double() - want.double()).abs()
    step = torch.from_numpy(2 * _half_ulp(want.double().cpu().numpy(), torch.bfloat16)).to(DEV)
    assert (d <= step).all()


def _random_gemm_shapes(n, seed):
    """Seeded shapes over every tile plan: M from 1 to 5000, N and K multiples
    of 16 up to 13000 and 6000 (ragged against every tile shape and both stage
    depths)."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        M = int(rng.choice([rng.integers(1, 300), rng.integers(300, 2000), rng.integers(2000, 5000)]))
        N = 16 * int(rng.integers(1, 13000 // 16))
        K = 16 * int(rng.integers(1, 6000 // 16))
        out.append((M, N, K))
    return out


@pytest.mark.parametrize("M,N,K", _random_gemm_shapes(14, 2024))
def test_gemm_random_shapes_match_torch_scaled_mm(qik, M, N, K):
    """Random shapes, through the entry point FP8Linear uses (qik_fp8_gemm_ws,
    K split included): at least 99% of the outputs bit-identical to
    torch._scaled_mm, the rest within one bf16 step."""
    a, w, xq, wq, sx, sw = _gemm_operands(M, N, K, 7 * M + 3 * N + K)
    sa, sb = torch.tensor([sx], device=DEV), torch.tensor([sw], device=DEV)
    try:
        want = torch._scaled_mm(a, w.t(), scale_a=sa, scale_b=sb, out_dtype=torch.bfloat16)
    except (RuntimeError, NotImplementedError) as e:
        pytest.skip(f"torch._scaled_mm unavailable here: {e}")
    got = qik.fp8_linear(a, w, sa, sb, None)
    same = (got.view(torch.int16) == want.view(torch.int16)).float().mean().item()
    print(f"M={M} N={N} K={K}: {same:.6f} of the outputs bit-identical to torch._scaled_mm")
    assert same >= 0.99
    d = (got.double() - want.double()).abs()
    step = torch.from_numpy(2 * _half_ulp(want.double().cpu().numpy(), torch.bfloat16)).to(DEV)
    assert (d <= step).all()
