"""Oracle: fp8e4m3fn / bf16 rounding and the slab quantisation (CPU)."""

import numpy as np
import pytest
import torch

from oracle import fp8 as of


def test_decode_table_closed_form_points():
    t = of.e4m3fn_decode_table()
    assert t[0x00] == 0.0 and np.signbit(t[0x80])
    assert t[0x01] == 2.0 ** -9            # smallest subnormal
    assert t[0x07] == 7 * 2.0 ** -9        # largest subnormal
    assert t[0x08] == 2.0 ** -6            # smallest normal
    assert t[0x38] == 1.0                  # exponent 7 = bias
    assert t[0x7E] == 448.0 and t[0xFE] == -448.0
    assert np.isnan(t[0x7F]) and np.isnan(t[0xFF])
    pos = t[:127]
    assert (np.diff(pos) > 0).all()        # codes 0..126 are increasing


def test_decode_table_matches_torch():
    tt = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    t = of.e4m3fn_decode_table()
    same = (t == tt) | (np.isnan(t) & np.isnan(tt))
    assert same.all()


def test_encode_rne_matches_torch_cast():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        (rng.standard_normal(200000) * 40).astype(np.float32),
        (rng.standard_normal(50000) * 1e-2).astype(np.float32),   # subnormal range
    ]).clip(-448, 448)
    t = of.e4m3fn_decode_table()[:127].astype(np.float64)
    mids = ((t[:-1] + t[1:]) / 2).astype(np.float32)             # exact ties
    x = np.concatenate([x, mids, -mids, np.float32([0.0, -0.0, 448.0, -448.0, 2.0 ** -10])])
    want = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(of.e4m3fn_encode(x), want)


def test_ties_go_to_even_mantissa():
    # 1.0 = 0x38, next is 1.125 = 0x39; the midpoint 1.0625 rounds to the even code 0x38
    assert of.e4m3fn_encode(np.float32([1.0625]))[0] == 0x38
    # 1.125 = 0x39 and 1.25 = 0x3A; midpoint 1.1875 -> 0x3A (even)
    assert of.e4m3fn_encode(np.float32([1.1875]))[0] == 0x3A
    # half the smallest subnormal ties to zero
    assert of.e4m3fn_encode(np.float32([2.0 ** -10]))[0] == 0x00


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(1)
    u = rng.integers(0, 2 ** 32, size=200000, dtype=np.uint64).astype(np.uint32)
    u = u[(u & 0x7F800000) != 0x7F800000]   # finite only
    x = u.view(np.float32)
    want = torch.from_numpy(x.copy()).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(of.bf16_round(x), want)


def _torch_store(v):
    """The slab store's quantisation written with torch library ops on the CPU.

    ``amax * (1 / 448)`` is how torch on the GPU evaluates the reference's
    ``amax / 448.0`` (scalar divisor -> multiply by the fp32 reciprocal).
    """
    vt = v.transpose(1, 2).float()
    scale = vt.abs().amax(dim=(2, 3)).float() * torch.tensor(1.0 / 448.0, dtype=torch.float32)
    scale = scale.clamp_min(1e-12)
    vq = (vt / scale[:, :, None, None]).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return vq.view(torch.uint8).numpy(), scale.numpy()


def test_quantize_per_head_matches_torch_ops():
    g = torch.Generator().manual_seed(3)
    v = torch.randn(2, 96, 3, 128, generator=g).to(torch.bfloat16)
    v[0, :, 1] *= 1e-3                      # a small-magnitude head
    v[1, :, 2] = 0                          # an all-zero head -> scale clamps to 1e-12
    codes, scale = of.quantize_per_head(v.float().numpy())
    tc, ts = _torch_store(v)
    np.testing.assert_array_equal(scale, ts)
    np.testing.assert_array_equal(codes, tc)
    assert scale[1, 2] == np.float32(1e-12)


def test_quantize_round_trip_error_bound():
    """fp8-V store/dequant relative error < 0.03 (tests/test_kv_cache.py:29-38)."""
    g = torch.Generator().manual_seed(4)
    v = torch.randn(1, 640, 4, 128, generator=g).to(torch.bfloat16)
    codes, scale = of.quantize_per_head(v.float().numpy())
    deq = of.dequant_bf16(codes, scale[:, :, None, None])            # [B, H, P, D]
    ref = v.float().numpy().transpose(0, 2, 1, 3)
    rel = np.linalg.norm(deq - ref) / np.linalg.norm(ref)
    assert rel < 0.03


def test_scale_uses_reciprocal_multiply_not_division():
    """The two roundings differ for some amax: the oracle must follow the reciprocal form."""
    amax = np.float32(np.linspace(0.5, 8.0, 20001))
    inv = np.float32(1.0) / np.float32(448.0)
    assert (amax * inv != amax / np.float32(448.0)).any()
    v = np.zeros((1, 1, 1, 2), dtype=np.float32)
    for a in amax[:200]:
        v[0, 0, 0, 0] = a
        _, scale = of.quantize_per_head(v)
        assert scale[0, 0] == max(a * inv, np.float32(1e-12))


# --- W8A8 linear: tensorwise quantisation and the scaled GEMM (fp8.py:24-60, 87-88) ---


def test_tensor_scale_known_answers():
    # all zeros: the clamp (fp8.py:26)
    assert of.tensor_scale(np.zeros(10, np.float32)) == np.float32(1e-12)
    # amax * fp32(1/448), not amax / 448 (the GPU's scalar division)
    x = np.float32([3.0, -7.0, 1.0])
    assert of.tensor_scale(x) == np.float32(np.float32(7.0) * (np.float32(1.0) / np.float32(448.0)))
    assert np.isnan(of.tensor_scale(np.float32([1.0, np.nan])))


@pytest.mark.parametrize("fn", [of.quantize_tensorwise, of.quantize_weight_tensorwise])
def test_tensorwise_quant_known_answers(fn):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(4096) * 5).astype(np.float32)
    codes, s = fn(x)
    # the largest magnitude lands on the largest code
    i = np.argmax(np.abs(x))
    assert codes[i] == (0xFE if x[i] < 0 else 0x7E)
    # representable values times the scale come back as themselves
    table = of.e4m3fn_decode_table()
    vals = table[rng.integers(0, 127, 1000)] * rng.choice([-1, 1], 1000)
    vals[0] = 448.0
    y = (vals * np.float32(0.37)).astype(np.float32)
    c, sy = fn(y)
    np.testing.assert_allclose(of.decode(c) * sy, y, rtol=1e-6)
    # the codes dequantise to within half an fp8 step of x / scale
    back = of.decode(codes) * s
    assert (np.abs(back - x) <= np.abs(x) * 2.0 ** -4 + s * 2.0 ** -10).all()


def test_activation_and_weight_forms_differ_only_at_rounding():
    rng = np.random.default_rng(4)
    x = (rng.standard_normal(200000)).astype(np.float32)
    ca, sa = of.quantize_tensorwise(x)
    cw, sw = of.quantize_weight_tensorwise(x)
    assert sa == sw
    diff = ca != cw
    assert diff.mean() < 1e-3                      # x*(1/s) and x/s differ by an ulp at most
    assert (np.abs(ca[diff].astype(int) - cw[diff].astype(int)) == 1).all()


def test_tensorwise_quant_matches_torch_on_cpu():
    """The same steps written with torch's CPU ops (the reciprocal of 448 formed
    explicitly, as the GPU does) give the same codes."""
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((64, 300)) * 3).astype(np.float32)
    t = torch.from_numpy(x)
    s = torch.clamp_min(t.abs().amax() * torch.tensor(1.0 / 448.0, dtype=torch.float32), 1e-12)
    want = (t * (1.0 / s)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got, gs = of.quantize_tensorwise(x)
    assert np.float32(s.item()) == gs
    np.testing.assert_array_equal(got, want)


def test_scaled_mm_brute_force_and_identity():
    rng = np.random.default_rng(6)
    a = rng.integers(0, 127, (5, 48)).astype(np.uint8) | (rng.integers(0, 2, (5, 48)) << 7).astype(np.uint8)
    w = rng.integers(0, 127, (7, 48)).astype(np.uint8)
    bias = rng.standard_normal(7).astype(np.float32)
    got = of.scaled_mm(a, w, 0.5, 0.25, bias)
    t = of.e4m3fn_decode_table().astype(np.float64)
    for m in range(5):
        for n in range(7):
            s = sum(t[a[m, k]] * t[w[n, k]] for k in range(48))
            assert got[m, n] == s * 0.125 + np.float64(bias[n])
    # W = e_k (code of 1.0 at column k): column k of A times the scales
    eye = np.zeros((48, 48), np.uint8)
    eye[np.arange(48), np.arange(48)] = 0x38
    np.testing.assert_array_equal(of.scaled_mm(a, eye, 2.0, 3.0), t[a] * 6.0)
