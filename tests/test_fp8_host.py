"""fp8 pieces that run without a GPU: the host weight quantiser and the
FP8Linear module contract (copy, pickle, device moves).

The host quantiser replaces ``quantize_weight_tensorwise`` (fp8.py:56-60) for a
weight in host memory, so it must give the bytes the reference's own torch ops
give on the CPU: scale = (amax / 448).clamp_min(1e-12) and codes =
(w / scale).clamp(+-448).to(float8_e4m3fn), both divisions true fp32 divisions.
Those torch ops are what the tests compare with, plus the oracle's encoder (pinned
against torch's cast and the format's closed form in test_oracle_fp8.py).
"""

import copy
import gc
import io
import pickle
import weakref

import numpy as np
import pytest
import torch

from oracle import fp8 as of
from qwen_image_kernel_amd import _lib
from qwen_image_kernel_amd import fp8 as f8


def torch_cpu_weight_quant(w):
    """fp8.py:56-60, run on the CPU."""
    s = (w.abs().amax().float() / 448.0).clamp_min(1e-12)
    return (w.float() / s).clamp(-448.0, 448.0).to(torch.float8_e4m3fn), s.reshape(1)


def _bits(t):
    return t.view(torch.uint8) if t.dtype == torch.float8_e4m3fn else t.view(torch.int32)


def _check(w):
    got_q, got_s = f8.quantize_weight_tensorwise(w)
    want_q, want_s = torch_cpu_weight_quant(w)
    assert got_q.shape == w.shape and got_q.dtype == torch.float8_e4m3fn and got_q.device.type == "cpu"
    assert got_s.shape == (1,) and got_s.dtype == torch.float32
    assert torch.equal(_bits(got_s), _bits(want_s)), (got_s, want_s)
    assert torch.equal(_bits(got_q), _bits(want_q))
    return got_q, got_s


def _inputs(shape, dtype, seed, kind="normal"):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g)
    if kind == "outlier":
        x.view(-1)[x.numel() // 3] = 3e4
    elif kind == "tiny":
        x = x * 1e-20
    elif kind == "zero":
        x = torch.zeros(*shape)
    elif kind == "wide":
        x = x * torch.exp2(torch.randint(-20, 20, shape, generator=g).float())
    return x.to(dtype)


@pytest.mark.parametrize("shape,dtype,kind", [
    ((3072, 512), torch.float32, "normal"),
    ((1024, 300), torch.float32, "wide"),
    ((517, 129), torch.bfloat16, "normal"),
    ((333, 257), torch.float16, "wide"),
    ((1,), torch.float32, "normal"),
    ((7, 3), torch.bfloat16, "outlier"),
    ((64, 256), torch.float32, "tiny"),
    ((64, 256), torch.float16, "zero"),
    ((100003,), torch.float32, "outlier"),
])
def test_host_weight_quantiser_matches_torch_cpu_ops(shape, dtype, kind):
    _check(_inputs(shape, dtype, 11 + len(shape), kind))


@pytest.mark.parametrize("amax", [448.0, 1.0, 0.02, 3.0e-3, 1e-9, 65504.0, 3.3e38])
def test_host_weight_quantiser_every_bf16_value(amax):
    """Every finite bf16 magnitude up to the planted amax, both signs: every
    code boundary and tie the quotient can land on."""
    u = np.arange(0, 0x7F80, dtype=np.uint32) << 16
    vals = u.view(np.float32)
    vals = vals[vals <= np.float32(amax)]
    w = torch.from_numpy(np.concatenate([vals, -vals, np.float32([amax])]))
    _check(w)
    _check(w.to(torch.bfloat16))


def test_host_weight_quantiser_every_fp16_value():
    u = np.arange(0, 0x7C00, dtype=np.uint16)
    vals = u.view(np.float16)
    w = torch.from_numpy(np.concatenate([vals, -vals]))
    _check(w)
    _check(w.float())


def test_host_weight_quantiser_non_finite_poisons_like_torch():
    for bad in (float("nan"), float("inf"), float("-inf")):
        w = _inputs((64, 32), torch.float32, 3)
        w[5, 7] = bad
        _check(w)


def test_host_weight_quantiser_codes_match_the_oracle():
    w = _inputs((256, 384), torch.float32, 4, "wide")
    q, s = f8.quantize_weight_tensorwise(w)
    quot = (w.numpy() / s.numpy()[0]).astype(np.float32).clip(-448, 448)
    np.testing.assert_array_equal(q.view(torch.uint8).numpy(), of.e4m3fn_encode(quot))


def test_host_weight_quantiser_does_not_depend_on_threads():
    w = _inputs((4096, 257), torch.float32, 5, "wide")
    outs = []
    for nt in (1, 3, 8, 64):
        codes = torch.empty(w.shape, dtype=torch.float8_e4m3fn)
        scale = torch.empty(1)
        _lib.check(_lib.load().qik_fp8_quantize_weight_host(w.data_ptr(), _lib.DTYPE_FP32, w.numel(),
                                                            codes.data_ptr(), scale.data_ptr(), nt), "host quant")
        outs.append((codes.view(torch.uint8).clone(), scale.clone()))
    for c, s in outs[1:]:
        assert torch.equal(c, outs[0][0]) and torch.equal(s, outs[0][1])


def test_host_weight_quantiser_rejects_bad_arguments():
    lib = _lib.load()
    buf = torch.zeros(16)
    out = torch.empty(16, dtype=torch.uint8)
    s = torch.empty(1)
    assert lib.qik_fp8_quantize_weight_host(buf.data_ptr(), 7, 16, out.data_ptr(), s.data_ptr(), 1) == -3
    assert lib.qik_fp8_quantize_weight_host(buf.data_ptr(), _lib.DTYPE_FP32, 0, out.data_ptr(), s.data_ptr(), 1) == -5
    assert lib.qik_fp8_quantize_weight_host(None, _lib.DTYPE_FP32, 16, out.data_ptr(), s.data_ptr(), 1) == -1
    with pytest.raises(ValueError):
        f8.quantize_weight_tensorwise(torch.zeros(0))
    with pytest.raises(ValueError):
        f8.quantize_weight_tensorwise(torch.zeros(4, dtype=torch.float64))


def test_from_linear_on_a_host_without_gpu():
    """FP8Linear.from_linear of a CPU nn.Linear (the offline conversion,
    quantize_offline.py:15-25) gives the reference's buffers on the CPU."""
    torch.manual_seed(2)
    lin = torch.nn.Linear(1024, 512, bias=True, dtype=torch.bfloat16)
    fc = f8.FP8Linear.from_linear(lin)
    assert fc.weight.device.type == "cpu" and fc.weight.dtype == torch.float8_e4m3fn
    want_q, want_s = torch_cpu_weight_quant(lin.weight.data.float())
    assert torch.equal(fc.weight.view(torch.uint8), want_q.view(torch.uint8))
    assert torch.equal(fc.weight_scale, want_s)
    assert fc.bias.dtype == torch.bfloat16 and torch.equal(fc.bias, lin.bias.data)
    net = torch.nn.Sequential(torch.nn.Linear(256, 256), torch.nn.GELU(), torch.nn.Linear(256, 64, bias=False))
    assert f8.convert_linears_fp8(net) == ["0", "2"]
    sd = f8.fp8_state_dict(net)
    assert sd["0.weight"].dtype == torch.float8_e4m3fn and sd["2.weight_scale"].shape == (1,)


def _filled_module():
    """An FP8Linear whose launch cache holds an entry with ctypes argument
    structs (as a forward on the device leaves it)."""
    m = f8.FP8Linear(512, 256, bias=True)
    x = torch.zeros(4, 512, dtype=torch.bfloat16)
    ent = f8._prepare_linear(x, m.weight, m.weight_scale, m.bias, 256)
    ent.qargs = _lib.QikFp8QuantArgs()
    ent.gargs = _lib.QikFp8GemmArgs()
    m.__dict__["_calls"] = {(x.shape, x.stride(), x.dtype, x.device): ent}
    return m, ent


def test_fp8linear_copies_and_pickles_after_a_forward():
    m, _ = _filled_module()
    with pytest.raises((ValueError, TypeError)):
        pickle.dumps(m.__dict__["_calls"])  # the cache itself is not picklable ...
    c = copy.deepcopy(m)                    # ... but the module is
    assert "_calls" not in c.__dict__ and "_calls" in m.__dict__
    for name in ("weight", "weight_scale", "bias"):
        assert torch.equal(getattr(c, name).view(torch.uint8), getattr(m, name).view(torch.uint8))
    pickle.dumps(m)
    # a round trip through torch.save / torch.load (plain pickle cannot load
    # fp8 storages back, the reference's module alike)
    buf = io.BytesIO()
    torch.save(m, buf)
    buf.seek(0)
    r = torch.load(buf, weights_only=False)  # a module this test wrote itself
    assert "_calls" not in r.__dict__
    assert r.in_features == 512 and r.out_features == 256 and torch.equal(r.weight_scale, m.weight_scale)


def test_fp8linear_cache_holds_no_tensor_and_is_dropped_by_moves():
    m, ent = _filled_module()
    w = weakref.ref(m.weight)
    assert ent.matches(m.weight, m.weight_scale, m.bias)
    m.to(torch.device("cpu"))               # _apply: the cache goes
    assert "_calls" not in m.__dict__
    m.__dict__["_calls"] = {"k": ent}
    m.weight = torch.zeros(256, 512, dtype=torch.float8_e4m3fn)  # buffer replaced
    assert not ent.matches(m.weight, m.weight_scale, m.bias)
    gc.collect()
    assert w() is None                      # the entry did not keep the old weight alive
    m2, ent2 = _filled_module()
    m2.weight_scale.mul_(2.0)               # in-place change: versions differ
    assert not ent2.matches(m2.weight, m2.weight_scale, m2.bias)
    m2.half()
    assert "_calls" not in m2.__dict__
