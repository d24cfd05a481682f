"""Benchmark: block-causal attention TFLOP/s (unmasked FLOPs) on one MI355X.

One step = one denoising step's attention at the two headline shapes:
32 layers of the 1024px text-to-image prefill shape (B1 H24 D128, 256 causal
text + 4096 image tokens, fresh K/V, ragged L, independent inputs per layer)
followed by 32 layers of the 768px single-reference edit decode shape (4096
target queries against a 2560-token slab prefix with bf16 K and fp8e4m3fn V
plus 4096 fresh keys, uniform L).  Inputs are resident in HBM before timing.

value = unmasked FLOPs of the step / wall time of the step, where a FLOP pair
counts 2*D for QK^T and 2*D for PV per allowed (query, key) pair.

Prints ONE JSON line (rank 0, N=1).  ``--gpus N`` with N > 1 exits with a
message: this build runs on one GPU.

``side_ops`` in the same line (outside the timed step, not part of ``value``):
the two HBM-bound kernels beside the attention call, each at its shape in the
headline workloads -- per-head RMSNorm + RoPE of the 1024px Q ([1, 4352, 24,
128] bf16) and the slab store of the 768px edit prefix ([1, 2560, 24, 128] K
and V, V to fp8) -- device time per call of prebuilt C-ABI launches back to back (``us``), the
time per call of Python API calls issued back to back (``api_us``: two events around the
batch, so it is the device time unless the host is slower) and the host time per API call
(``host_us``: wall time of a loop of calls, the device running behind), priced in algorithmic HBM
bytes against 8 TB/s, beside the same torch computation on the host CPU; and
the W8A8 fp8 linear (FP8Linear, the DiT's projections) at the reference test's
shape ([1536, 4096] x [4096, 4096]), at the 1024px layer's fused QKV,
MLP-in and MLP-out shapes (4352 tokens, H*D = 3072) and at the text stream's
fused QKV and MLP-out (256 tokens): GEMM device time, TFLOP/s against
the 5.0 PF dense fp8 peak, the activation quantiser's time, the whole
FP8Linear call through the Python API, torch._scaled_mm (hipBLASLt, the call
the reference makes) on the same device, timed in batches alternating with the
GEMM's (medians), and an fp32 matmul of the
dequantised operands on the host CPU for the reference shape.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "block-causal attn TFLOP/s (unmasked) & % bf16 MFMA peak, 1024px + edit"
PEAK_BF16_TFLOPS = 2516.6   # MI355X dense bf16 MFMA: 256 CU x 4096 FLOP/clk x 2.4 GHz ("2.5 PF")
PEAK_HBM_GBS = 8000.0
PEAK_FP8_TFLOPS = 5000.0    # MI355X dense fp8 MFMA ("5.0 PF" dense)


def parse():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layers", type=int, default=32, help="layers per shape in one step")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="target duration of the CPU baseline sample (0 disables it)")
    ap.add_argument("--clock-seconds", type=float, default=1.5,
                    help="after the timed region, sample the GPU clock for this long under the same "
                         "launches (0 disables it)")
    ap.add_argument("--only", choices=["t2i_1024", "edit_768"], default=None,
                    help="time one shape only (profiling aid; the default times both)")
    ap.add_argument("--all-workloads", action="store_true",
                    help="instead of the benchmark, time every workload of the benchmark set (t2i_512, "
                         "t2i_1024, edit_768, multiref_cfg), print one JSON line and exit")
    ap.add_argument("--head-share", action="store_true",
                    help="instead of the benchmark, time one GPU's share of the heads (H/n for n = 1, 2, 4, "
                         "8) of t2i_1024 and edit_768, print one JSON line and exit")
    ap.add_argument("--copy-calibration-mb", type=int, default=0,
                    help="instead of the benchmark, run 5 plain device copies of this many MiB "
                         "(reference point for the FETCH_SIZE / WRITE_SIZE counters) and exit")
    return ap.parse_args()


def copy_calibration(mb: int) -> None:
    import torch

    n = mb * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes_per_copy": n * 4, "copies": 5}), flush=True)


def cpu_leg(wl, inp, out, budget_s: float) -> dict:
    """The CPU baseline leg of one workload: torch explicit-mask SDPA in fp32
    (the reference's CPU path) on the host cores, timed per (b, h) on a
    bounded sample of heads of the layer the GPU just computed; and the GPU
    output of those heads against it (max-abs and mean-abs over every element
    of the sampled heads, the parity bar being 2e-2 / 2e-3)."""
    import torch

    from oracle import attention as oa

    cpu = {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}
    bl = oa.CpuSdpaBaseline(cpu["query"], cpu["key"], cpu["value"], wl.lengths(), cpu["cache_k"], cpu["cache_v"],
                            cpu["cache_v_scale"])
    got = out.float().cpu()
    heads, elapsed, max_abs, sum_abs, n = [], 0.0, 0.0, 0.0, 0
    pairs = [(b, h) for h in range(wl.H) for b in range(wl.B)]
    for b, h in pairs:
        t0 = time.perf_counter()
        ref = bl.run(b, h)
        elapsed += time.perf_counter() - t0
        d = (got[b, :, h] - ref).abs()
        max_abs = max(max_abs, float(d.max()))
        sum_abs += float(d.sum())
        n += d.numel()
        heads.append((b, h))
        if elapsed >= budget_s:
            break
    flops = 4 * wl.D * bl.pairs * len(heads)
    return {"cpu_tflops": round(flops / elapsed / 1e12, 6), "cpu_seconds": round(elapsed, 3),
            "cpu_heads": len(heads), "cpu_threads": torch.get_num_threads(), "cpu_model": cpu_model(),
            "cpu_what": "fp32 F.scaled_dot_product_attention with a bool [SQ, KV] mask per (b, h), fp8 V dequantised first",
            "max_abs_vs_cpu": float(f"{max_abs:.3e}"), "mean_abs_vs_cpu": float(f"{sum_abs / n:.3e}"),
            "heads_compared": len(heads)}


def _ws_launches(wl, nl: int, seed: int, dev):
    """``nl`` independent layers of workload ``wl`` as prebuilt qik_attn_fwd_ws launches.

    Returns (layers, calls, run): the input dicts, (args, workspace, bytes,
    output) per layer, and a function launching every layer once on the
    current stream."""
    import ctypes

    import torch

    import qwen_image_kernel_amd.workloads as wls
    from qwen_image_kernel_amd import _lib
    from qwen_image_kernel_amd.attention import make_args

    lib = _lib.load()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    layers = [wls.make_inputs(wl, seed=seed + i, device="cuda", gen_device="cuda") for i in range(nl)]
    calls = []
    for inp in layers:
        out = torch.empty_like(inp["query"])
        L = None if wl.uniform else inp["prefix_lengths"]
        a = make_args(inp["query"], inp["key"], inp["value"], L, None, out, inp["cache_k"], inp["cache_v"],
                      inp["cache_v_scale"], wl.uniform)
        nb = ctypes.c_int64()
        _lib.check(lib.qik_attn_workspace_size(ctypes.byref(a), ctypes.byref(nb)), "qik_attn_workspace_size")
        ws = torch.zeros(max(nb.value, 256), dtype=torch.uint8, device=dev)
        calls.append((a, ws, nb.value, out))

    def run():
        for a, ws, nb, _ in calls:
            _lib.check(lib.qik_attn_fwd_ws(ctypes.byref(a), ws.data_ptr(), nb, stream), "qik_attn_fwd_ws")

    return layers, calls, run


def _us_per_launch(run, n_calls: int, groups: int = 5, passes: int = 4) -> float:
    """3 warm-up passes, then ``groups`` groups of ``passes`` passes with HIP
    events around each group; the median group's time per launch in us."""
    import torch

    for _ in range(3):
        run()
    torch.cuda.synchronize()
    ts = []
    for _ in range(groups):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(passes):
            run()
        e1.record()
        torch.cuda.synchronize()
        ts.append(e0.elapsed_time(e1) * 1e3 / (passes * n_calls))
    return sorted(ts)[len(ts) // 2]


def all_workloads(cpu_seconds: float = 3.0) -> None:
    """Kernel time of every workload of the benchmark set through qik_attn_fwd_ws.

    Per workload: 8 independent layers launched back to back (multiref_cfg:
    4), 3 warm-up passes, then 5 groups of 4 passes with HIP events around
    each group; the median group gives the time per launch.  Then the CPU
    baseline leg (``cpu_leg``) on about ``cpu_seconds`` of heads of the first
    layer, with the GPU output of those heads compared against it.
    """
    import torch

    import qwen_image_kernel_amd.workloads as wls

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    res, runs = {}, []
    for name in ("t2i_512", "t2i_1024", "edit_768", "multiref_cfg", "ref_decode_1024"):
        wl = wls.workload(name)
        nl = 4 if name == "multiref_cfg" else 8
        layers, calls, run = _ws_launches(wl, nl, 40, dev)
        us = _us_per_launch(run, len(calls))
        tf = wl.flops() / us / 1e6
        res[name] = {"us_per_launch": round(us, 2), "tflops": round(tf, 1),
                     "pct_bf16_peak": round(100 * tf / PEAK_BF16_TFLOPS, 2), "layers": nl,
                     "shape": [wl.B, wl.SQ, wl.H, wl.D], "P": wl.P, "SN": wl.SN,
                     "unmasked_gflop": round(wl.flops() / 1e9, 3)}
        if cpu_seconds > 0:
            res[name].update(cpu_leg(wl, layers[0], calls[0][3], cpu_seconds))
            res[name]["gpu_over_cpu"] = round(res[name]["tflops"] / res[name]["cpu_tflops"], 1)
        print(name, json.dumps(res[name]), file=sys.stderr, flush=True)
        if name in ("t2i_1024", "edit_768"):
            runs.append((name, run))
    print(json.dumps({"all_workloads": res, "gpu_clock": clock_under_load(runs, dev, 1.5)}), flush=True)


def head_share() -> None:
    """One GPU's share of the heads of the two headline shapes, through qik_attn_fwd_ws.

    Attention shards by head without communication: on n GPUs each runs the
    same sequence with H/n heads.  For n = 1, 2, 4, 8 (H = 24, 12, 6, 3) this
    times 8 independent layers of that share launched back to back, as
    ``all_workloads`` does, and reports the time per launch, TFLOP/s against
    the bf16 peak, the row blocks of the launch and the workspace it takes.
    """
    import dataclasses

    import torch

    import qwen_image_kernel_amd.workloads as wls

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    res = {}
    for name in ("t2i_1024", "edit_768"):
        base = wls.workload(name)
        for n in (1, 2, 4, 8):
            wl = dataclasses.replace(base, H=base.H // n)
            _, calls, run = _ws_launches(wl, 8, 60, dev)
            us = _us_per_launch(run, len(calls))
            tf = wl.flops() / us / 1e6
            key = f"{name}_h{wl.H}"
            res[key] = {"gpus_sharing": n, "heads": wl.H, "us_per_launch": round(us, 2),
                        "tflops": round(tf, 1), "pct_bf16_peak": round(100 * tf / PEAK_BF16_TFLOPS, 2),
                        "row_blocks": wl.B * wl.H * -(-wl.SQ // 128), "workspace_bytes": calls[0][2],
                        "unmasked_gflop": round(wl.flops() / 1e9, 3)}
            print(key, json.dumps(res[key]), file=sys.stderr, flush=True)
    print(json.dumps({"head_share": res}), flush=True)


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "attn_fwd_traffic.txt")


def profiled_traffic(name: str):
    """HBM bytes per launch of the kernel for one shape, from the committed counter summary.

    The counters (FETCH_SIZE, WRITE_SIZE, each scaled by a plain-copy
    calibration) come from separate rocprofv3 --pmc runs of this script; the
    summary lists '<shape> <bytes>' lines.  None when the file or shape is absent.
    """
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                parts = line.split()
                if len(parts) == 2 and not line.startswith("#") and parts[0] == name:
                    return int(parts[1])
    except OSError:
        pass
    return None


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(wls, budget_s: float) -> dict:
    """Torch explicit-mask SDPA in fp32 on the host cores, on whole layers of both shapes.

    One layer of each shape is prepared once (untimed), then full layers (all
    heads) are timed alternately until ``budget_s`` seconds of CPU work (at
    least one layer of each, at most 40 layers).
    """
    import torch

    from oracle import attention as oa

    threads = torch.get_num_threads()
    prepared = []
    for name in ("t2i_1024", "edit_768"):
        wl = wls.workload(name)
        inp = wls.make_inputs(wl, seed=9000, device="cpu")
        bl = oa.CpuSdpaBaseline(inp["query"], inp["key"], inp["value"], wl.lengths(),
                                inp["cache_k"], inp["cache_v"], inp["cache_v_scale"])
        prepared.append((name, wl, bl))
    done_flops = 0
    elapsed = 0.0
    layers = {"t2i_1024": 0, "edit_768": 0}
    while sum(layers.values()) < 40 and (min(layers.values()) == 0 or elapsed < budget_s):
        for name, wl, bl in prepared:
            t0 = time.perf_counter()
            for b in range(wl.B):
                for h in range(wl.H):
                    bl.run(b, h)
            elapsed += time.perf_counter() - t0
            done_flops += 4 * wl.D * bl.pairs * wl.B * wl.H
            layers[name] += 1
    return {
        "value": round(done_flops / elapsed / 1e12, 6),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"{layers['t2i_1024']} layer(s) of t2i_1024 + {layers['edit_768']} of edit_768 "
                   f"(all 24 heads, fp32 F.scaled_dot_product_attention with a bool [SQ,KV] mask, fp8 V "
                   f"dequantised first) in {elapsed:.2f} s; torch threads {threads}, os.cpu_count() "
                   f"{os.cpu_count()}, {cpu_model()}"),
        "seconds": round(elapsed, 3),
    }


def _sysfs_device_dir(dev) -> str | None:
    """sysfs directory of the HIP device (PCI domain:bus:device.0), or the only card's."""
    import glob

    import torch

    p = torch.cuda.get_device_properties(dev)
    cand = f"/sys/bus/pci/devices/{p.pci_domain_id:04x}:{p.pci_bus_id:02x}:{p.pci_device_id:02x}.0"
    if os.path.exists(os.path.join(cand, "pp_dpm_sclk")):
        return cand
    cards = sorted(glob.glob("/sys/class/drm/card*/device/pp_dpm_sclk"))
    return os.path.dirname(cards[0]) if len(cards) == 1 else None


def _read_sclk_mhz(path: str) -> float | None:
    """The current shader clock from pp_dpm_sclk (the line marked '*', e.g. '1: 2400Mhz *')."""
    with open(path) as f:
        for line in f:
            if line.rstrip().endswith("*"):
                v = line.split(":", 1)[1].strip().rstrip("*").strip().lower().removesuffix("mhz")
                return float(v)
    return None


def _read_power_w(ddir: str) -> float | None:
    import glob

    for name in ("power1_input", "power1_average"):
        for f in sorted(glob.glob(os.path.join(ddir, "hwmon", "hwmon*", name))):
            try:
                with open(f) as fh:
                    return int(fh.read().strip()) / 1e6
            except (OSError, ValueError):
                continue
    return None


def clock_under_load(calls, dev, seconds: float = 1.5) -> dict:
    """GPU shader clock while the benchmark's own launches keep the GPU busy.

    Runs after the timed region: the step's launches are repeated for about
    ``seconds`` while a host thread samples the device's sysfs ``pp_dpm_sclk``
    (and board power) every 20 ms.  Every source is optional.  (amd-smi's
    per-XCD clock readings were tried here and dropped: one snapshot of them
    read anywhere from the sysfs median down to a tenth of it.)
    """
    import threading

    import torch

    out: dict = {"when": f"{seconds} s of the same launches right after the timed region"}
    ddir = _sysfs_device_dir(dev)
    samples, power = [], []
    stop = threading.Event()

    def sampler():
        while not stop.is_set():
            try:
                v = _read_sclk_mhz(os.path.join(ddir, "pp_dpm_sclk"))
                if v is not None:
                    samples.append(v)
                w = _read_power_w(ddir)
                if w is not None:
                    power.append(w)
            except OSError:
                return
            time.sleep(0.02)

    th = threading.Thread(target=sampler, daemon=True) if ddir else None
    if th:
        th.start()
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _, fn in calls:
            fn()
        torch.cuda.synchronize()
    stop.set()
    if th:
        th.join()
    if samples:
        s = sorted(samples)
        out["sysfs_pp_dpm_sclk_mhz"] = {"median": s[len(s) // 2], "min": s[0], "max": s[-1], "samples": len(s),
                                        "path": os.path.join(ddir, "pp_dpm_sclk")}
    if power:
        p = sorted(power)
        out["board_power_w"] = {"median": round(p[len(p) // 2], 1), "max": round(p[-1], 1)}
    return out


def _batch_us(fn, reps: int) -> float:
    """Device time per call of fn() launched back to back (two events around the batch)."""
    import torch

    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps * 1e3


def _interleaved_us(fns: dict, reps: int, rounds: int) -> dict:
    """Device time per call of each fn, measured in alternating batches (the
    order reversed every round, so no fn always runs first after the others),
    median over the rounds: kernels compared under the same clock and cache
    state."""
    import statistics

    times = {k: [] for k in fns}
    items = list(fns.items())
    for r in range(rounds):
        for k, fn in (items if r % 2 == 0 else items[::-1]):
            times[k].append(_batch_us(fn, reps))
    return {k: statistics.median(v) for k, v in times.items()}


def _host_us(fn, reps: int) -> float:
    """Host (wall) time per call of fn() in a loop that only issues work: the
    device runs behind and is synchronised once, after the loop."""
    import torch

    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        fn()
    t1 = time.perf_counter()
    torch.cuda.synchronize()
    return (t1 - t0) / reps * 1e6


def _cpu_us(fn, reps: int) -> float:
    fn()
    t0 = time.perf_counter()
    for _ in range(reps):
        fn()
    return (time.perf_counter() - t0) / reps * 1e6


def side_ops(qik, wls, dev, with_cpu: bool) -> dict:
    """RMSNorm + RoPE of the 1024px Q and the slab store of the 768px edit prefix."""
    import torch

    out = {}
    g = torch.Generator(device="cuda").manual_seed(77)
    t2i = wls.workload("t2i_1024")
    B, S, H, D = t2i.B, t2i.SQ, t2i.H, t2i.D
    x = torch.randn(B, S, H, D, generator=g, device=dev).to(torch.bfloat16)
    w = torch.randn(D, generator=g, device=dev) * 0.3 + 1.0
    inv = 1.0 / (10000 ** (torch.arange(0, D, 2, device=dev).float() / D))
    ang = torch.outer(torch.arange(S, device=dev).float(), inv)
    freqs = torch.polar(torch.ones_like(ang), ang)
    import ctypes

    from qwen_image_kernel_amd import _lib, fused

    lib = _lib.load()
    stream = torch.cuda.current_stream(dev).cuda_stream
    cos, sin = freqs.real.float().contiguous(), freqs.imag.float().contiguous()
    y = torch.empty_like(x)
    ra = fused.rms_rope_args(x, w, cos, sin, y, 1e-6)
    us = _batch_us(lambda: lib.qik_rms_rope(ctypes.byref(ra), stream), 50)
    api = lambda: qik.fused_rms_norm_rope(x, w, freqs, 1e-6)
    api_us, host_us = _batch_us(api, 50), _host_us(api, 200)
    nbytes = 2 * B * S * H * D * 2 + D * 4 + S * (D // 2) * 8   # x in, out, weight, cos/sin
    entry = {"shape": [B, S, H, D], "kernel": "rms_rope_kernel<128,bf16>", "us": round(us, 2),
             "api_us": round(api_us, 2), "host_us": round(host_us, 2),
             "algorithmic_bytes": nbytes, "gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
             "frac_hbm": round(nbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4)}
    if with_cpu:
        xc, wc, fc = x.cpu(), w.cpu(), freqs.cpu()

        def stock():  # the stock composition (tests/test_fused.py:21-33) in torch on the CPU
            var = xc.float().pow(2).mean(-1, keepdim=True)
            y = (xc * torch.rsqrt(var + 1e-6) * wc).to(xc.dtype)
            r = torch.view_as_complex(y.float().reshape(B, S, H, -1, 2)) * fc.unsqueeze(1)
            return torch.view_as_real(r).flatten(-2).to(xc.dtype)
        entry["cpu_torch_us"] = round(_cpu_us(stock, 3), 1)
        entry["cpu_threads"] = torch.get_num_threads()
    out["rms_rope_t2i_1024_q"] = entry

    ed = wls.workload("edit_768")
    B, P, H, D = ed.B, ed.P, ed.H, ed.D
    k = torch.randn(B, P, H, D, generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn(B, P, H, D, generator=g, device=dev).to(torch.bfloat16)
    cache = qik.ContiguousKVCache(1, B, P + 272, H, D, v_fp8=True, device=dev)
    layer = cache.get_layer(0)
    sa, keep = layer.store_args(k, v, P)
    nws = ctypes.c_int64()
    _lib.check(lib.qik_slab_store_workspace_size(ctypes.byref(sa), ctypes.byref(nws)), "workspace size")
    ws = torch.empty(max(nws.value, 4), dtype=torch.uint8, device=dev)
    us = _batch_us(lambda: lib.qik_slab_store_ws(ctypes.byref(sa), ws.data_ptr(), nws.value, stream), 50)
    us3 = _batch_us(lambda: lib.qik_slab_store(ctypes.byref(sa), stream), 50)
    api = lambda: layer.store(k, v)
    api_us, host_us = _batch_us(api, 50), _host_us(api, 200)
    nbytes = B * P * H * D * (2 + 2 + 2 + 1) + B * H * 4   # k, v in; k bf16, v fp8 out; scales
    entry = {"shape": [B, P, H, D],
             "kernels": "slab_copy_scale_kernel<128> + slab_quant_fp8_kernel<128> (qik_slab_store_ws)",
             "us": round(us, 2), "api_us": round(api_us, 2), "host_us": round(host_us, 2),
             "algorithmic_bytes": nbytes,
             "us_three_launch_form": round(us3, 2),
             "gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
             "frac_hbm": round(nbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4)}
    if with_cpu:
        kc, vc = k.cpu(), v.cpu()
        ccache = qik.ContiguousKVCache(1, B, P + 272, H, D, v_fp8=True, device="cpu")
        entry["cpu_torch_us"] = round(_cpu_us(lambda: ccache.get_layer(0).store(kc, vc), 3), 1)
    out["slab_store_edit_768_prefix"] = entry

    # one attention call at the smallest benchmark shape, where host time shows
    from qwen_image_kernel_amd.attention import make_args

    sm = wls.workload("t2i_512")
    inp = wls.make_inputs(sm, seed=79, device=dev, gen_device="cuda")
    o = torch.empty_like(inp["query"])
    aa = make_args(inp["query"], inp["key"], inp["value"], inp["prefix_lengths"], None, o, None, None, None, False)
    nws = ctypes.c_int64()
    _lib.check(lib.qik_attn_workspace_size(ctypes.byref(aa), ctypes.byref(nws)), "workspace size")
    aws = torch.zeros(max(nws.value, 256), dtype=torch.uint8, device=dev)
    us = _batch_us(lambda: lib.qik_attn_fwd_ws(ctypes.byref(aa), aws.data_ptr(), nws.value, stream), 50)
    api = lambda: qik.block_causal_flash_attention(inp["query"], inp["key"], inp["value"], inp["prefix_lengths"], None)
    api_us, host_us = _batch_us(api, 50), _host_us(api, 200)
    out["attention_t2i_512_call"] = {"shape": [sm.B, sm.SQ, sm.H, sm.D], "kernel": "attn_fwd_kernel (qik_attn_fwd_ws)",
                                     "us": round(us, 2), "api_us": round(api_us, 2),
                                     "host_us": round(host_us, 2),
                                     "tflops": round(sm.flops() / us / 1e6, 1)}
    out.update(fp8_linear_ops(qik, dev, with_cpu))
    return out


def fp8_linear_ops(qik, dev, with_cpu: bool) -> dict:
    """The fp8 GEMM (qik_fp8_gemm) at three projection shapes, with its quantiser."""
    import ctypes

    import torch

    from qwen_image_kernel_amd import _lib
    from qwen_image_kernel_amd import fp8 as f8

    lib = _lib.load()
    stream = torch.cuda.current_stream(dev).cuda_stream
    out = {}
    shapes = [("fp8_linear_1536x4096x4096", 1536, 4096, 4096, "reference test shape (tests/test_fp8.py:16)"),
              ("fp8_linear_4352x9216x3072", 4352, 9216, 3072, "1024px layer, fused QKV (H*D = 3072)"),
              ("fp8_linear_4352x12288x3072", 4352, 12288, 3072, "1024px layer, MLP in (hidden 4*3072)"),
              ("fp8_linear_4352x3072x12288", 4352, 3072, 12288, "1024px layer, MLP out (hidden 4*3072)"),
              ("fp8_linear_256x9216x3072", 256, 9216, 3072, "text stream (256 tokens), fused QKV"),
              ("fp8_linear_256x3072x12288", 256, 3072, 12288, "text stream (256 tokens), MLP out")]
    g = torch.Generator(device="cuda").manual_seed(78)
    for name, M, N, K, what in shapes:
        x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
        lin = torch.nn.Linear(K, N, bias=False, dtype=torch.bfloat16, device=dev)
        with torch.no_grad():
            lin.weight.normal_(0.0, 0.02, generator=g)
        fq = f8.FP8Linear.from_linear(lin)
        xq, sa = f8.quantize_tensorwise(x)
        y = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        a = f8._gemm_args(xq, fq.weight, sa, fq.weight_scale, None, y)
        gneed = ctypes.c_int64(0)
        _lib.check(lib.qik_fp8_gemm_workspace_size(ctypes.byref(a), ctypes.byref(gneed)), "workspace size")
        gws = torch.empty(max(gneed.value // 4, 4), dtype=torch.float32, device=dev)
        fns = {"ours": lambda: lib.qik_fp8_gemm_ws(ctypes.byref(a), gws.data_ptr(), gneed.value, stream)}
        try:
            wt = fq.weight.t()
            torch._scaled_mm(xq, wt, scale_a=sa, scale_b=fq.weight_scale, out_dtype=torch.bfloat16)
            fns["torch"] = lambda: torch._scaled_mm(xq, wt, scale_a=sa, scale_b=fq.weight_scale,
                                                    out_dtype=torch.bfloat16)
            sm_err = None
        except (RuntimeError, NotImplementedError) as e:
            sm_err = f"unavailable: {type(e).__name__}"
        med = _interleaved_us(fns, 10, 6)
        us = med["ours"]
        qa = f8.quant_args(x.reshape(-1), xq, sa, _lib.FP8_ACTIVATION)
        nws = ctypes.c_int64()
        _lib.check(lib.qik_fp8_quant_workspace_size(ctypes.byref(qa), ctypes.byref(nws)), "workspace size")
        qws = torch.zeros(max(nws.value, 4), dtype=torch.uint8, device=dev)  # zero before first use
        q_us = _batch_us(lambda: lib.qik_fp8_quantize(ctypes.byref(qa), qws.data_ptr(), nws.value, stream), 30)
        api_us, host_us = _batch_us(lambda: fq(x), 30), _host_us(lambda: fq(x), 100)
        flops = 2.0 * M * N * K
        kern = ("fp8_gemm_split_kernel + splitk_reduce_kernel (qik_fp8_gemm_ws, K split)" if gneed.value
                else "fp8_gemm_kernel (qik_fp8_gemm_ws)")
        entry = {"shape_mnk": [M, N, K], "what": what, "kernel": kern,
                 "us": round(us, 2), "tflops": round(flops / (us * 1e-6) / 1e12, 1),
                 "frac_fp8_peak": round(flops / (us * 1e-6) / 1e12 / PEAK_FP8_TFLOPS, 4),
                 "quantize_us": round(q_us, 2),
                 "quantize_gbs": round(M * K * 3 / (q_us * 1e-6) / 1e9, 1), "api_us": round(api_us, 2),
                 "host_us": round(host_us, 2)}
        entry["torch_scaled_mm_us"] = round(med["torch"], 2) if sm_err is None else sm_err
        entry["timing"] = "medians of 6 alternating batches of 10 back-to-back launches, ours and torch._scaled_mm"
        if with_cpu and M == 1536:
            xd = (xq.float() * sa).cpu()
            wd = (fq.weight.float() * fq.weight_scale).cpu()
            entry["cpu_fp32_matmul_us"] = round(_cpu_us(lambda: xd @ wd.t(), 2), 1)
            entry["cpu_threads"] = torch.get_num_threads()
        out[name] = entry
        del x, lin, fq, xq, y, gws
    return out


def main():
    args = parse()
    if args.steps < 1:
        print("bench.py: --steps must be at least 1", file=sys.stderr, flush=True)
        sys.exit(2)
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(per-head work shards without communication, but no multi-GPU path is built)",
              file=sys.stderr, flush=True)
        sys.exit(2)

    if args.copy_calibration_mb > 0:
        copy_calibration(args.copy_calibration_mb)
        return
    if args.all_workloads:
        all_workloads(min(args.cpu_seconds, 4.0))
        return
    if args.head_share:
        head_share()
        return

    import torch

    import qwen_image_kernel_amd as qik
    import qwen_image_kernel_amd.workloads as wls

    assert torch.cuda.is_available(), "bench.py needs a HIP device"
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    names = [args.only] if args.only else ["t2i_1024", "edit_768"]

    # ---- inputs resident in HBM, one independent set per layer
    layers = {}
    for name in names:
        wl = wls.workload(name)
        layers[name] = [wls.make_inputs(wl, seed=1000 * (wls.NAMES.index(name) + 1) + i, device=dev,
                                        gen_device="cuda") for i in range(args.layers)]
    torch.cuda.synchronize()

    calls = []  # (name, fn)
    for name in names:
        wl = wls.workload(name)
        for inp in layers[name]:
            def fn(wl=wl, inp=inp):
                return qik.block_causal_flash_attention(
                    inp["query"], inp["key"], inp["value"], inp["prefix_lengths"], None,
                    cache_k=inp["cache_k"], cache_v=inp["cache_v"], cache_v_scale=inp["cache_v_scale"],
                    uniform_full=wl.uniform)
            calls.append((name, fn))
    step_flops = sum(wls.workload(n).flops() for n, _ in calls)

    for _ in range(args.warmup):
        for _, fn in calls:
            fn()
    torch.cuda.synchronize()

    # per-launch events on the stream the kernel runs on (torch's current stream),
    # on the last timed step only: a timed event pair between two launches adds
    # 7-9 us to each launch (measured), which a pipeline without events does not
    # pay, so the other steps run the launches back to back
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in calls]
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    t_start.record()
    for step in range(args.steps - 1):
        for _, fn in calls:
            fn()
    for (name, fn), (e0, e1) in zip(calls, ev):
        e0.record()
        fn()
        e1.record()
    t_end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    total_ms = t_start.elapsed_time(t_end)
    per_kernel_ms = {n: [] for n in names}
    for (name, _), (e0, e1) in zip(calls, ev):
        per_kernel_ms[name].append(e0.elapsed_time(e1))
    ms_per_step = total_ms / args.steps
    value = step_flops / (ms_per_step * 1e-3) / 1e12

    per_workload = {}
    for name in names:
        wl = wls.workload(name)
        ts = sorted(per_kernel_ms[name])
        avg = sum(ts) / len(ts)
        per_workload[name] = {
            "tflops": round(wl.flops() / (avg * 1e-3) / 1e12, 2),
            "pct_bf16_peak": round(100 * wl.flops() / (avg * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 2),
            "kernel_avg_us": round(avg * 1e3, 2),
            "kernel_median_us": round(ts[len(ts) // 2] * 1e3, 2),
            "launches": len(ts),
            "unmasked_gflop_per_layer": round(wl.flops() / 1e9, 3),
            "min_hbm_mb_per_layer": round(wl.min_bytes() / 1e6, 2),
            "min_hbm_gbs": round(wl.min_bytes() / (avg * 1e-3) / 1e9, 1),
        }
    dom = max(names, key=lambda n: per_workload[n]["kernel_avg_us"] * per_workload[n]["launches"])
    dwl = wls.workload(dom)
    achieved = dwl.flops() / (per_workload[dom]["kernel_avg_us"] * 1e-6) / 1e12

    clock = clock_under_load(calls, dev, args.clock_seconds) if args.clock_seconds > 0 else None
    del layers, calls
    sops = side_ops(qik, wls, dev, with_cpu=args.cpu_seconds > 0)

    cpu = None
    if args.cpu_seconds > 0:
        cpu = cpu_baseline(wls, args.cpu_seconds)

    line = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: N(0,1) fp32 cast to bf16, slab V quantised to fp8e4m3fn per (b,h) (amax/448)",
        "config": {
            "workload": (f"{args.layers} layers x " + " + ".join(names) + " (D=128, H=24, B=1)"),
            "t2i_1024": "SQ=SN=4352 (text 256 causal + image 4096 block), fresh K/V, ragged L",
            "edit_768": "SQ=4096 target, slab P=2560 (bf16 K, fp8 V, capacity P+272) + fresh SN=4096, uniform L",
            "layers_per_shape": args.layers,
        },
        "pct_bf16_peak": round(100 * value / PEAK_BF16_TFLOPS, 2),
        "roofline": {
            "bound": "mfma",
            "kernel": f"attn_fwd_kernel ({dom})",
            "launch": ("qik_attn_fwd_ws: one workgroup per resident slot (2 per CU) pulling row "
                       "blocks from per-XCD queues; the last partial round's row blocks split in two "
                       "pieces (7/10 and 3/10 of their KV tiles) merged through the workspace"),
            "achieved": round(achieved, 2),
            "launch_timing": "HIP events around each launch of the last timed step, on the launch stream",
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
            "traffic": profiled_traffic(dom),
            "traffic_source": "profiles/attn_fwd_traffic.txt (rocprofv3 FETCH_SIZE/WRITE_SIZE, copy-calibrated)",
            "algorithmic_flops_per_launch": dwl.flops(),
            "compulsory_bytes_per_launch": dwl.min_bytes(),
        },
        "per_workload": per_workload,
        "gpu_clock": clock,
        "side_ops": sops,
        "cpu_baseline": cpu,
        "wall_s_timed": round(wall, 3),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
