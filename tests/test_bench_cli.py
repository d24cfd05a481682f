"""bench.py's contract paths that need no GPU: the one-GPU refusal, argument
checks, the committed traffic summary it reads for roofline.traffic, and the
sysfs clock parser."""

import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def _run(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True, text=True,
                          timeout=120, cwd=ROOT)


@pytest.mark.parametrize("n", [2, 8])
def test_more_than_one_gpu_exits_with_a_message(n):
    r = _run("--gpus", str(n))
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_steps_must_be_positive():
    r = _run("--steps", "0")
    assert r.returncode == 2 and "--steps" in r.stderr


def test_traffic_summary_has_both_shapes():
    for name in ("t2i_1024", "edit_768"):
        b = bench.profiled_traffic(name)
        assert isinstance(b, int) and 100e6 < b < 400e6, (name, b)
    assert bench.profiled_traffic("no_such_shape") is None


def test_sclk_parser(tmp_path):
    f = tmp_path / "pp_dpm_sclk"
    f.write_text("0: 500Mhz\n1: 1912Mhz *\n2: 2400Mhz\n")
    assert bench._read_sclk_mhz(str(f)) == 1912.0
    f.write_text("0: 500Mhz\n1: 2400Mhz\n")
    assert bench._read_sclk_mhz(str(f)) is None
