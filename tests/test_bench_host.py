"""bench.py's host-side arithmetic and contract, on the CPU (nothing here
touches a GPU).

The expected figures are the per-config costs the benchmark contract quotes
(one triangle-attention direction at N=512: F = 1.119e11 flop, B = 2.02e8
bytes, T* = 44.8 us; one triangle-multiplication direction at N=768:
F = 2.319e11, B = 4.55e8, T* = 92.8 us; one PairformerLayer at N=1024: T* =
1.13 ms), so a changed coefficient in the bench's formulas fails here."""

import importlib.util
import json
import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_triangle_module_costs_match_the_contract(bench):
    f, b = bench.tri_module_cost("triattn", 512)
    assert f == pytest.approx(1.119e11, rel=1e-3) and b == pytest.approx(2.02e8, rel=1e-2)
    assert bench.t_star_ms(f, b) * 1e3 == pytest.approx(44.8, rel=1e-2)  # MFMA-bound
    f, b = bench.tri_module_cost("trimul", 768)
    assert f == pytest.approx(2.319e11, rel=1e-3) and b == pytest.approx(4.55e8, rel=1e-2)
    assert bench.t_star_ms(f, b) * 1e3 == pytest.approx(92.8, rel=1e-2)


def test_kernel_flops_per_launch(bench):
    table = bench.kernel_table(1024)
    assert table["trimul_contract"][0] == pytest.approx(2.75e11, rel=1e-2)  # 2 * 128 * N^3
    assert table["triattn_core"][0] == pytest.approx(5.50e11, rel=1e-2)  # 4 * H * d * N^3
    # one layer: 2 x tri-mult + 2 x tri-att + transition + sequence stack = 2.831e12 flop, T* 1.13 ms
    layer = 2 * sum(bench.tri_module_cost(k, 1024)[0] for k in ("trimul", "triattn"))
    layer += table["pair_transition"][0] + 1.10e10
    assert layer == pytest.approx(2.831e12, rel=1e-2)
    assert bench.t_star_ms(2.831e12, 0) == pytest.approx(1.13, rel=1e-2)


def test_roofline_bound_is_the_larger_time(bench):
    mfma = bench.roofline_of(2.5e12, 1e6, 2.0)  # 1 ms of flops, 0.125 us of bytes
    assert mfma["bound"] == "mfma" and mfma["unit"] == "TFLOP/s" and mfma["frac"] == pytest.approx(0.5)
    hbm = bench.roofline_of(1e9, 8e9, 2.0)  # 0.4 us of flops, 1 ms of bytes
    assert hbm["bound"] == "hbm" and hbm["unit"] == "GB/s" and hbm["frac"] == pytest.approx(0.5)


def test_measured_traffic_comes_from_the_committed_counters(bench):
    data = json.loads((ROOT / "profiles" / "hbm_traffic_n1024.json").read_text())
    assert bench.measured_traffic("triattn_core", 1024) == data["bytes_per_launch"]["triattn_core"]
    assert bench.measured_traffic("triattn_core", 512) is None  # taken at N=1024 only


def test_more_than_one_gpu_exits_with_a_message():
    env = dict(os.environ, HIP_VISIBLE_DEVICES="", CUDA_VISIBLE_DEVICES="")
    proc = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                          env=env, timeout=120)
    assert proc.returncode == 2
    assert "one GPU" in json.loads(proc.stdout.strip().splitlines()[-1])["error"]
