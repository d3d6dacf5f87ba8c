"""Host-side pieces of bench.py's output contract (no GPU needed): the
refusal of more than one GPU, the per-frame spread statistics and the host
CPU description that accompanies the CPU baseline."""

import importlib.util
import os
import pathlib
import subprocess
import sys

import numpy as np

REPO = pathlib.Path(__file__).resolve().parents[1]


def _bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", REPO / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(REPO / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode != 0
    assert r.stdout == ""  # no JSON line
    assert "--gpus 2 is not supported" in r.stderr


def test_spread_is_median_and_deciles():
    b = _bench()
    ms = np.array([0.50, 0.52, 0.51, 0.90, 0.53, 0.49, 0.50, 0.51, 0.52, 0.50], dtype=np.float32)
    st = b.spread(ms)
    assert st["frames"] == 10
    assert st["p10"] <= st["median"] <= st["p90"]
    # Sorted: 0.49 0.50 0.50 0.50 0.51 0.51 0.52 0.52 0.53 0.90 (linear interpolation).
    assert abs(st["median"] - 0.51) < 1e-6
    assert abs(st["p10"] - (0.49 + 0.9 * 0.01)) < 1e-6
    assert abs(st["p90"] - (0.53 + 0.1 * 0.37)) < 1e-6
    assert b.spread([0.7])["median"] == b.spread([0.7])["p90"]


def test_host_cpu_description():
    h = _bench().host_cpu()
    assert set(h) == {"cpu_model", "hardware_concurrency", "usable_threads"}
    assert h["hardware_concurrency"] == os.cpu_count()
    assert 1 <= h["usable_threads"] <= h["hardware_concurrency"]
    assert isinstance(h["cpu_model"], str) and h["cpu_model"]
