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


def _row(index, name, kind, flops, nbytes, ms, bound="mfma", cold=None):
    r = {"index": index, "name": name, "kind": kind, "flops": flops, "bytes": nbytes, "ms": ms, "bound": bound}
    if cold is not None:
        r["cold_ms"] = cold
    return r


def test_dominant_kernel_is_the_largest_share_of_the_frame(tmp_path):
    """Twelve 12 us launches of one variant outweigh one 80 us launch: the
    roofline object names the group, with its per-launch fraction, and keeps
    the longest single launch beside it."""
    b = _bench()
    rows = [_row(0, "n5", "pair", 1e9, 1.4e8, 0.040, "hbm", 0.05),
            _row(1, "n78", "ws_a", 77e9, 1e8, 0.080, cold=0.088)]
    rows += [_row(2 + i, f"n{12 + 5 * i}_dw+block", "dwblock", 4.32e9, 8.9e6, 0.012 + 0.001 * (i % 2), cold=0.018)
             for i in range(12)]
    # Same kind at another shape is another group.
    rows.append(_row(14, "n99", "dwblock", 1e9, 2e6, 0.004))
    traffic = tmp_path / "t.md"
    traffic.write_text("traffic: n12_dw+block dwblock 10000000 5000000\ntraffic: n78 ws_a 1 2\n")
    groups = b.group_launches(rows)
    assert [g["launches"] for g in groups[:2]] == [12, 1]
    roof = b.roofline_of(groups, str(traffic))
    assert roof["launches_per_frame"] == 12
    assert abs(roof["kernel_ms"] - 0.0125) < 1e-12
    assert abs(roof["achieved"] - 4.32e9 / 0.0125e-3 / 1e12) < 1e-6
    assert abs(roof["frac"] - roof["achieved"] / 2500.0) < 1e-12
    assert roof["traffic"] == 15000000.0  # measured on n12, the same variant and shape
    assert abs(roof["frame_share"] - 0.150 / (0.150 + 0.080 + 0.040 + 0.004)) < 1e-12
    assert abs(roof["frac_cold"] - 4.32e9 / 0.018e-3 / 1e12 / 2500.0) < 1e-12
    assert "12 launches" in roof["kernel"]
    longest = b.roofline_of([dict(max(rows, key=lambda r: r["ms"]), launches=1, names=None)], str(traffic))
    assert longest["kernel"] == "n78 [ws_a]" and longest["traffic"] == 3.0
    # An HBM-bound group is priced in GB/s.
    hbm = b.roofline_of([dict(rows[0], launches=1, names=None)], str(traffic))
    assert hbm["unit"] == "GB/s" and abs(hbm["achieved"] - 1.4e8 / 0.040e-3 / 1e9) < 1e-6
    assert hbm["traffic"] is None
