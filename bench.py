"""Benchmark of the FP16 conv-graph path on one MI355X.

Workload: the MLVC-shaped synthetic per-frame graph at 1920x1088
("mlvc_1920x1088": frame unshuffle, 4-level strided analysis to 1/16 with
C 64->128->192->256, 12 depthwise-separable residual blocks, shuffle
upsampling synthesis, 64-channel recurrent reference carried between
frames), FP16 storage with FP32 accumulation, seeded random-init weights,
synthetic U[0,1] frame. One step = one frame = one hipGraph replay with the
input already resident in HBM and the recurrent state carried on device.

Prints one JSON line with frames/s (value), aggregate conv TFLOP/s and its
fraction of the 2.5 PFLOP/s dense FP16 MFMA peak, the roofline position of
the dominant kernel (timed live with HIP events on the backend stream) and
the CPU oracle's frames/s on a bounded sample of the same workload. A
per-kernel table goes to stderr.
"""

from __future__ import annotations

import argparse
import json
import os
import pathlib
import sys
import tempfile
import time

REPO = pathlib.Path(__file__).resolve().parent
sys.path[:0] = [str(REPO / "mlvc.cpp_amd" / "python"), str(REPO / "oracle")]

CONFIG = "mlvc_1920x1088"
PEAK_MFMA_TFLOPS = 2500.0  # dense FP16 MFMA, MI355X
PEAK_HBM_GBS = 8000.0      # HBM3E
RIDGE = PEAK_MFMA_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def kernel_table(gpu, reps: int):
    rows = []
    for l in gpu.launches():
        ms = gpu.time_launch(l["index"], reps)
        ai = l["flops"] / l["bytes"] if l["bytes"] else 0.0
        bound = "mfma" if ai >= RIDGE else "hbm"
        t = ms * 1e-3
        tflops = l["flops"] / t / 1e12 if l["flops"] else 0.0
        gbs = l["bytes"] / t / 1e9
        frac = tflops / PEAK_MFMA_TFLOPS if bound == "mfma" else gbs / PEAK_HBM_GBS
        rows.append(dict(l, ms=ms, ai=ai, bound=bound, tflops=tflops, gbs=gbs, frac=frac))
    return rows


def cpu_baseline(model_dir, bindings, shape, budget_s: float):
    import mlvc_hip
    import mlvc_oracle

    plan = mlvc_oracle.OraclePlan(model_dir, CONFIG, bindings)
    plan.reset_state()
    x0 = mlvc_hip.synth_input(CONFIG, 0, 0, shape)
    plan.run([x0])  # warm-up frame (first-touch of buffers)
    frames, t0 = 0, time.perf_counter()
    while True:
        plan.run([mlvc_hip.synth_input(CONFIG, 0, frames + 1, shape)])
        frames += 1
        el = time.perf_counter() - t0
        if el >= budget_s or frames >= 64:
            break
    return {"value": frames / el, "unit": "frames/s", "cores": plan.threads, "kind": "port",
            "sample": f"{frames} consecutive frames of {CONFIG} (recurrent state carried) after 1 warm-up frame, "
                      f"{el:.1f} s wall, oracle AVX2+FMA+F16C path, {plan.threads} threads"}


PMC_REPS = 10
CALIB_BYTES = 128 << 20  # calibration stream kernel: reads and writes this many bytes


def pmc_pass(indices) -> int:
    """Dispatches for rocprofv3 --pmc: the calibration stream kernel (FP16
    LeakyReLU over CALIB_BYTES, so FETCH_SIZE and WRITE_SIZE each have a
    known algorithmic value) and then the chosen launches of the graph. Their
    per-dispatch counters, scaled by calibration, give HBM bytes per launch."""
    import ctypes as C

    import mlvc_hip

    dev = mlvc_hip.device_lib()
    dev.mlvc_hip_malloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
    dev.mlvc_hip_free.argtypes = [C.c_void_p]
    dev.mlvc_hip_zero.argtypes = [C.c_void_p, C.c_size_t, C.c_void_p]
    dev.mlvc_hip_leaky_relu.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_float, C.c_void_p]
    dev.mlvc_hip_stream_synchronize.argtypes = [C.c_void_p]
    bufs = [C.c_void_p(), C.c_void_p()]
    for b in bufs:
        if dev.mlvc_hip_malloc(C.byref(b), CALIB_BYTES) != 0:
            raise mlvc_hip.MlvcError(dev.mlvc_hip_last_error().decode())
    if dev.mlvc_hip_zero(bufs[0], CALIB_BYTES, None) != 0:
        raise mlvc_hip.MlvcError(dev.mlvc_hip_last_error().decode())
    for _ in range(PMC_REPS):
        if dev.mlvc_hip_leaky_relu(bufs[0], bufs[1], CALIB_BYTES // 2, 0.1, None) != 0:
            raise mlvc_hip.MlvcError(dev.mlvc_hip_last_error().decode())
    dev.mlvc_hip_stream_synchronize(None)
    for b in bufs:
        dev.mlvc_hip_free(b)
    with tempfile.TemporaryDirectory() as d:
        mlvc_hip.synth_write(CONFIG, d, 0)
        bindings, _ = mlvc_hip.synth_bindings(CONFIG)
        gpu = mlvc_hip.Backend(d, "hip", device_id=0)
        gpu.load(CONFIG, bindings)
        gpu.upload_inputs([mlvc_hip.synth_input(CONFIG, 0, 0, gpu.in_shapes[0])])
        gpu.reset_state()
        gpu.time_frames(1)
        launches = gpu.launches()
        for i in indices:
            log(f"pmc launch {i}: {launches[i]['name']} [{launches[i]['kind']}] x{PMC_REPS + 1}")
            gpu.time_launch(i, PMC_REPS)
        gpu.close()
    log(f"pmc calibration: {PMC_REPS} x leaky_relu over {CALIB_BYTES} bytes")
    return 0


def measured_traffic(path, launch_name, kind):
    """HBM bytes per launch (FETCH_SIZE + WRITE_SIZE, calibrated) for the
    launch `launch_name` run by kernel variant `kind`, from a committed
    rocprofv3 --pmc summary; None when no entry was measured on that variant."""
    try:
        for line in pathlib.Path(path).read_text().splitlines():
            f = line.split()
            if len(f) == 5 and f[0] == "traffic:" and f[1] == launch_name and f[2] == kind:
                return float(f[3]) + float(f[4])
    except OSError:
        pass
    return None


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--kernel-reps", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--api-frames", type=int, default=30,
                    help="frames timed through run() (host frame in, host reconstruction out)")
    ap.add_argument("--pmc-pass", default=None, metavar="I,J,...",
                    help="counter-collection mode for rocprofv3 --pmc: run the calibration stream kernel, then "
                         "launches I,J,... of the graph, PMC_REPS times each; no timing, no JSON line")
    ap.add_argument("--traffic", default=str(REPO / "profiles" / "hbm_traffic_1920x1088.md"),
                    help="PMC summary holding 'traffic: <launch> <variant> <fetch bytes> <write bytes>' lines")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: the per-frame schedule is a serial chain linked by the recurrent "
              f"state, so it is not split across GPUs (independent streams or GOPs would go one per GPU); "
              f"--gpus {args.gpus} is not supported", file=sys.stderr)
        return 2
    rank = int(os.environ.get("RANK", "0"))

    import mlvc_hip

    if args.pmc_pass is not None:
        return pmc_pass([int(i) for i in args.pmc_pass.split(",") if i])

    with tempfile.TemporaryDirectory() as d:
        mlvc_hip.synth_write(CONFIG, d, 0)
        bindings, _ = mlvc_hip.synth_bindings(CONFIG)
        gpu = mlvc_hip.Backend(d, "hip", device_id=0)
        gpu.load(CONFIG, bindings)
        shape = gpu.in_shapes[0]
        gpu.upload_inputs([mlvc_hip.synth_input(CONFIG, 0, 0, shape)])
        gpu.reset_state()
        gpu.time_frames(args.warmup)
        # Timed region: K frames replayed back to back; the call synchronises
        # on an event recorded after the last frame.
        t0 = time.perf_counter()
        gpu_ms = gpu.time_frames(args.steps)
        wall = time.perf_counter() - t0
        fps = args.steps / wall
        launches = gpu.launches()
        conv_flops = sum(l["flops"] for l in launches)
        frame_bytes = sum(l["bytes"] for l in launches)
        rows = kernel_table(gpu, args.kernel_reps)
        dom = max(rows, key=lambda r: r["ms"])
        dom_t = dom["ms"] * 1e-3
        if dom["bound"] == "mfma":
            roof = {"bound": "mfma", "achieved": dom["flops"] / dom_t / 1e12, "peak": PEAK_MFMA_TFLOPS,
                    "unit": "TFLOP/s"}
        else:
            roof = {"bound": "hbm", "achieved": dom["bytes"] / dom_t / 1e9, "peak": PEAK_HBM_GBS, "unit": "GB/s"}
        roof["frac"] = roof["achieved"] / roof["peak"]
        roof["traffic"] = measured_traffic(args.traffic, dom["name"], dom["kind"])
        roof["kernel"] = f"{dom['name']} [{dom['kind']}]"
        roof["kernel_ms"] = dom["ms"]
        log(f"{'#':>3} {'launch':28} {'kernel':48} {'us':>9} {'TFLOP/s':>8} {'GB/s':>8} {'AI':>7} bound frac")
        for r in rows:
            log(f"{r['index']:3d} {r['name'][:28]:28} {r['kind'][:48]:48} {r['ms']*1e3:9.1f} {r['tflops']:8.1f} "
                f"{r['gbs']:8.0f} {r['ai']:7.1f} {r['bound']:5} {r['frac']:.3f}")
        sum_kernel_ms = sum(r["ms"] for r in rows)
        log(f"sum of isolated kernel times {sum_kernel_ms:.3f} ms/frame; graph replay {gpu_ms / args.steps:.3f} ms/frame "
            f"(events), {wall * 1e3 / args.steps:.3f} ms/frame (wall); {conv_flops / 1e9:.1f} GFLOP and "
            f"{frame_bytes / 1e6:.0f} MB algorithmic per frame")
        # Through the plain run() API instead: the frame is copied in from
        # host memory and the reconstruction copied back every frame (pinned
        # staging, PCIe). Reported beside the value, never as it.
        x0 = mlvc_hip.synth_input(CONFIG, 0, 0, shape)
        gpu.run([x0])
        t1 = time.perf_counter()
        for _ in range(args.api_frames):
            gpu.run([x0])
        api_fps = args.api_frames / (time.perf_counter() - t1)
        base = None
        if not args.no_cpu_baseline and rank == 0:
            base = cpu_baseline(d, bindings, shape, args.cpu_seconds)
        gpu.close()

    conv_tflops = conv_flops * fps / 1e12
    line = {
        "metric": "conv-graph frames/s @1920x1088 + FP16 conv TFLOP/s (% MFMA peak), 1 GPU",
        "value": fps,
        "unit": "frames/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": wall * 1e3 / args.steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {"workload": f"{CONFIG}: MLVC-shaped synthetic per-frame conv graph, 1x3x1088x1920 frame, "
                               f"analysis to 1/16 (C 64-128-192-256), 12 depthwise-separable residual blocks, "
                               f"shuffle synthesis, 64-ch recurrent reference at 544x960",
                   "frames_per_step": 1, "gflop_per_frame": conv_flops / 1e9,
                   "algorithmic_mb_per_frame": frame_bytes / 1e6, "kernels_per_frame": len(launches)},
        "conv_tflops": conv_tflops,
        "conv_mfma_peak_frac": conv_tflops / PEAK_MFMA_TFLOPS,
        "gpu_event_ms_per_step": gpu_ms / args.steps,
        "run_api_frames_per_s": api_fps,
        "roofline": roof,
        "cpu_baseline": base,
    }
    if rank == 0:
        print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
