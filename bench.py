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
the CPU oracle's frames/s on a bounded sample of the same workload, and the
codec I/O measurements around the encoder / decoder graphs (conversion
kernels at 1080p, buffered end-to-end frames/s) and the real-model operator
kernels (fused ReGLU, feature update, quantisation tails, GATHER, ...)
against the HBM roofline, and launch by launch the single 3x3 conv, the
conv sweep and the two residual-block workloads against their summed
per-kernel roofline. A per-kernel table goes to stderr.
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


def kernel_table(gpu, reps: int, cold_reps: int = 0):
    """Per launch: mean of `reps` back-to-back launches (warm: inputs and
    weights stay in L2 / MALL between repeats) and, with cold_reps > 0, the
    median of `cold_reps` single launches each after a cache-evicting copy
    (cold: everything comes from HBM)."""
    import numpy as np

    rows = []
    for l in gpu.launches():
        ms = gpu.time_launch(l["index"], reps)
        ai = l["flops"] / l["bytes"] if l["bytes"] else 0.0
        bound = "mfma" if ai >= RIDGE else "hbm"

        def rates(ms):
            t = ms * 1e-3
            tflops = l["flops"] / t / 1e12 if l["flops"] else 0.0
            gbs = l["bytes"] / t / 1e9
            return tflops, gbs, tflops / PEAK_MFMA_TFLOPS if bound == "mfma" else gbs / PEAK_HBM_GBS

        tflops, gbs, frac = rates(ms)
        row = dict(l, ms=ms, ai=ai, bound=bound, tflops=tflops, gbs=gbs, frac=frac)
        if cold_reps > 0:
            cold = float(np.median(gpu.time_launch_cold(l["index"], cold_reps, COLD_FLUSH_BYTES)))
            row.update(cold_ms=cold, cold_frac=rates(cold)[2])
        rows.append(row)
    return rows


CODEC_SHAPE = (1920, 1080, 1920, 1088)  # 1080p I420 frame into the 1920x1088 model image


def codec_io_kernels(reps: int) -> dict:
    """Device-resident timing of the two codec I/O conversion kernels at the
    1080p frame / 1920x1088 model shape (HIP events on one stream around
    `reps` back-to-back launches). Algorithmic bytes: each tensor once (frame
    bytes, FP16 model image; the frame side reads only the active area)."""
    import ctypes as C

    import numpy as np

    import mlvc_hip

    L = mlvc_hip.device_lib()
    L.mlvc_hip_malloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
    L.mlvc_hip_free.argtypes = [C.c_void_p]
    L.mlvc_hip_memcpy_h2d.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]
    L.mlvc_hip_stream_create.argtypes = [C.POINTER(C.c_void_p)]
    L.mlvc_hip_stream_destroy.argtypes = [C.c_void_p]
    L.mlvc_hip_stream_synchronize.argtypes = [C.c_void_p]
    L.mlvc_hip_event_create.argtypes = [C.POINTER(C.c_void_p)]
    L.mlvc_hip_event_destroy.argtypes = [C.c_void_p]
    L.mlvc_hip_event_record.argtypes = [C.c_void_p, C.c_void_p]
    L.mlvc_hip_event_synchronize.argtypes = [C.c_void_p]
    L.mlvc_hip_event_elapsed_ms.argtypes = [C.c_void_p, C.c_void_p, C.POINTER(C.c_float)]
    L.mlvc_hip_yuv420_to_model.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p] + [C.c_int] * 5 + [C.c_void_p]
    L.mlvc_hip_model_to_yuv420.argtypes = [C.c_void_p, C.c_void_p] + [C.c_int] * 7 + [C.c_float, C.c_void_p]

    def ok(rc):
        if rc != 0:
            raise mlvc_hip.MlvcError(L.mlvc_hip_last_error().decode())

    w, h, mw, mh = CODEC_SHAPE
    frame_bytes = w * h * 3 // 2
    image_bytes = 3 * mw * mh * 2
    rng = np.random.default_rng(0)
    frame = rng.integers(0, 256, frame_bytes, dtype=np.uint8)
    lut = (np.arange(256, dtype=np.float32) / np.float32(255.0)).astype(np.float16).view(np.uint16)
    bufs = []

    def put(a):
        p = C.c_void_p()
        ok(L.mlvc_hip_malloc(C.byref(p), a.nbytes))
        ok(L.mlvc_hip_memcpy_h2d(p, a.ctypes.data, a.nbytes, None))
        bufs.append(p)
        return p

    src, table = put(frame), put(lut)
    image = C.c_void_p()
    out = C.c_void_p()
    ok(L.mlvc_hip_malloc(C.byref(image), image_bytes))
    ok(L.mlvc_hip_malloc(C.byref(out), frame_bytes))
    bufs += [image, out]
    s, e0, e1 = C.c_void_p(), C.c_void_p(), C.c_void_p()
    ok(L.mlvc_hip_stream_create(C.byref(s)))
    ok(L.mlvc_hip_event_create(C.byref(e0)))
    ok(L.mlvc_hip_event_create(C.byref(e1)))
    ok(L.mlvc_hip_stream_synchronize(None))

    def timed(launch):
        for _ in range(3):
            launch()
        ok(L.mlvc_hip_event_record(e0, s))
        for _ in range(reps):
            launch()
        ok(L.mlvc_hip_event_record(e1, s))
        ok(L.mlvc_hip_event_synchronize(e1))
        ms = C.c_float()
        ok(L.mlvc_hip_event_elapsed_ms(e0, e1, C.byref(ms)))
        return ms.value / reps * 1e3

    to_model_us = timed(lambda: ok(L.mlvc_hip_yuv420_to_model(src, table, image, w, h, mw, mh, 0, s)))
    to_frame_us = timed(lambda: ok(L.mlvc_hip_model_to_yuv420(image, out, w, h, mw, mh, 0, 0, 0, 1.0, s)))
    for p in bufs:
        L.mlvc_hip_free(p)
    L.mlvc_hip_event_destroy(e0)
    L.mlvc_hip_event_destroy(e1)
    L.mlvc_hip_stream_destroy(s)
    to_model_b = frame_bytes + image_bytes
    to_frame_b = 3 * w * h * 2 + frame_bytes
    return {"shape": f"{w}x{h} I420 frame <-> 1x3x{mh}x{mw} FP16 model image",
            "frame_to_model_us": to_model_us, "frame_to_model_gbs": to_model_b / to_model_us / 1e3,
            "frame_to_model_hbm_frac": to_model_b / to_model_us / 1e3 / PEAK_HBM_GBS,
            "model_to_frame_us": to_frame_us, "model_to_frame_gbs": to_frame_b / to_frame_us / 1e3,
            "model_to_frame_hbm_frac": to_frame_b / to_frame_us / 1e3 / PEAK_HBM_GBS,
            "algorithmic_bytes": {"frame_to_model": to_model_b, "model_to_frame": to_frame_b}}


# Standalone bandwidth kernels at the residual-block workload's shapes (C128
# at 92x160, C256 at 46x80: depthwise 3x3, the 3x3 conv C->4C's pixel
# shuffle, the pixel unshuffle before a 1x1 conv) and at the 1920x1088
# graph's shuffle shapes: (name, op, (n, c, h, w) input).
STANDALONE = [
    ("dw3x3_c128_92x160", "depthwise", (1, 128, 92, 160)),
    ("dw3x3_c256_46x80", "depthwise", (1, 256, 46, 80)),
    ("d2s2_c512_92x160", "depth_to_space", (1, 512, 92, 160)),
    ("d2s2_c1024_46x80", "depth_to_space", (1, 1024, 46, 80)),
    ("s2d2_c128_92x160", "space_to_depth", (1, 128, 92, 160)),
    ("s2d2_c256_46x80", "space_to_depth", (1, 256, 46, 80)),
    ("dw3x3_c256_68x120", "depthwise", (1, 256, 68, 120)),
    ("d2s2_c256_272x480", "depth_to_space", (1, 256, 272, 480)),
    ("d2s2_c12_544x960", "depth_to_space", (1, 12, 544, 960)),
    ("s2d2_c3_1088x1920", "space_to_depth", (1, 3, 1088, 1920)),
]


def standalone_kernels(reps: int, cold_reps: int) -> dict:
    """Device-resident timing of the standalone depthwise / DEPTH_TO_SPACE /
    SPACE_TO_DEPTH kernels through the device C ABI, at STANDALONE's shapes.
    Warm: HIP events around `reps` back-to-back launches (operands stay in
    L2 / MALL when they fit). Cold: per launch, a 512 MiB device copy evicts
    L2 and the MALL outside the events, then events around the one launch
    (median of `cold_reps`; includes the dispatch latency a lone launch
    pays). Algorithmic bytes: input and output once (plus the depthwise
    weights and bias). Beside each kernel, the same two timings of a device
    copy of its input into its output (the runtime's copy kernel, the same
    bytes less the depthwise taps): the floor a launch of that size sees."""
    import ctypes as C

    import numpy as np

    import mlvc_hip

    L = mlvc_hip.device_lib()
    vp, ci = C.c_void_p, C.c_int
    L.mlvc_hip_malloc.argtypes = [C.POINTER(vp), C.c_size_t]
    L.mlvc_hip_free.argtypes = [vp]
    L.mlvc_hip_memcpy_h2d.argtypes = [vp, vp, C.c_size_t, vp]
    L.mlvc_hip_memcpy_d2d.argtypes = [vp, vp, C.c_size_t, vp]
    L.mlvc_hip_stream_create.argtypes = [C.POINTER(vp)]
    L.mlvc_hip_stream_destroy.argtypes = [vp]
    L.mlvc_hip_stream_synchronize.argtypes = [vp]
    L.mlvc_hip_event_create.argtypes = [C.POINTER(vp)]
    L.mlvc_hip_event_destroy.argtypes = [vp]
    L.mlvc_hip_event_record.argtypes = [vp, vp]
    L.mlvc_hip_event_synchronize.argtypes = [vp]
    L.mlvc_hip_event_elapsed_ms.argtypes = [vp, vp, C.POINTER(C.c_float)]
    L.mlvc_hip_depthwise.argtypes = [vp, vp, vp, vp] + [ci] * 12 + [vp]
    L.mlvc_hip_depth_to_space.argtypes = [vp, vp] + [ci] * 5 + [vp]
    L.mlvc_hip_space_to_depth.argtypes = [vp, vp] + [ci] * 5 + [vp]

    def ok(rc):
        if rc != 0:
            raise mlvc_hip.MlvcError(L.mlvc_hip_last_error().decode())

    bufs = []

    def alloc(nbytes):
        p = vp()
        ok(L.mlvc_hip_malloc(C.byref(p), max(nbytes, 16)))
        bufs.append(p)
        return p

    def put(a):
        p = alloc(a.nbytes)
        ok(L.mlvc_hip_memcpy_h2d(p, a.ctypes.data, a.nbytes, None))
        return p

    rng = np.random.default_rng(3)
    s, e0, e1 = vp(), vp(), vp()
    ok(L.mlvc_hip_stream_create(C.byref(s)))
    ok(L.mlvc_hip_event_create(C.byref(e0)))
    ok(L.mlvc_hip_event_create(C.byref(e1)))
    flush = alloc(COLD_FLUSH_BYTES)
    half = COLD_FLUSH_BYTES // 2

    def elapsed_us():
        ok(L.mlvc_hip_event_synchronize(e1))
        ms = C.c_float()
        ok(L.mlvc_hip_event_elapsed_ms(e0, e1, C.byref(ms)))
        return ms.value * 1e3

    def timed_warm_cold(launch):
        cold = []
        for _ in range(cold_reps):
            ok(L.mlvc_hip_memcpy_d2d(vp(flush.value + half), flush, half, s))
            ok(L.mlvc_hip_event_record(e0, s))
            launch()
            ok(L.mlvc_hip_event_record(e1, s))
            cold.append(elapsed_us())
        for _ in range(3):
            launch()
        ok(L.mlvc_hip_event_record(e0, s))
        for _ in range(reps):
            launch()
        ok(L.mlvc_hip_event_record(e1, s))
        return elapsed_us() / reps, float(np.median(cold)) if cold else None

    rows = []
    try:
        for name, op, (n, c, h, w) in STANDALONE:
            elems = n * c * h * w
            x = put(rng.uniform(-1, 1, elems).astype(np.float16).view(np.uint16))
            y = alloc(elems * 2)
            nbytes = 4 * elems
            if op == "depthwise":
                wt = put(rng.normal(0, 1 / 3, c * 9).astype(np.float16).view(np.uint16))
                bias = put(rng.normal(0, 0.01, c).astype(np.float32))
                nbytes += c * 9 * 2 + c * 4
                launch = lambda: ok(L.mlvc_hip_depthwise(x, wt, bias, y, n, c, h, w, h, w, 3, 3, 1, 1, 1, 1, s))
            elif op == "depth_to_space":
                launch = lambda: ok(L.mlvc_hip_depth_to_space(x, y, n, c, h, w, 2, s))
            else:
                launch = lambda: ok(L.mlvc_hip_space_to_depth(x, y, n, c, h, w, 2, s))
            copy = lambda: ok(L.mlvc_hip_memcpy_d2d(y, x, elems * 2, s))
            ok(L.mlvc_hip_stream_synchronize(None))
            warm_us, cold_us = timed_warm_cold(launch)
            copy_warm_us, copy_cold_us = timed_warm_cold(copy)
            rows.append({"name": name, "op": op, "shape": [n, c, h, w], "algorithmic_bytes": nbytes,
                         "warm_us": warm_us, "warm_gbs": nbytes / warm_us / 1e3,
                         "warm_hbm_frac": nbytes / warm_us / 1e3 / PEAK_HBM_GBS,
                         "cold_us": cold_us, "cold_gbs": nbytes / cold_us / 1e3 if cold_us else None,
                         "cold_hbm_frac": nbytes / cold_us / 1e3 / PEAK_HBM_GBS if cold_us else None,
                         "copy_warm_us": copy_warm_us, "copy_cold_us": copy_cold_us})
    finally:
        ok(L.mlvc_hip_stream_synchronize(s))
        for p in bufs:
            L.mlvc_hip_free(p)
        L.mlvc_hip_event_destroy(e0)
        L.mlvc_hip_event_destroy(e1)
        L.mlvc_hip_stream_destroy(s)
    return {"kernels": rows, "cold_flush_bytes": COLD_FLUSH_BYTES,
            "workload": "standalone depthwise 3x3 / block-2 DEPTH_TO_SPACE / SPACE_TO_DEPTH at the residual-block "
                        "shapes (C128 @92x160, C256 @46x80 and their 4C shuffles) and the 1920x1088 graph's shuffle "
                        "shapes; warm = back-to-back launches, cold = one launch after a cache-evicting copy"}


def log_standalone(res: dict) -> None:
    for k in res["kernels"]:
        cold = (f"cold {k['cold_us']:7.1f} us {k['cold_gbs']:6.0f} GB/s {k['cold_hbm_frac']:.3f}"
                if k["cold_us"] is not None else "")
        copy = (f"  copy warm {k['copy_warm_us']:6.1f} cold {k['copy_cold_us']:6.1f} us"
                if k["copy_cold_us"] is not None else f"  copy warm {k['copy_warm_us']:6.1f} us")
        log(f"standalone {k['name']:20} {k['algorithmic_bytes'] / 1e6:8.2f} MB  warm {k['warm_us']:7.1f} us "
            f"{k['warm_gbs']:6.0f} GB/s {k['warm_hbm_frac']:.3f}  {cold}{copy}")


def codec_buffered(frames: int) -> dict:
    """End to end through BufferedCodecBackend at the 1080p frame shape: two
    slots in flight, each submit uploading a pinned frame (encoder) or latent
    (decoder), converting, replaying the frame graph and downloading the
    latent (encoder) or frame (decoder). PCIe-inclusive; host time per frame."""
    import numpy as np

    import mlvc_hip

    w, h, mw, mh = CODEC_SHAPE
    res = {}
    with tempfile.TemporaryDirectory() as d:
        mlvc_hip.synth_write("codec_enc_1920x1088", d, 0)
        mlvc_hip.synth_write("codec_dec_1920x1088", d, 0)
        bindings, _ = mlvc_hip.synth_bindings("codec_enc_1920x1088")
        rng = np.random.default_rng(1)
        frame = rng.integers(0, 256, w * h * 3 // 2, dtype=np.uint8)
        for model in ("MLVCEncoder", "MLVCDecoder"):
            b = mlvc_hip.Backend(d, "hip")
            b.load(model, bindings)
            b.configure_codec_io(w, h, mw, mh, 1.0, slots=2)
            b.reset_state()
            enc = model == "MLVCEncoder"

            def submit(slot):
                if enc:
                    b.encoder_input_yuv(slot)[:] = frame
                    b.submit_encoder(slot, 5)
                else:
                    b.submit_decoder(slot, 5)

            for i in range(4):  # warm-up
                submit(i % 2)
                b.wait_codec_slot(i % 2)
            t0 = time.perf_counter()
            for i in range(frames):
                slot = i % 2
                b.wait_codec_slot(slot)
                submit(slot)
            b.wait_codec_slot(0)
            b.wait_codec_slot(1)
            res[("encoder" if enc else "decoder") + "_frames_per_s"] = frames / (time.perf_counter() - t0)
            b.close()
    res["workload"] = "codec_enc/dec_1920x1088 (MLVCEncoder / MLVCDecoder pair), 1920x1080 I420 frames, 2 slots"
    return res


REALOPS = "realops_544x960"
REALOPS_KINDS = ("y0_tail", "y1_tail", "feature_update", "feature_update_outputs", "reglu", "gather", "slice", "concat",
                 "clip", "sigmoid", "reciprocal", "round", "add", "sub", "mul")


def realops(reps: int, frames: int) -> dict:
    """The real-model operators at the recurrent feature's resolution
    (realops_544x960: ReGLU FFN, q-index GATHER scaling, feature update with
    the 64-channel state at 544x960, standalone ReGLU, deferred-CONCAT
    feature update, y0/y1 quantisation tails with Q=96 at 272x480): frames/s
    of the whole graph (hipGraph replay, inputs resident) and each
    non-conv kernel's algorithmic bytes against the HBM roofline."""
    import numpy as np

    import mlvc_hip

    with tempfile.TemporaryDirectory() as d:
        mlvc_hip.synth_write(REALOPS, d, 0)
        bindings, _ = mlvc_hip.synth_bindings(REALOPS)
        gpu = mlvc_hip.Backend(d, "hip", device_id=0)
        gpu.load(REALOPS, bindings)
        x = mlvc_hip.synth_input(REALOPS, 0, 0, gpu.in_shapes[0])
        gpu.upload_inputs([x, np.array([5], np.int32)])
        gpu.reset_state()
        gpu.time_frames(10)
        ms = gpu.time_frames(frames)
        kernels = []
        for r in kernel_table(gpu, reps):
            if r["kind"] not in REALOPS_KINDS:
                continue
            kernels.append({"launch": r["name"], "kind": r["kind"], "us": r["ms"] * 1e3, "algorithmic_bytes": r["bytes"],
                            "gbs": r["gbs"], "hbm_frac": r["gbs"] / PEAK_HBM_GBS})
        n_launch = len(gpu.launches())
        gpu.close()
    for k in kernels:
        log(f"realops {k['kind']:24} {k['launch'][:24]:24} {k['us']:8.1f} us {k['gbs']:7.0f} GB/s {k['hbm_frac']:.3f}")
    return {"workload": f"{REALOPS}: ReGLU FFN, q-index GATHER, feature update (C=64 at 544x960, both forms), "
                        f"y0/y1 quantisation tails (Q=96 at 272x480) around 1x1/3x3 convs",
            "frames_per_s": frames / (ms * 1e-3), "kernels_per_frame": n_launch, "kernels": kernels}


def ops_kernels(reps: int) -> dict:
    """The real-model operator kernels of realops_544x960 launched straight
    through the device C ABI, without the graph, the backend or a hipGraph
    (so a profiler sees plain kernel dispatches): ReGLU 128->64, ADD, MUL by a
    [1,32,1,1] row, channel SLICE and both feature-update forms at 544x960;
    the y0 / y1 quantisation tails at Q=96, 272x480. Random FP16 operands in
    each kernel's working range; HIP events around `reps` back-to-back
    launches after 3 warm-up launches. Algorithmic bytes: every operand read
    and every result written once."""
    import ctypes as C

    import numpy as np

    import mlvc_hip

    L = mlvc_hip.device_lib()
    vp, ci, sz, i64p = C.c_void_p, C.c_int, C.c_size_t, C.POINTER(C.c_int64)
    L.mlvc_hip_malloc.argtypes = [C.POINTER(vp), sz]
    L.mlvc_hip_free.argtypes = [vp]
    L.mlvc_hip_memcpy_h2d.argtypes = [vp, vp, sz, vp]
    L.mlvc_hip_stream_create.argtypes = [C.POINTER(vp)]
    L.mlvc_hip_stream_destroy.argtypes = [vp]
    L.mlvc_hip_stream_synchronize.argtypes = [vp]
    L.mlvc_hip_event_create.argtypes = [C.POINTER(vp)]
    L.mlvc_hip_event_destroy.argtypes = [vp]
    L.mlvc_hip_event_record.argtypes = [vp, vp]
    L.mlvc_hip_event_synchronize.argtypes = [vp]
    L.mlvc_hip_event_elapsed_ms.argtypes = [vp, vp, C.POINTER(C.c_float)]
    L.mlvc_hip_binary.argtypes = [vp, i64p, vp, i64p, vp, i64p, ci, vp]
    L.mlvc_hip_slice.argtypes = [vp, i64p, vp, i64p, i64p, i64p, vp]
    L.mlvc_hip_reglu.argtypes = [vp, vp, ci, ci, sz, C.c_float, C.c_float, vp]
    L.mlvc_hip_prepare_tables.argtypes = [vp]
    L.mlvc_hip_feature_update.argtypes = [vp] * 6 + [ci, ci, sz, vp]
    L.mlvc_hip_y0_tail.argtypes = [vp, vp]
    L.mlvc_hip_y1_tail.argtypes = [vp, vp]

    class Y0(C.Structure):
        _fields_ = [(f, vp) for f in ("latent", "prior", "quant_scale", "update_scale0", "update_scale1", "normalized",
                                      "clipped", "y_raw", "concat2", "concat3")] + \
                   [("n", ci), ("q", ci), ("hw", sz), ("clip_min", C.c_float)]

    class Y1(C.Structure):
        _fields_ = [(f, vp) for f in ("normalized", "prior", "quant_scale", "update_scale0", "update_scale1", "concat2",
                                      "clipped", "y_raw", "out")] + [("n", ci), ("q", ci), ("hw", sz)]

    def ok(rc):
        if rc != 0:
            raise mlvc_hip.MlvcError(L.mlvc_hip_last_error().decode())

    bufs = []

    def alloc(elems):
        p = vp()
        ok(L.mlvc_hip_malloc(C.byref(p), max(2 * elems, 16)))
        bufs.append(p)
        return p

    rng = np.random.default_rng(5)

    def put(c, hw, lo=-2.0, hi=2.0):
        a = rng.uniform(lo, hi, c * hw).astype(np.float16).view(np.uint16)
        p = alloc(a.size)
        ok(L.mlvc_hip_memcpy_h2d(p, a.ctypes.data, a.nbytes, None))
        return p

    def dims(*d):
        return (C.c_int64 * 4)(*d)

    h, w, ch, q = 544, 960, 64, 96
    hw, hw2 = h * w, (h // 2) * (w // 2)
    s, e0, e1 = vp(), vp(), vp()
    ok(L.mlvc_hip_stream_create(C.byref(s)))
    ok(L.mlvc_hip_event_create(C.byref(e0)))
    ok(L.mlvc_hip_event_create(C.byref(e1)))
    rows = []
    try:
        ok(L.mlvc_hip_prepare_tables(s))
        cases = []
        # ReGLU of the graph's 1x1 conv output: [1,128,hw] -> [1,64,hw].
        x, y = put(2 * ch, hw, -3, 8), alloc(ch * hw)
        cases.append(("reglu_c128_544x960", "reglu", 3 * ch * hw * 2,
                      lambda x=x, y=y: ok(L.mlvc_hip_reglu(x, y, 1, ch, hw, -1.0, 6.0, s))))
        # The FFN residual ADD and the q-row MUL on 32 channels.
        a, b, y = put(32, hw), put(32, hw), alloc(32 * hw)
        dd = dims(1, 32, h, w)
        cases.append(("add_c32_544x960", "binary", 3 * 32 * hw * 2,
                      lambda a=a, b=b, y=y, dd=dd: ok(L.mlvc_hip_binary(a, dd, b, dd, y, dd, 0, s))))
        row, dr = put(32, 1, 0.5, 1.5), dims(1, 32, 1, 1)
        cases.append(("mul_row_c32_544x960", "binary", 2 * 32 * hw * 2 + 32 * 2,
                      lambda a=a, row=row, y=y, dd=dd, dr=dr: ok(L.mlvc_hip_binary(a, dd, row, dr, y, dd, 2, s))))
        # Channels 0..31 of the 64-channel state.
        st = put(ch, hw)
        dx, dy, st0, st1 = dims(1, ch, h, w), dims(1, ch // 2, h, w), dims(0, 0, 0, 0), dims(1, 1, 1, 1)
        cases.append(("slice_c64_to_32_544x960", "slice", 2 * (ch // 2) * hw * 2,
                      lambda st=st, y=y: ok(L.mlvc_hip_slice(st, dx, y, dy, st0, st1, s))))
        # Feature update: x [1,3C,hw], history [1,C,hw], scale [C] ->
        # feature [1,2C,hw] (C = 64), and the deferred form with scaled and
        # blended also written (C = 32).
        fx, fh, fs, ff = put(3 * ch, hw, -6, 6), put(ch, hw), put(ch, 1, 0.5, 1.5), alloc(2 * ch * hw)
        cases.append(("feature_update_c64_544x960", "feature_update", (3 * ch + ch + 2 * ch) * hw * 2 + ch * 2,
                      lambda: ok(L.mlvc_hip_feature_update(fx, fh, fs, ff, None, None, 1, ch, hw, s))))
        c2 = ch // 2
        gx, gh, gs = put(3 * c2, hw, -6, 6), put(c2, hw), put(c2, 1, 0.5, 1.5)
        gf, gsc, gbl = alloc(2 * c2 * hw), alloc(c2 * hw), alloc(c2 * hw)
        cases.append(("feature_update_outputs_c32_544x960", "feature_update_outputs",
                      (3 * c2 + c2 + 4 * c2) * hw * 2 + c2 * 2,
                      lambda: ok(L.mlvc_hip_feature_update(gx, gh, gs, gf, gsc, gbl, 1, c2, hw, s))))
        # Quantisation tails at half resolution, Q = 96.
        y0 = Y0(put(2 * q, hw2, -20, 20).value,
                put(4 * q, hw2, -0.5, 3).value, put(2 * q, hw2, 0.5, 2).value, put(q, hw2, 0.5, 1.5).value,
                put(q, hw2, 0.5, 1.5).value, alloc(2 * q * hw2).value, alloc(2 * q * hw2).value,
                alloc(q * hw2).value, alloc(2 * q * hw2).value, alloc(6 * q * hw2).value, 1, q, hw2, 0.11)
        cases.append(("y0_tail_q96_272x480", "y0_tail", 23 * q * hw2 * 2,
                      lambda: ok(L.mlvc_hip_y0_tail(C.byref(y0), s))))
        y1 = Y1(y0.normalized, put(2 * q, hw2, -4, 4).value, y0.quant_scale, y0.update_scale0, y0.update_scale1,
                y0.concat2, y0.clipped, alloc(q * hw2).value, alloc(2 * q * hw2).value, 1, q, hw2)
        cases.append(("y1_tail_q96_272x480", "y1_tail", 15 * q * hw2 * 2,
                      lambda: ok(L.mlvc_hip_y1_tail(C.byref(y1), s))))
        ok(L.mlvc_hip_stream_synchronize(None))
        for name, kind, nbytes, launch in cases:
            for _ in range(3):
                launch()
            ok(L.mlvc_hip_event_record(e0, s))
            for _ in range(reps):
                launch()
            ok(L.mlvc_hip_event_record(e1, s))
            ok(L.mlvc_hip_event_synchronize(e1))
            ms = C.c_float()
            ok(L.mlvc_hip_event_elapsed_ms(e0, e1, C.byref(ms)))
            us = ms.value * 1e3 / reps
            rows.append({"name": name, "kind": kind, "us": us, "algorithmic_bytes": nbytes,
                         "gbs": nbytes / us / 1e3, "hbm_frac": nbytes / us / 1e3 / PEAK_HBM_GBS})
            log(f"ops {name:36} {nbytes / 1e6:8.2f} MB {us:8.2f} us {nbytes / us / 1e3:7.0f} GB/s "
                f"{nbytes / us / 1e3 / PEAK_HBM_GBS:.3f} ({reps + 3} launches)")
    finally:
        ok(L.mlvc_hip_stream_synchronize(s))
        for p in bufs:
            L.mlvc_hip_free(p)
        L.mlvc_hip_event_destroy(e0)
        L.mlvc_hip_event_destroy(e1)
        L.mlvc_hip_stream_destroy(s)
    return {"workload": "realops_544x960's operator kernels through the device C ABI (no graph): ReGLU, ADD, "
                        "row MUL, SLICE, feature update (C=64, and C=32 with 3 outputs) at 544x960; y0/y1 tails "
                        "(Q=96) at 272x480",
            "kernels": rows}


# The smaller workloads, each timed launch by launch beside its summed
# per-kernel roofline time (min over MFMA and HBM peaks of each launch's
# algorithmic FLOPs and bytes): (label, synthetic graph, what it is).
SMALL_CONFIGS = [
    ("single_conv", "conv3x3_184x320", "3x3 conv 64->64 @184x320 + bias + LeakyReLU(0.01)"),
    ("conv_sweep", "conv_sweep_640x368", "1x1 and 3x3 convs at 184x320/C64, 92x160/C128, 46x80/C256 and the "
                                         "stride-2 3x3 convs between the levels"),
    ("dwblock_92x160_c128", "dwblock_92x160_c128", "depthwise-separable residual block, unshuffle(2)->1x1 4C->C and "
                                                    "3x3 C->4C->shuffle(2) at 92x160, C=128"),
    ("dwblock_46x80_c256", "dwblock_46x80_c256", "the same at 46x80, C=256"),
]


def small_configs(reps: int, cold_reps: int, frames: int) -> dict:
    """Per launch of each SMALL_CONFIGS graph: warm (mean of `reps`
    back-to-back launches) and cold (median of `cold_reps` single launches
    after a cache-evicting copy) time, TFLOP/s, GB/s, roofline bound and
    fraction; per graph: the hipGraph replay time per pass (events around
    `frames` replays) against the summed per-launch roofline time."""
    import mlvc_hip

    out = {}
    for label, config, what in SMALL_CONFIGS:
        with tempfile.TemporaryDirectory() as d:
            mlvc_hip.synth_write(config, d, 0)
            bindings, _ = mlvc_hip.synth_bindings(config)
            gpu = mlvc_hip.Backend(d, "hip", device_id=0)
            gpu.load(config, bindings)
            gpu.upload_inputs([mlvc_hip.synth_input(config, i, 0, s) for i, s in enumerate(gpu.in_shapes)])
            if bindings:
                gpu.reset_state()
            gpu.time_frames(10)
            replay_us = gpu.time_frames(frames) / frames * 1e3
            rows = kernel_table(gpu, reps, cold_reps)
            gpu.close()
        launches, roof_us = [], 0.0
        for r in rows:
            r_us = max(r["flops"] / (PEAK_MFMA_TFLOPS * 1e12), r["bytes"] / (PEAK_HBM_GBS * 1e9)) * 1e6
            roof_us += r_us
            launches.append({"name": r["name"], "kernel": r["kind"], "gflop": r["flops"] / 1e9,
                             "algorithmic_mb": r["bytes"] / 1e6, "us": r["ms"] * 1e3, "tflops": r["tflops"],
                             "gbs": r["gbs"], "bound": r["bound"], "frac": r["frac"], "roofline_us": r_us,
                             **({"cold_us": r["cold_ms"] * 1e3, "cold_frac": r["cold_frac"]} if "cold_ms" in r else {})})
            log(f"{label:20} {r['name'][:22]:22} {r['kind'][:46]:46} {r['ms'] * 1e3:7.1f} us {r['tflops']:7.1f} TFLOP/s "
                f"{r['gbs']:6.0f} GB/s {r['bound']} {r['frac']:.3f}"
                + (f"  cold {r['cold_ms'] * 1e3:6.1f} us {r['cold_frac']:.3f}" if "cold_ms" in r else ""))
        sum_us = sum(l["us"] for l in launches)
        log(f"{label:20} replay {replay_us:.1f} us per pass, sum of launches {sum_us:.1f} us, summed roofline "
            f"{roof_us:.2f} us ({roof_us / sum_us:.3f} of the launches' time)")
        out[label] = {"graph": config, "workload": what, "replay_us": replay_us, "sum_launch_us": sum_us,
                      "roofline_us": roof_us, "roofline_frac": roof_us / sum_us, "launches": launches}
    return out


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
    return {"value": frames / el, "unit": "frames/s", "cores": plan.threads, "kind": "port", **host_cpu(),
            "sample": f"{frames} consecutive frames of {CONFIG} (recurrent state carried) after 1 warm-up frame, "
                      f"{el:.1f} s wall, oracle AVX2+FMA+F16C path, {plan.threads} threads"}


COLD_FLUSH_BYTES = 512 << 20


def spread(ms) -> dict:
    """Median and 10th/90th percentiles of per-frame times (ms)."""
    import numpy as np

    q = np.percentile(np.asarray(ms, dtype=np.float64), [50, 10, 90])
    return {"median": float(q[0]), "p10": float(q[1]), "p90": float(q[2]), "frames": len(ms)}


def host_cpu() -> dict:
    """CPU model, hardware thread count and the threads this process may use."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "hardware_concurrency": os.cpu_count(),
            "usable_threads": len(os.sched_getaffinity(0))}


PMC_REPS = 10
CALIB_BYTES = 128 << 20  # calibration stream kernel: reads and writes this many bytes


def calibration_stream() -> None:
    """PMC_REPS dispatches of the calibration stream kernel: FP16 LeakyReLU
    over CALIB_BYTES, so FETCH_SIZE and WRITE_SIZE each have a known
    algorithmic value that scales the counters of the kernels after it."""
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
    log(f"pmc calibration: {PMC_REPS} x leaky_relu over {CALIB_BYTES} bytes")


def pmc_pass(indices) -> int:
    """Dispatches for rocprofv3 --pmc: the calibration stream kernel and then
    the chosen launches of the graph. Their per-dispatch counters, scaled by
    calibration, give HBM bytes per launch."""
    import mlvc_hip

    calibration_stream()
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
    return 0


def measured_traffic(path, launch_names, kind):
    """HBM bytes per launch (FETCH_SIZE + WRITE_SIZE, calibrated) for a launch
    among `launch_names` (launches of one variant on one shape) run by kernel
    variant `kind`, from a committed rocprofv3 --pmc summary; None when no
    entry was measured on that variant."""
    try:
        for line in pathlib.Path(path).read_text().splitlines():
            f = line.split()
            if len(f) == 5 and f[0] == "traffic:" and f[1] in launch_names and base_kind(f[2]) == base_kind(kind):
                return float(f[3]) + float(f[4])
    except OSError:
        pass
    return None


def base_kind(kind: str) -> str:
    """A launch's kernel variant without the activation-layout tags of chained
    fused blocks (+nhwc_in, +nhwc_out: the same kernel and work, its input or
    output handed over channel-last)."""
    return kind.replace("+nhwc_in", "").replace("+nhwc_out", "")


def group_launches(rows):
    """Launches of one kernel variant on one shape (same kind up to layout
    tags, FLOPs and bytes) merged: mean time per launch, number of launches
    and their summed time, largest summed time first."""
    groups = {}
    for r in rows:
        key = (base_kind(r["kind"]), r["flops"], r["bytes"])
        g = groups.setdefault(key, dict(r, kind=key[0], launches=0, total_ms=0.0, names=[]))
        g["launches"] += 1
        g["total_ms"] += r["ms"]
        g["names"].append(r["name"])
        if "cold_ms" in r:
            g.setdefault("_cold", []).append(r["cold_ms"])
    out = []
    for g in groups.values():
        g["ms"] = g["total_ms"] / g["launches"]
        if "_cold" in g:
            g["cold_ms"] = sum(g["_cold"]) / len(g["_cold"])
            del g["_cold"]
        out.append(g)
    return sorted(out, key=lambda g: -g["total_ms"])


def roofline_of(groups, traffic_path) -> dict:
    """Roofline object of the first group: achieved algorithmic TFLOP/s
    (MFMA-bound) or GB/s (HBM-bound) of one launch over its mean duration."""
    dom = groups[0]
    t = dom["ms"] * 1e-3
    if dom["bound"] == "mfma":
        roof = {"bound": "mfma", "achieved": dom["flops"] / t / 1e12, "peak": PEAK_MFMA_TFLOPS, "unit": "TFLOP/s"}
    else:
        roof = {"bound": "hbm", "achieved": dom["bytes"] / t / 1e9, "peak": PEAK_HBM_GBS, "unit": "GB/s"}
    roof["frac"] = roof["achieved"] / roof["peak"]
    names = dom["names"] or [dom["name"]]
    roof["traffic"] = measured_traffic(traffic_path, names, dom["kind"])
    roof["kernel"] = f"{names[0]} [{dom['kind']}]" if len(names) == 1 else \
        f"{names[0]}..{names[-1]} ({len(names)} launches) [{dom['kind']}]"
    roof["kernel_ms"] = dom["ms"]
    roof["launches_per_frame"] = dom["launches"]
    if "total_ms" in dom:
        roof["frame_share"] = dom["total_ms"] / sum(g["total_ms"] for g in groups)
    if "cold_ms" in dom:
        roof["kernel_cold_ms"] = dom["cold_ms"]
        cold_t = dom["cold_ms"] * 1e-3
        roof["frac_cold"] = (dom["flops"] / cold_t / 1e12 / PEAK_MFMA_TFLOPS if dom["bound"] == "mfma"
                             else dom["bytes"] / cold_t / 1e9 / PEAK_HBM_GBS)
    roof["algorithmic_per_launch"] = {"flops": dom["flops"], "bytes": dom["bytes"]}
    return roof


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--kernel-reps", type=int, default=20)
    ap.add_argument("--launch-cold-reps", type=int, default=5,
                    help="single launches per kernel timed after a cache-evicting copy (0: skip)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-codec", action="store_true", help="skip the codec I/O measurements")
    ap.add_argument("--codec-frames", type=int, default=60)
    ap.add_argument("--no-realops", action="store_true", help="skip the real-model operator measurements")
    ap.add_argument("--realops-frames", type=int, default=50)
    ap.add_argument("--no-standalone", action="store_true",
                    help="skip the standalone depthwise / pixel-shuffle measurements")
    ap.add_argument("--standalone-only", action="store_true",
                    help="run only the standalone kernel measurements (for a kernel trace of them); no JSON line")
    ap.add_argument("--standalone-cold", type=int, default=20, help="cold launches timed per standalone kernel")
    ap.add_argument("--no-small-configs", action="store_true",
                    help="skip the single-conv, conv-sweep and residual-block workloads")
    ap.add_argument("--small-configs-only", action="store_true",
                    help="run only the single-conv, conv-sweep and residual-block workloads; no JSON line")
    ap.add_argument("--small-frames", type=int, default=100, help="graph replays timed per small workload")
    ap.add_argument("--codec-only", action="store_true",
                    help="run only the codec I/O conversion kernels (after the calibration stream kernel, for "
                         "rocprofv3 kernel traces and counter passes); no JSON line")
    ap.add_argument("--ops-only", action="store_true",
                    help="run only the real-model operator kernels through the device C ABI, no graph (after the "
                         "calibration stream kernel, for rocprofv3 kernel traces and counter passes); no JSON line")
    ap.add_argument("--cold-frames", type=int, default=50,
                    help="frames timed with L2 and MALL flushed before each (0: skip)")
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
    # Conv tile choices recorded on an MI355X (written by the backend's tuner
    # under MLVC_HIP_TUNE_FILE): the benchmark, its kernel trace and its
    # counter passes then run the same kernels.
    tuning = REPO / "mlvc.cpp_amd" / "tuning" / "mi355x.txt"
    if tuning.exists():
        os.environ.setdefault("MLVC_HIP_TUNE_FILE", str(tuning))

    import mlvc_hip

    if args.pmc_pass is not None:
        return pmc_pass([int(i) for i in args.pmc_pass.split(",") if i])
    if args.standalone_only:
        log_standalone(standalone_kernels(args.kernel_reps, args.standalone_cold))
        return 0
    if args.small_configs_only:
        small_configs(args.kernel_reps, args.launch_cold_reps, args.small_frames)
        return 0
    if args.ops_only:
        calibration_stream()
        ops_kernels(args.kernel_reps)
        return 0
    if args.codec_only:
        calibration_stream()
        c = codec_io_kernels(args.kernel_reps)
        log(f"codec I/O: frame->model {c['frame_to_model_us']:.2f} us ({c['frame_to_model_gbs']:.0f} GB/s), "
            f"model->frame {c['model_to_frame_us']:.2f} us ({c['model_to_frame_gbs']:.0f} GB/s), "
            f"{args.kernel_reps + 3} launches each")
        return 0

    with tempfile.TemporaryDirectory() as d:
        mlvc_hip.synth_write(CONFIG, d, 0)
        bindings, _ = mlvc_hip.synth_bindings(CONFIG)
        gpu = mlvc_hip.Backend(d, "hip", device_id=0)
        gpu.load(CONFIG, bindings)
        shape = gpu.in_shapes[0]
        gpu.upload_inputs([mlvc_hip.synth_input(CONFIG, 0, 0, shape)])
        gpu.reset_state()
        gpu.time_frames(args.warmup)
        # Right after load() the GPU is still raising its clocks (per-frame
        # times settle after about 30 frames), so the other measurements come
        # first: cold frames (a 512 MiB device copy before each frame,
        # outside its events, evicts L2, 4 MB per XCD, and the 256 MB MALL;
        # the clock ramp can only make them read slower), the per-launch
        # table and the per-frame spread (events around every frame of a
        # back-to-back run). Then the state is reset and the W warm-up frames
        # run again right before the K timed ones.
        cold = gpu.time_frames_each(args.cold_frames, COLD_FLUSH_BYTES) if args.cold_frames > 0 else None
        rows = kernel_table(gpu, args.kernel_reps, args.launch_cold_reps)
        each = gpu.time_frames_each(args.steps)
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
        frame_ms = spread(each)
        cold_ms = dict(spread(cold), flush_bytes=COLD_FLUSH_BYTES) if cold is not None else None
        log(f"per frame: median {frame_ms['median']:.3f} ms (p10 {frame_ms['p10']:.3f}, p90 {frame_ms['p90']:.3f})"
            + (f"; cold (L2 + MALL flushed) median {cold_ms['median']:.3f} ms (p10 {cold_ms['p10']:.3f}, "
               f"p90 {cold_ms['p90']:.3f})" if cold_ms else ""))
        # The dominant kernel is the one with the largest share of the frame:
        # launches of one kernel variant on one shape (the 12 fused residual
        # blocks) count together. The longest single launch goes beside it.
        roof = roofline_of(group_launches(rows), args.traffic)
        longest = roofline_of([dict(max(rows, key=lambda r: r["ms"]), launches=1, names=None)], args.traffic)
        roof["longest_launch"] = {k: longest[k] for k in ("kernel", "kernel_ms", "bound", "achieved", "unit", "frac",
                                                          "traffic", "kernel_cold_ms", "frac_cold") if k in longest}
        log(f"{'#':>3} {'launch':28} {'kernel':48} {'us':>9} {'TFLOP/s':>8} {'GB/s':>8} {'AI':>7} bound frac"
            + ("  cold us  frac" if args.launch_cold_reps > 0 else ""))
        for r in rows:
            log(f"{r['index']:3d} {r['name'][:28]:28} {r['kind'][:48]:48} {r['ms']*1e3:9.1f} {r['tflops']:8.1f} "
                f"{r['gbs']:8.0f} {r['ai']:7.1f} {r['bound']:5} {r['frac']:.3f}"
                + (f" {r['cold_ms']*1e3:8.1f} {r['cold_frac']:.3f}" if "cold_ms" in r else ""))
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
    codec = None
    if not args.no_codec:
        codec = codec_io_kernels(args.kernel_reps)
        codec.update(codec_buffered(args.codec_frames))
        log(f"codec I/O: frame->model {codec['frame_to_model_us']:.1f} us ({codec['frame_to_model_gbs']:.0f} GB/s), "
            f"model->frame {codec['model_to_frame_us']:.1f} us ({codec['model_to_frame_gbs']:.0f} GB/s); buffered "
            f"encoder {codec['encoder_frames_per_s']:.0f} frames/s, decoder {codec['decoder_frames_per_s']:.0f} frames/s")

    alone = None
    if not args.no_standalone:
        alone = standalone_kernels(args.kernel_reps, args.standalone_cold)
        log_standalone(alone)

    ops = None
    if not args.no_realops:
        ops = realops(args.kernel_reps, args.realops_frames)
        log(f"realops: {ops['frames_per_s']:.0f} frames/s, {ops['kernels_per_frame']} kernels/frame")

    small = None
    if not args.no_small_configs:
        small = small_configs(args.kernel_reps, args.launch_cold_reps, args.small_frames)

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
        "frame_ms": frame_ms,
        "cold_frame_ms": cold_ms,
        "run_api_frames_per_s": api_fps,
        "roofline": roof,
        "launches": [{"name": r["name"], "kernel": r["kind"], "us": r["ms"] * 1e3, "bound": r["bound"], "frac": r["frac"],
                      **({"cold_us": r["cold_ms"] * 1e3, "cold_frac": r["cold_frac"]} if "cold_ms" in r else {})}
                     for r in rows],
        "cpu_baseline": base,
        "codec_io": codec,
        "realops": ops,
        "standalone": alone,
        "small_configs": small,
    }
    if rank == 0:
        print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
