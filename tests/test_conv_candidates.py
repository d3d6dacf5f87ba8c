"""Host-side tile-variant eligibility of the conv entry points (no device
work: mlvc_hip_conv_candidates only inspects the geometry).

The weight-streaming 3x3 variants stage 16-byte row segments through buffer
loads whose offsets must stay below 2^31 (up to one pass of channel planes
past the last one); mlvc_hip_conv_launch refuses them otherwise. So a
geometry whose planes are too large must not list them as candidates: the
load-time tuner would time a variant that cannot launch, and a recorded
tuning-file choice keyed by launch name (not resolution) could name one.
"""

import ctypes as C
import pathlib

import mlvc_hip


class ConvDesc(C.Structure):
    _fields_ = [(f, C.c_int) for f in ("n", "ic", "ih", "iw", "oc", "oh", "ow", "kh", "kw", "stride_h", "stride_w",
                                       "pad_h", "pad_w")] + [
        ("x", C.c_void_p), ("x2", C.c_void_p), ("ic_split", C.c_int), ("in_s2d_block", C.c_int),
        ("packed_w", C.c_void_p), ("bias", C.c_void_p), ("epilogue", C.c_int), ("alpha", C.c_float),
        ("clip_lo", C.c_float), ("clip_hi", C.c_float), ("residual", C.c_void_p), ("y", C.c_void_p),
        ("out_d2s_block", C.c_int), ("variant", C.c_int), ("vector_io", C.c_int), ("ksplit", C.c_int),
        ("split_c", C.c_int), ("workspace", C.c_void_p), ("workspace_bytes", C.c_size_t), ("in_nhwc", C.c_int),
        ("out_nhwc", C.c_int)]


def candidates(ic, h, w, oc, k=3, stride=1, pad=1, d2s=0, desc=None):
    lib = mlvc_hip.device_lib()
    oh = (h + 2 * pad - k) // stride + 1
    ow = (w + 2 * pad - k) // stride + 1
    d = desc or ConvDesc(n=1, ic=ic, ih=h, iw=w, oc=oc, oh=oh, ow=ow, kh=k, kw=k, stride_h=stride, stride_w=stride,
                         pad_h=pad, pad_w=pad, ic_split=0, in_s2d_block=0, epilogue=1, alpha=0.01, out_d2s_block=d2s)
    buf = (C.c_int * 512)()
    count = C.c_int()
    lib.mlvc_hip_conv_candidates.argtypes = [C.POINTER(ConvDesc), C.POINTER(C.c_int), C.c_int, C.POINTER(C.c_int)]
    lib.mlvc_hip_conv_variant_name.restype = C.c_char_p
    assert lib.mlvc_hip_conv_candidates(C.byref(d), buf, 512, C.byref(count)) == 0, lib.mlvc_hip_last_error()
    assert count.value <= 512
    return [lib.mlvc_hip_conv_variant_name(buf[i]).decode() for i in range(count.value)]


def test_weight_streaming_variants_listed_for_ordinary_planes():
    names = candidates(128, 64, 64, 256, d2s=2)
    assert any(n.startswith("ws_") for n in names), names
    assert any(n.startswith("ws_") for n in candidates(192, 136, 240, 256, stride=2))


def test_no_weight_streaming_variant_when_row_offsets_reach_2_31():
    # 128 channels of 2048 x 4096 FP16 planes (16 MiB each): 128 planes plus
    # one 16- or 32-channel pass is past 2^31 bytes.
    names = candidates(128, 2048, 4096, 64)
    assert names, "the other 3x3 variants still run the geometry"
    assert not [n for n in names if n.startswith("ws_")], names
    # Stride 2 as well.
    names = candidates(128, 2048, 4096, 64, stride=2)
    assert names and not [n for n in names if n.startswith("ws_")], names


def plan(ic, h, w, oc, k=3, stride=1, pad=1, n=1, epilogue=1):
    lib = mlvc_hip.device_lib()
    oh = (h + 2 * pad - k) // stride + 1
    ow = (w + 2 * pad - k) // stride + 1
    d = ConvDesc(n=n, ic=ic, ih=h, iw=w, oc=oc, oh=oh, ow=ow, kh=k, kw=k, stride_h=stride, stride_w=stride,
                 pad_h=pad, pad_w=pad, epilogue=epilogue, alpha=0.01)
    lib.mlvc_hip_conv_plan.argtypes = [C.POINTER(ConvDesc)]
    lib.mlvc_hip_conv_workspace_bytes.argtypes = [C.POINTER(ConvDesc)]
    lib.mlvc_hip_conv_workspace_bytes.restype = C.c_size_t
    assert lib.mlvc_hip_conv_plan(C.byref(d)) == 0, lib.mlvc_hip_last_error()
    return d, lib.mlvc_hip_conv_workspace_bytes(C.byref(d))


# (ic, h, w, oc, k, stride, expected ksplit, split_c): the rule of
# mlvc_hip_conv_plan on deep 1x1 convs over few pixels, and on shallow,
# wide or 3x3 ones (never split).
SPLITS = [
    (1024, 23, 40, 256, 1, 1, 8, 128),     # unshuffled 1x1 4C->C at 23x40, C=256: 16 items
    (1024, 46, 80, 256, 1, 1, 8, 128),     # the same over 4x the pixels: 58 items
    (512, 46, 80, 128, 1, 1, 1, 512),      # the C=128 workload's, at 46x80: K = 512 < 576
    (576, 46, 80, 128, 1, 1, 5, 128),      # s = min(8, 17, 9) = 8, ranges of 128: 4 + a last 64
    (640, 6, 10, 192, 1, 1, 5, 128),       # s = min(8, 512, 10) = 8: 64 * ceil(640 / 512) = 128
    (1024, 184, 320, 256, 1, 1, 1, 1024),  # 920 items
    (256, 46, 80, 256, 1, 1, 1, 256),      # K = 256
    (192, 136, 240, 256, 3, 2, 1, 192),    # 3x3: not split
    (256, 46, 80, 256, 3, 1, 1, 256),      # 3x3: not split
]


def test_split_rule():
    for ic, h, w, oc, k, s, want_k, want_c in SPLITS:
        d, ws = plan(ic, h, w, oc, k, s, pad=k // 2)
        got = (d.ksplit if d.ksplit > 1 else 1, d.split_c if d.ksplit > 1 else ic)
        assert got == (want_k, want_c), (ic, h, w, oc, k, s, got)
        if d.ksplit > 1:
            assert ws == d.ksplit * d.n * oc * d.oh * d.ow * 4
            names = candidates(ic, h, w, oc, k, s, pad=k // 2, desc=d)
            assert names and all(nm.startswith("mfma_") for nm in names), names
        else:
            assert ws == 0
    # The epilogue does not change the split (a ReGLU conv is split like a
    # plain one); a batch with enough work items is not split.
    assert plan(1024, 46, 80, 256, 1, 1, pad=0, epilogue=3)[0].ksplit == 8
    assert plan(1024, 46, 80, 256, 1, 1, pad=0, n=16)[0].ksplit <= 1


# The tuned convs of the 1920x1088 graph: (launch, ic, h, w, oc, stride,
# DEPTH_TO_SPACE block, channel-last input, channel-last output).
TUNED_1920 = [
    ("n6_conv3x3", 64, 544, 960, 128, 2, 0, 0, 1),
    ("n8_conv3x3", 128, 272, 480, 192, 2, 0, 1, 1),
    ("n10_conv3x3", 192, 136, 240, 256, 2, 0, 1, 1),
    ("n72_conv3x3", 256, 68, 120, 768, 1, 2, 1, 1),
    ("n75_conv3x3", 192, 136, 240, 512, 1, 2, 1, 1),
    ("n78_conv3x3", 128, 272, 480, 256, 1, 2, 1, 0),
    ("n81_conv3x3", 64, 544, 960, 12, 1, 2, 0, 0),
]


def test_recorded_tuning_names_candidates_of_each_launch():
    """Every choice the recorded tuning file makes for the 1920x1088 graph is
    a variant that can run that launch's geometry and operand layouts, so the
    benchmark and the profiles run exactly the recorded tiles (a name that
    could not would send the tuner back to timing the candidates)."""
    path = pathlib.Path(__file__).resolve().parents[1] / "mlvc.cpp_amd" / "tuning" / "mi355x.txt"
    chosen = dict(line.split() for line in path.read_text().splitlines() if line.strip())
    for name, ic, h, w, oc, stride, d2s, cl_in, cl_out in TUNED_1920:
        oh, ow = (h - 1) // stride + 1, (w - 1) // stride + 1
        d = ConvDesc(n=1, ic=ic, ih=h, iw=w, oc=oc, oh=oh, ow=ow, kh=3, kw=3, stride_h=stride, stride_w=stride,
                     pad_h=1, pad_w=1, epilogue=1, alpha=0.01, out_d2s_block=d2s, in_nhwc=cl_in, out_nhwc=cl_out)
        names = candidates(ic, h, w, oc, stride=stride, d2s=d2s, desc=d)
        assert chosen[f"mlvc_1920x1088:{name}"] in names, (name, chosen[f"mlvc_1920x1088:{name}"], names)
