"""Codec I/O on the GPU: the frame <-> model image kernels and the buffered
encoder / decoder path (BufferedCodecBackend), against the oracle.

Conversions are byte/half work and must match the oracle bit for bit
(execution_plan.cpp:1044-1322 semantics, pinned against the reference's
core/src/yuv.cpp in test_oracle_codec_io.py). The buffered path must give
exactly what run() gives on the same converted inputs (same kernels, same
state sequence), and the graph outputs stay within the FP16 parity bar of
the oracle.
"""

import ctypes as C

import numpy as np
import pytest

import mlvc_hip
import mlvc_oracle as O
from conftest import assert_parity
from devmem import Dev

pytestmark = pytest.mark.gpu


@pytest.fixture
def dev():
    d = Dev()
    yield d
    d.close()


def gpu_yuv_to_model(dev, f, w, h, mw, mh, rotated, pixel_range):
    src = dev.put(f)
    table = dev.put(np.array([O.oracle_lib().oracle_float_to_half(np.float32(v) / np.float32(255.0) * np.float32(pixel_range))
                              for v in range(256)], np.uint16))
    out = dev.alloc(3 * mw * mh * 2)
    dev.check(dev.lib.mlvc_hip_yuv420_to_model(src, table, out, w, h, mw, mh, rotated, None))
    return dev.get(out, (3, mh, mw), np.uint16)


def gpu_model_to_yuv(dev, x, w, h, pad, pixel_range):
    mh, mw = x.shape[-2], x.shape[-1]
    src = dev.put(x)
    out = dev.alloc(O.yuv_frame_bytes(w, h))
    dev.check(dev.lib.mlvc_hip_model_to_yuv420(src, out, w, h, mw, mh, pad[0], pad[2], pad[4], pixel_range, None))
    return dev.get(out, (O.yuv_frame_bytes(w, h),), np.uint8)


# (w, h, mw, mh): vector paths (w, mw % 8 == 0), scalar tails, rotated, the
# 1920x1080 -> 1920x1088 video case.
SHAPES = [(128, 64, 128, 64), (120, 60, 128, 64), (34, 18, 40, 20), (30, 14, 36, 18), (60, 120, 128, 64),
          (14, 30, 32, 16), (2, 2, 8, 8), (1920, 1080, 1920, 1088)]


@pytest.mark.parametrize("shape", SHAPES, ids=[f"{s[0]}x{s[1]}in{s[2]}x{s[3]}" for s in SHAPES])
@pytest.mark.parametrize("pixel_range", [1.0, 0.7, 2.0])
def test_frame_to_model_kernel(dev, shape, pixel_range):
    w, h, mw, mh = shape
    rng = np.random.default_rng(w + 7 * h)
    f = rng.integers(0, 256, O.yuv_frame_bytes(w, h), dtype=np.uint8)
    pad = O.frame_padding(w, h, mw, mh)
    got = gpu_yuv_to_model(dev, f, w, h, mw, mh, pad[4], pixel_range)
    want = O.yuv_to_model(f, w, h, mw, mh, pad[4], pixel_range)
    bad = np.argwhere(got != want)
    assert bad.size == 0, f"{len(bad)} values differ, first at {bad[:4].tolist()}"


@pytest.mark.parametrize("shape", SHAPES, ids=[f"{s[0]}x{s[1]}in{s[2]}x{s[3]}" for s in SHAPES])
@pytest.mark.parametrize("pixel_range", [1.0, 0.7, 2.0])
def test_model_to_frame_kernel(dev, shape, pixel_range):
    w, h, mw, mh = shape
    rng = np.random.default_rng(3 * w + h)
    x = (rng.uniform(-0.15, 1.15, (3, mh, mw)) * pixel_range).astype(np.float16).view(np.uint16)
    pad = O.frame_padding(w, h, mw, mh)
    got = gpu_model_to_yuv(dev, x, w, h, pad, pixel_range)
    want = O.model_to_yuv(x, w, h, pad, pixel_range)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{bad.size} bytes differ, first at {bad[:8].tolist()}"


@pytest.mark.parametrize("case", [((12, 8, 16, 12), (3, 1, 2, 2, 0)), ((16, 8, 24, 12), (8, 0, 2, 2, 0)),
                                  ((8, 12, 16, 12), (3, 1, 2, 2, 1))], ids=["odd_left", "aligned_left", "rotated"])
def test_model_to_frame_offsets(dev, case):
    (w, h, mw, mh), pad = case
    rng = np.random.default_rng(w * h)
    x = rng.uniform(-0.1, 1.1, (3, mh, mw)).astype(np.float16).view(np.uint16)
    assert np.array_equal(gpu_model_to_yuv(dev, x, w, h, pad, 1.0), O.model_to_yuv(x, w, h, pad, 1.0))


@pytest.mark.parametrize("pixel_range", [1.0, 0.7])
def test_quantisation_every_half(dev, pixel_range):
    # Every FP16 bit pattern (NaN -> 0 on both sides here: the oracle's
    # std::clamp passes NaN through to an x86 conversion, so NaNs are
    # replaced) through luma, and shuffled through both chroma planes.
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    bits = np.where(np.isnan(bits.view(np.float16)), 0, bits).astype(np.uint16)
    rng = np.random.default_rng(5)
    x = np.stack([bits, rng.permutation(bits), rng.permutation(bits)]).reshape(3, 256, 256)
    pad = (0, 0, 0, 0, 0)
    assert np.array_equal(gpu_model_to_yuv(dev, x, 256, 256, pad, pixel_range),
                          O.model_to_yuv(x, 256, 256, pad, pixel_range))


def test_round_trip_identity_full_size(dev):
    w, h, mw, mh = 1920, 1080, 1920, 1088
    rng = np.random.default_rng(9)
    f = rng.integers(0, 256, O.yuv_frame_bytes(w, h), dtype=np.uint8)
    pad = O.frame_padding(w, h, mw, mh)
    x = gpu_yuv_to_model(dev, f, w, h, mw, mh, 0, 1.0)
    assert np.array_equal(gpu_model_to_yuv(dev, x, w, h, pad, 1.0), f)


# ---- buffered encoder / decoder ----------------------------------------

MW, MH = 128, 64  # codec_*_tiny model image


@pytest.fixture
def pair(tmp_path):
    mlvc_hip.synth_write("codec_enc_tiny", tmp_path, 0)
    mlvc_hip.synth_write("codec_dec_tiny", tmp_path, 0)
    bindings, _ = mlvc_hip.synth_bindings("codec_enc_tiny")
    return tmp_path, bindings


def backend(d, model, bindings):
    b = mlvc_hip.Backend(d, "hip")
    b.load(model, bindings)
    return b


@pytest.mark.parametrize("frame_wh", [(128, 60), (60, 128)], ids=["native", "rotated"])
def test_buffered_encoder_then_decoder(pair, frame_wh):
    d, bindings = pair
    w, h = frame_wh
    frames, q = 4, 7
    rng = np.random.default_rng(21)
    clips = [rng.integers(0, 256, O.yuv_frame_bytes(w, h), dtype=np.uint8) for _ in range(frames)]

    enc = backend(d, "MLVCEncoder", bindings)
    pad = enc.configure_codec_io(w, h, MW, MH, 1.0, slots=2)
    assert enc.codec_slot_count() == 2
    enc.reset_state()
    enc_run = backend(d, "MLVCEncoder", bindings)
    enc_run.reset_state()
    oracle_enc = O.OraclePlan(d, "MLVCEncoder", bindings)
    oracle_enc.reset_state()

    latents = []
    for i, f in enumerate(clips):
        slot = i % 2
        if i >= 2:
            enc.wait_codec_slot(slot)
        enc.encoder_input_yuv(slot)[:] = f
        enc.submit_encoder(slot, q)
        if i >= 1:  # the other slot is in flight: finish the previous frame
            prev = (i - 1) % 2
            enc.wait_codec_slot(prev)
            latents.append(enc.encoder_outputs(prev)[0].copy())
    enc.wait_codec_slot((frames - 1) % 2)
    latents.append(enc.encoder_outputs((frames - 1) % 2)[0].copy())

    for i, f in enumerate(clips):
        x = O.yuv_to_model(f, w, h, MW, MH, pad[4], 1.0).reshape(1, 3, MH, MW)
        want = enc_run.run([x, np.array([q], np.int32)])[0]
        assert np.array_equal(latents[i].reshape(want.shape), want), f"frame {i}: buffered != run()"
        assert_parity(want, oracle_enc.run([x, np.array([q], np.int32)])[0], f"encoder frame {i}")

    dec = backend(d, "MLVCDecoder", bindings)
    dec.configure_codec_io(w, h, MW, MH, 1.0, padding=pad, slots=3)
    dec.reset_state()
    dec_run = backend(d, "MLVCDecoder", bindings)
    dec_run.reset_state()
    oracle_dec = O.OraclePlan(d, "MLVCDecoder", bindings)
    oracle_dec.reset_state()
    for i, y in enumerate(latents):
        slot = i % 3
        dec.decoder_inputs(slot)[0][:] = y
        dec.submit_decoder(slot, q)
        dec.wait_codec_slot(slot)
        got = dec.decoder_output_yuv(slot)
        ys = y.reshape(1, 256, MH // 16, MW // 16)
        x_hat = dec_run.run([ys, np.array([q], np.int32)])[0]
        assert np.array_equal(got, O.model_to_yuv(x_hat.reshape(3, MH, MW), w, h, pad, 1.0)), f"frame {i}"
        assert_parity(x_hat, oracle_dec.run([ys, np.array([q], np.int32)])[0], f"decoder frame {i}")
    for b in (enc, enc_run, dec, dec_run):
        b.close()


def test_codec_graphs_are_the_oracle_gpu_arithmetic(pair):
    """Encoder then decoder over 4 frames, each backend carrying its own
    recurrent state: every output of both graphs equals the isa-2 oracle
    plan's (the matrix core's summation order) bit for bit, so their
    difference from the reference order (held to the FP16 bar above) is
    summation order alone."""
    d, bindings = pair
    rng = np.random.default_rng(5)
    q = np.array([3], np.int32)
    enc, dec = backend(d, "MLVCEncoder", bindings), backend(d, "MLVCDecoder", bindings)
    model_enc = O.OraclePlan(d, "MLVCEncoder", bindings, isa=2)
    model_dec = O.OraclePlan(d, "MLVCDecoder", bindings, isa=2)
    for b in (enc, dec, model_enc, model_dec):
        b.reset_state()
    for i in range(4):
        f = rng.integers(0, 256, O.yuv_frame_bytes(MW, MH), dtype=np.uint8)
        x = O.yuv_to_model(f, MW, MH, MW, MH, 0, 1.0).reshape(1, 3, MH, MW)
        got, want = enc.run([x, q]), model_enc.run([x, q])
        for k, (g, w) in enumerate(zip(got, want)):
            assert np.array_equal(g, w), f"encoder frame {i} output {k}: {np.count_nonzero(g != w)} of {g.size} differ"
        ys = got[0].reshape(1, 256, MH // 16, MW // 16)
        got, want = dec.run([ys, q]), model_dec.run([ys, q])
        for k, (g, w) in enumerate(zip(got, want)):
            assert np.array_equal(g, w), f"decoder frame {i} output {k}: {np.count_nonzero(g != w)} of {g.size} differ"
    enc.close()
    dec.close()


def test_buffered_contract(pair):
    d, bindings = pair
    enc = backend(d, "MLVCEncoder", bindings)
    with pytest.raises(mlvc_hip.MlvcError, match="unavailable"):
        enc.encoder_input_yuv(0)
    with pytest.raises(mlvc_hip.MlvcError, match="padded dimensions"):
        enc.configure_codec_io(128, 60, MW, MH, 1.0, padding=(0, 0, 0, 0, 0))
    with pytest.raises(mlvc_hip.MlvcError, match="pixel range"):
        enc.configure_codec_io(128, 60, MW, MH, 0.0)
    enc.configure_codec_io(128, 60, MW, MH, 1.0, slots=1)
    with pytest.raises(mlvc_hip.MlvcError, match="already configured"):
        enc.configure_codec_io(128, 60, MW, MH, 1.0)
    with pytest.raises(mlvc_hip.MlvcError, match="reset_state"):
        enc.submit_encoder(0, 1)
    enc.reset_state()
    with pytest.raises(mlvc_hip.MlvcError, match="out of range"):
        enc.submit_encoder(1, 1)
    with pytest.raises(mlvc_hip.MlvcError, match="decoder codec I/O is unavailable"):
        enc.decoder_inputs(0)
    enc.submit_encoder(0, 1)
    for touch in (lambda: enc.encoder_input_yuv(0), lambda: enc.encoder_outputs(0), lambda: enc.submit_encoder(0, 1)):
        with pytest.raises(mlvc_hip.MlvcError, match="pending"):
            touch()
    enc.wait_codec_slot(0)
    enc.wait_codec_slot(0)  # waiting an idle slot is a no-op
    assert len(enc.encoder_outputs(0)) == 1
    enc.close()

    plain = mlvc_hip.Backend(d, "hip")
    mlvc_hip.synth_write("mlvc_tiny", d, 0)
    plain.load("mlvc_tiny", mlvc_hip.synth_bindings("mlvc_tiny")[0])
    with pytest.raises(mlvc_hip.MlvcError, match="unsupported codec graph"):
        plain.configure_codec_io(128, 64, 128, 64, 1.0)
    plain.close()


def test_run_takes_int32_control_input(pair):
    d, bindings = pair
    dec = backend(d, "MLVCDecoder", bindings)
    dec.reset_state()
    assert dec.in_dtypes == [np.uint16, np.int32]
    y = np.zeros((1, 256, MH // 16, MW // 16), np.uint16)
    x_hat = dec.run([y, np.array([2], np.int32)])[0]
    assert x_hat.shape == (1, 3, MH, MW)
    dec.close()
