"""The oracle's codec I/O conversions (frame <-> model image) against the
reference's own core/src/yuv.cpp built from source (oracle/_ref), plus the
identities the conversion fixes by construction.

Reference behaviour restated by the oracle: execution_plan.cpp:1044-1322
(write_yuv420_to_nhwc_fp16 / read_nhwc_fp16_to_yuv420 of the buffered codec
path) and core/src/yuv.cpp:325-527 (frame_padding, prepare_model_input,
prepare_model_output_into), which compute the same values.
"""

import numpy as np
import pytest

import mlvc_oracle as O

needs_ref = pytest.mark.skipif(not O.ref_available(), reason="reference kernels not built (no checkout)")

# (w, h, mw, mh): exact fit, right/bottom padding, rotated fits, tiny.
SHAPES = [(32, 16, 32, 16), (20, 12, 24, 16), (18, 30, 32, 24), (6, 10, 16, 8), (2, 2, 2, 2), (30, 14, 32, 16)]
RANGES = [1.0, 0.5, 2.0, 0.3]


def frame(rng, w, h):
    return rng.integers(0, 256, O.yuv_frame_bytes(w, h), dtype=np.uint8)


def image(rng, mh, mw, pixel_range):
    # Values around [0, range] with margins so clamping is exercised; FP16.
    v = rng.uniform(-0.15, 1.15, (3, mh, mw)) * pixel_range
    return v.astype(np.float16).view(np.uint16)


@needs_ref
@pytest.mark.parametrize("shape", SHAPES, ids=[f"{s[0]}x{s[1]}in{s[2]}x{s[3]}" for s in SHAPES])
@pytest.mark.parametrize("pixel_range", RANGES)
def test_frame_to_model_matches_reference(shape, pixel_range):
    w, h, mw, mh = shape
    rng = np.random.default_rng(w * 131 + h)
    f = frame(rng, w, h)
    want, ref_pad = O.ref_prepare_model_input(f, w, h, mw, mh, pixel_range)
    pad = O.frame_padding(w, h, mw, mh)
    assert pad == ref_pad
    got = O.yuv_to_model(f, w, h, mw, mh, pad[4], pixel_range)
    assert np.array_equal(got, want)


@needs_ref
@pytest.mark.parametrize("shape", SHAPES, ids=[f"{s[0]}x{s[1]}in{s[2]}x{s[3]}" for s in SHAPES])
@pytest.mark.parametrize("pixel_range", RANGES)
def test_model_to_frame_matches_reference(shape, pixel_range):
    w, h, mw, mh = shape
    rng = np.random.default_rng(w * 17 + h * 3 + int(pixel_range * 10))
    x = image(rng, mh, mw, pixel_range)
    pad = O.frame_padding(w, h, mw, mh)
    assert np.array_equal(O.model_to_yuv(x, w, h, pad, pixel_range), O.ref_prepare_model_output(x, w, h, pad, pixel_range))


@needs_ref
@pytest.mark.parametrize("rotated", [0, 1])
def test_model_to_frame_with_offsets_matches_reference(rotated):
    # The decoder side honours arbitrary left/top offsets of the active area.
    w, h = (12, 8) if not rotated else (8, 12)
    mw, mh = 16, 12
    pad = (3, 1, 2, 2, rotated) if not rotated else (3, 1, 2, 2, 1)
    aw, ah = (w, h) if not rotated else (h, w)
    assert aw + pad[0] + pad[1] == mw and ah + pad[2] + pad[3] == mh
    rng = np.random.default_rng(7 + rotated)
    x = image(rng, mh, mw, 1.0)
    assert np.array_equal(O.model_to_yuv(x, w, h, pad, 1.0), O.ref_prepare_model_output(x, w, h, pad, 1.0))


@needs_ref
@pytest.mark.parametrize("pixel_range", [1.0, 0.7])
def test_luma_quantisation_every_half(pixel_range):
    # Every finite FP16 value through the luma path (NaNs excluded: the
    # reference casts NaN to uint8, which C++ leaves undefined).
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    exp = (bits >> 10) & 0x1F
    bits = np.where((exp == 0x1F) & ((bits & 0x3FF) != 0), 0, bits).astype(np.uint16)
    mw, mh = 256, 256
    x = np.zeros((3, mh, mw), np.uint16)
    x[0] = bits.reshape(mh, mw)
    pad = (0, 0, 0, 0, 0)
    got = O.model_to_yuv(x, mw, mh, pad, pixel_range)
    want = O.ref_prepare_model_output(x, mw, mh, pad, pixel_range)
    assert np.array_equal(got[: mw * mh], want[: mw * mh])


@pytest.mark.parametrize("shape", [(32, 16, 32, 16), (16, 32, 32, 16)])
def test_round_trip_identity(shape):
    # With pixel_range 1 the byte LUT value v/255 (FP16, rel. error <= 2^-11)
    # quantises back to v, and each chromas 2x2 block holds one value whose
    # mean is exact: frame -> model -> frame is the identity.
    w, h, mw, mh = shape
    rng = np.random.default_rng(3)
    f = frame(rng, w, h)
    pad = O.frame_padding(w, h, mw, mh)
    x = O.yuv_to_model(f, w, h, mw, mh, pad[4], 1.0)
    assert np.array_equal(O.model_to_yuv(x, w, h, pad, 1.0), f)


def test_known_values():
    # LUT: byte v -> FP16(v / 255 * range); padding repeats the last column/row.
    w, h, mw, mh = 4, 2, 8, 4
    f = np.arange(O.yuv_frame_bytes(w, h), dtype=np.uint8) * 20
    x = O.yuv_to_model(f, w, h, mw, mh, 0, 1.0).view(np.float16)
    yplane = f[: w * h].reshape(h, w)
    expect_y = (yplane.astype(np.float32) / 255.0).astype(np.float16)
    assert np.array_equal(x[0, :h, :w], expect_y)
    assert np.array_equal(x[0, :h, w:], np.repeat(expect_y[:, -1:], mw - w, axis=1))
    assert np.array_equal(x[0, h:, :], np.repeat(x[0, h - 1 : h, :], mh - h, axis=0))
    u = f[w * h : w * h + 2].astype(np.float32) / 255.0
    assert np.array_equal(x[1, 0, :4], np.repeat(u, 2).astype(np.float16))
    # Quantisation: clamp, x255, round half to even.
    img = np.zeros((3, 2, 2), np.float16)
    img[0] = [[-1.0, 2.0], [0.5, 1.0 / 255.0]]
    y = O.model_to_yuv(img.view(np.uint16), 2, 2, (0, 0, 0, 0, 0), 1.0)
    assert list(y[:4]) == [0, 255, 128, 1]
    # Chroma mean of the 2x2 block.
    img[1] = [[0.0, 1.0], [1.0, 0.0]]
    y = O.model_to_yuv(img.view(np.uint16), 2, 2, (0, 0, 0, 0, 0), 1.0)
    assert y[4] == 128


def test_frame_padding_rules():
    assert O.frame_padding(1920, 1080, 1920, 1088) == (0, 0, 0, 8, 0)
    assert O.frame_padding(1080, 1920, 1920, 1088) == (0, 0, 0, 8, 1)
    with pytest.raises(O.OracleError):
        O.frame_padding(2000, 1080, 1920, 1088)
    with pytest.raises(O.OracleError):
        O.frame_padding(1919, 1080, 1920, 1088)


def _codec_pair(tmp_path):
    import mlvc_hip

    mlvc_hip.synth_write("codec_enc_tiny", tmp_path, 0)
    mlvc_hip.synth_write("codec_dec_tiny", tmp_path, 0)
    bindings, _ = mlvc_hip.synth_bindings("codec_enc_tiny")
    return bindings


def test_codec_graph_pair_closed_loop_on_oracle(tmp_path):
    # The synthetic MLVCEncoder runs the decoder's state path with the same
    # weights: loaded without state bindings (ref_in an input, ref_out an
    # output), the encoder's ref_out equals the decoder's for the same latent
    # and ref_in, frame after frame, so encoder and decoder stay in step.
    import mlvc_hip

    bindings = _codec_pair(tmp_path)
    assert bindings == [(2, 1)] and mlvc_hip.synth_bindings("codec_dec_tiny")[0] == bindings
    assert mlvc_hip.aot_inspect(tmp_path, "MLVCDecoder")["nodes"] > 0
    enc = O.OraclePlan(tmp_path, "MLVCEncoder")
    dec = O.OraclePlan(tmp_path, "MLVCDecoder")
    q = np.array([3], np.int32)
    rng = np.random.default_rng(11)
    ref = np.zeros((1, 64, 32, 64), np.uint16)
    for _ in range(2):
        x = rng.uniform(0, 1, (1, 3, 64, 128)).astype(np.float16).view(np.uint16)
        y, enc_ref = enc.run([x, q, ref])
        x_hat, dec_ref = dec.run([y, q, ref])
        assert np.array_equal(enc_ref, dec_ref)
        assert x_hat.shape == (1, 3, 64, 128) and np.isfinite(x_hat.view(np.float16)).all()
        assert np.abs(dec_ref.view(np.float16).astype(np.float32)).max() > 0
        ref = dec_ref
