"""Every conv tile variant on every conv geometry of the MLVC-shaped graphs.

The backend tunes the tile variant per launch at load time, so a variant that
is wrong on some geometry could pass the other tests only because it was not
the fastest there. Here MLVC_HIP_CONV_VARIANT forces each variant in turn;
each result must match the oracle, and all variants of one kernel size must
agree bit for bit (they accumulate in the same K order).
"""

import numpy as np
import pytest

import graphs
import mlvc_hip
import mlvc_oracle
from conftest import assert_parity

pytestmark = pytest.mark.gpu

# (name, n, ic, h, w, oc, k, stride, pad, options): the convs of mlvc_s_tiny
# (32x64), of the 1920x1088 graph at reduced size, and ragged shapes.
CASES = [
    ("unshuffle_in", 1, 12, 16, 32, 64, 3, 1, 1, dict(s2d=2, epilogue="lrelu")),
    ("concat_1x1", 1, 128, 16, 32, 64, 1, 1, 0, dict(concat_ic=64, epilogue="lrelu")),
    ("down_s2", 1, 64, 16, 32, 128, 3, 2, 1, dict(epilogue="lrelu")),
    ("down_s2_4x8", 1, 128, 8, 16, 192, 3, 2, 1, dict(epilogue="lrelu")),
    ("mid_4x8", 1, 192, 4, 8, 256, 3, 1, 1, dict(epilogue="lrelu")),
    ("synth_4x8", 1, 256, 4, 8, 192, 3, 1, 1, dict(epilogue="lrelu")),
    ("shuffle_4x8", 1, 192, 4, 8, 512, 3, 1, 1, dict(epilogue="lrelu", d2s=2)),
    ("shuffle_8x16", 1, 128, 8, 16, 256, 3, 1, 1, dict(epilogue="lrelu", d2s=2)),
    ("recon_16x32", 1, 64, 16, 32, 12, 3, 1, 1, dict(d2s=2)),
    ("ragged_s1", 1, 72, 13, 27, 96, 3, 1, 1, dict(epilogue="residual")),
    ("ragged_s2", 1, 40, 11, 26, 72, 3, 2, 1, dict()),
    ("ragged_1x1", 2, 48, 7, 13, 80, 1, 1, 0, dict(epilogue="residual")),
    ("d2s3_fallback", 1, 32, 9, 12, 18, 3, 1, 1, dict(epilogue="lrelu", d2s=3)),
    ("residual_d2s", 1, 64, 6, 16, 64, 3, 1, 1, dict(epilogue="residual", d2s=2)),
    # More tiles than the device holds workgroups at once: each workgroup
    # walks several tiles (next tile staged under the current one's last
    # chunk), across output-channel blocks and both images.
    ("many_tiles_s1", 2, 32, 256, 1024, 64, 3, 1, 1, dict(epilogue="lrelu")),
    ("many_tiles_d2s", 1, 32, 384, 768, 128, 3, 1, 1, dict(epilogue="lrelu", d2s=2)),
    ("many_tiles_s2", 2, 24, 600, 1000, 64, 3, 2, 1, dict(epilogue="residual")),
    ("many_tiles_1x1", 1, 128, 512, 512, 64, 1, 1, 0, dict(concat_ic=64, epilogue="lrelu")),
    ("many_tiles_s2_rows", 1, 64, 272, 960, 192, 3, 2, 1, dict(epilogue="lrelu")),
    # At most 16 output channels: plain and DEPTH_TO_SPACE(2) outputs, ragged
    # right edge, and more tiles than the device holds workgroups at once.
    ("small_oc_plain", 1, 32, 24, 64, 8, 3, 1, 1, dict(epilogue="lrelu")),
    ("small_oc_residual", 1, 64, 20, 40, 16, 3, 1, 1, dict(epilogue="residual")),
    ("recon_many_tiles", 2, 64, 136, 512, 12, 3, 1, 1, dict(d2s=2)),
    # Input channels not a multiple of the weight-streaming kernel's pass
    # width (32 or 64): the last pass is partial.
    ("ragged_ic_ws", 1, 80, 12, 32, 128, 3, 1, 1, dict(epilogue="lrelu")),
    ("ragged_ic_ws_d2s", 2, 48, 8, 16, 256, 3, 1, 1, dict(epilogue="lrelu", d2s=2)),
    # Split K (deep 1x1 convs over few pixels): 8 splits of an unshuffled
    # 1x1, five splits with a ragged last one (600 = 4 x 128 + 88 channels)
    # and a residual over two images, a plane of 77 pixels (the reduce
    # kernel's one-output-per-thread path) with LeakyReLU.
    ("split_1x1_s2d", 1, 1024, 6, 16, 256, 1, 1, 0, dict(s2d=2)),
    ("split_residual_n2", 2, 600, 6, 10, 64, 1, 1, 0, dict(epilogue="residual")),
    ("split_ragged_plane", 1, 768, 7, 11, 96, 1, 1, 0, dict(epilogue="lrelu")),
]

# Geometries the weight-streaming 3x3 kernel (conv_ws.hpp) takes: NCHW inputs
# with rows of a multiple of 8 pixels, no concat or SPACE_TO_DEPTH staging.
WS_CASES = {"mid_4x8", "shuffle_8x16", "many_tiles_s1", "many_tiles_d2s", "residual_d2s", "down_s2", "down_s2_4x8",
            "many_tiles_s2_rows", "ragged_ic_ws", "ragged_ic_ws_d2s"}


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_every_variant(tmp_path, monkeypatch, case):
    name, n, ic, h, w, oc, k, s, p, opts = case
    shapes = graphs.single_conv_graph(tmp_path, "m", n, ic, h, w, oc, k, s, p, seed=len(name), **opts)
    rng = np.random.default_rng(5)
    ins = [graphs.half(rng.uniform(-1, 1, sh)) for sh in shapes]
    want = mlvc_oracle.OraclePlan(tmp_path, "m").run(ins)[0]
    first, ran, split = None, [], False
    for v in mlvc_hip.conv_variants()[1:]:
        monkeypatch.setenv("MLVC_HIP_CONV_VARIANT", v)
        gpu = mlvc_hip.Backend(tmp_path, "hip")
        gpu.load("m")
        kinds = [l["kind"] for l in gpu.launches()]
        if not any(kd.startswith(v + "+") or kd == v for kd in kinds):
            gpu.close()
            continue  # not eligible for this geometry
        split = split or any("+split" in kd for kd in kinds)
        got = gpu.run(ins)[0]
        gpu.close()
        assert_parity(got, want, f"{name} with {v}")
        if first is None:
            first = (v, got)
        else:
            assert (got == first[1]).all(), f"{name}: {v} differs from {first[0]}"
        ran.append(v)
    assert len(ran) >= 2, ran
    if split:  # split K runs on the conv_mfma variants only
        assert all(v.startswith("mfma_") for v in ran), ran
    elif name in WS_CASES:  # the weight-streaming kernel is among them
        assert any(v.startswith("ws_") for v in ran), ran
    if name.startswith("split_"):
        assert split, name
