"""GPU parity of the synthetic workloads through the "hip" backend's C ABI
against the CPU oracle: the single 3x3 conv (1 launch), the conv sweep,
the depthwise-separable blocks with fused shuffles and the MLVC-shaped
recurrent graphs, both free-running (each side carries its own state) and
teacher-forced (the GPU is fed the oracle's state every frame, isolating
per-frame error from recurrence drift)."""

import numpy as np
import pytest

import mlvc_hip
import mlvc_oracle
from conftest import assert_parity

pytestmark = pytest.mark.gpu


def _write(tmp_path, config):
    mlvc_hip.synth_write(config, tmp_path, 0)
    return mlvc_hip.synth_bindings(config)


@pytest.mark.parametrize("config", ["conv3x3_184x320", "conv_sweep_640x368", "dwblock_92x160_c128",
                                    "dwblock_46x80_c256", "dwblock_tiny"])
def test_feedforward_configs(tmp_path, config):
    _write(tmp_path, config)
    gpu = mlvc_hip.Backend(tmp_path, "hip")
    gpu.load(config)
    ref = mlvc_oracle.OraclePlan(tmp_path, config)
    ins = [mlvc_hip.synth_input(config, i, 0, s) for i, s in enumerate(gpu.in_shapes)]
    got, want = gpu.run(ins), ref.run(ins)
    assert len(got) == len(want)
    for i, (g, w) in enumerate(zip(got, want)):
        assert_parity(g, w, f"{config} output {i}")
    if config == "conv3x3_184x320":
        assert len(gpu.launches()) == 1  # conv + bias + LeakyReLU in one kernel
    gpu.close()


@pytest.mark.parametrize("config,frames", [("mlvc_s_tiny", 4), ("mlvc_tiny", 4), ("mlvc_s_640x368", 8)])
def test_recurrent_free_running(tmp_path, config, frames):
    bindings, _ = _write(tmp_path, config)
    gpu = mlvc_hip.Backend(tmp_path, "hip")
    gpu.load(config, bindings)
    ref = mlvc_oracle.OraclePlan(tmp_path, config, bindings)
    with pytest.raises(mlvc_hip.MlvcError, match="reset_state"):
        gpu.run([mlvc_hip.synth_input(config, 0, 0, gpu.in_shapes[0])])
    gpu.reset_state()
    ref.reset_state()
    first = None
    for f in range(frames):
        x = mlvc_hip.synth_input(config, 0, f, gpu.in_shapes[0])
        got, want = gpu.run([x]), ref.run([x])
        assert len(got) == 1  # the state output is bound, only recon is returned
        assert_parity(got[0], want[0], f"{config} frame {f}")
        if f == 0:
            first = got[0].copy()
    # reset_state restores frame 0 exactly.
    gpu.reset_state()
    again = gpu.run([mlvc_hip.synth_input(config, 0, 0, gpu.in_shapes[0])])[0]
    assert (again == first).all()
    gpu.close()


@pytest.mark.parametrize("config,frames", [("mlvc_s_tiny", 3), ("mlvc_s_640x368", 8), ("mlvc_1920x1088", 32)])
def test_recurrent_teacher_forced(tmp_path, config, frames):
    _write(tmp_path, config)
    # Unbound: ref_in is an ordinary input and ref_out an ordinary output.
    gpu = mlvc_hip.Backend(tmp_path, "hip")
    gpu.load(config)
    ref = mlvc_oracle.OraclePlan(tmp_path, config)
    state = np.zeros(gpu.in_shapes[1], np.uint16)
    for f in range(frames):
        x = mlvc_hip.synth_input(config, 0, f, gpu.in_shapes[0])
        got, want = gpu.run([x, state]), ref.run([x, state])
        for i, (g, w) in enumerate(zip(got, want)):
            assert_parity(g, w, f"{config} frame {f} output {i}")
        state = want[1]
    gpu.close()


# Free-running bound of the 1920x1088 graph, from summation order alone. The
# oracle's GPU-order model (isa 2: each conv summed as 16-channel steps with
# taps inside, every 16-product group added to the FP32 accumulator once),
# run free-running against the reference order on the CPU over these 32
# frames, levels at recon mean |d|/RMS 1.33e-3-1.34e-3 from frame ~12 with
# max |d|/RMS <= 1.06e-2; teacher-forced it gives 6.8e-4 recon / 4.0e-4
# state, as the GPU does (tests/test_oracle_order_drift.py runs the same
# comparison on the 640x368 graph). The bounds are those figures with 12%
# (mean) and 40% (max) headroom.
DRIFT_MAX_REL, DRIFT_MEAN_REL = 1.5e-2, 1.5e-3


def test_mlvc_1920x1088_free_running(tmp_path):
    """The 1920x1088 graph over 32 frames, each backend carrying its own
    recurrent state. Frame 0 (both states zero) meets the FP16 bar. After it
    each side feeds its own FP16 rounding back through the 64-channel state,
    so the difference grows for about ten frames and then levels off (recon
    mean |d| about 1.33e-3 of RMS, against a flat 6.8e-4 when the GPU is fed
    the oracle's state every frame, which test_recurrent_teacher_forced holds
    to the FP16 bar). A CPU model of the GPU's summation order shows the same
    curve against the reference order, so the excess over the per-frame bar
    is summation order fed back through the state, not a bias of one layer.
    Every frame stays within the order-only bound above, and the last eight
    frames' mean error is no larger than the eight before them, give or take
    5%: the drift is bounded, not growing."""
    config = "mlvc_1920x1088"
    bindings, _ = _write(tmp_path, config)
    gpu = mlvc_hip.Backend(tmp_path, "hip")
    gpu.load(config, bindings)
    ref = mlvc_oracle.OraclePlan(tmp_path, config, bindings)
    gpu.reset_state()
    ref.reset_state()
    means = []
    for f in range(32):
        x = mlvc_hip.synth_input(config, 0, f, gpu.in_shapes[0])
        got, want = gpu.run([x])[0], ref.run([x])[0]
        if f == 0:
            assert_parity(got, want, f"{config} frame 0")
        st = mlvc_oracle.parity_stats(got, want)
        assert st["finite"], f"{config} frame {f}: non-finite output"
        assert st["max_rel"] <= DRIFT_MAX_REL and st["mean_rel"] <= DRIFT_MEAN_REL, f"{config} frame {f}: {st}"
        means.append(st["mean_rel"])
    assert np.mean(means[24:]) <= 1.05 * np.mean(means[16:24]), means
    gpu.close()


def test_device_resident_replay_matches_run(tmp_path):
    """Frames replayed from HBM (the bench path) produce the same outputs as
    run() on the same inputs."""
    config = "mlvc_s_tiny"
    bindings, _ = _write(tmp_path, config)
    a = mlvc_hip.Backend(tmp_path, "hip")
    a.load(config, bindings)
    b = mlvc_hip.Backend(tmp_path, "hip")
    b.load(config, bindings)
    x = mlvc_hip.synth_input(config, 0, 0, a.in_shapes[0])
    a.reset_state()
    b.reset_state()
    for _ in range(3):
        want = a.run([x])
    b.upload_inputs([x])
    b.time_frames(3)
    got = b.download_outputs()
    assert (got[0] == want[0]).all()
    a.close()
    b.close()


def test_per_frame_timing_replays_the_same_frames(tmp_path):
    """time_frames_each (with and without the cache-flush copy between frames)
    advances the recurrent state exactly as run() does and returns one
    positive time per frame."""
    config = "mlvc_s_tiny"
    bindings, _ = _write(tmp_path, config)
    a = mlvc_hip.Backend(tmp_path, "hip")
    a.load(config, bindings)
    b = mlvc_hip.Backend(tmp_path, "hip")
    b.load(config, bindings)
    x = mlvc_hip.synth_input(config, 0, 0, a.in_shapes[0])
    a.reset_state()
    b.reset_state()
    for _ in range(5):
        want = a.run([x])
    b.upload_inputs([x])
    warm = b.time_frames_each(3)
    cold = b.time_frames_each(2, 8 << 20)
    assert warm.shape == (3,) and cold.shape == (2,)
    assert (warm > 0).all() and (cold > 0).all()
    assert (b.download_outputs()[0] == want[0]).all()
    with pytest.raises(mlvc_hip.MlvcError, match="frames"):
        b.time_frames_each(0)
    a.close()
    b.close()


def test_cold_launch_timing(tmp_path):
    """time_launch_cold times single launches after a cache-evicting copy:
    one positive time per launch, and the argument checks of the C ABI."""
    config = "mlvc_s_tiny"
    bindings, _ = _write(tmp_path, config)
    b = mlvc_hip.Backend(tmp_path, "hip")
    b.load(config, bindings)
    b.upload_inputs([mlvc_hip.synth_input(config, 0, 0, b.in_shapes[0])])
    b.reset_state()
    b.time_frames(1)
    n = len(b.launches())
    for i in (0, n - 1):
        ms = b.time_launch_cold(i, 3, 8 << 20)
        assert ms.shape == (3,) and (ms > 0).all()
    with pytest.raises(mlvc_hip.MlvcError, match="reps"):
        b.time_launch_cold(0, 0, 8 << 20)
    with pytest.raises(mlvc_hip.MlvcError, match="flush_bytes"):
        b.time_launch_cold(0, 1, 0)
    b.close()


@pytest.mark.parametrize("config", ["mlvc_s_tiny", "mlvc_tiny", "dwblock_92x160_c128", "dwblock_46x80_c256"])
def test_fused_and_unfused_schedules_bit_identical(tmp_path, monkeypatch, config):
    """Every GPU fusion (S2D/CONCAT loads, epilogues, D2S stores, the fused
    depthwise-separable block) keeps the unfused rounding points and K order,
    so both schedules give identical bits."""
    bindings, _ = _write(tmp_path, config)
    fused = mlvc_hip.Backend(tmp_path, "hip")
    fused.load(config, bindings)
    monkeypatch.setenv("MLVC_HIP_DISABLE_FUSION", "1")
    plain = mlvc_hip.Backend(tmp_path, "hip")
    plain.load(config, bindings)
    monkeypatch.delenv("MLVC_HIP_DISABLE_FUSION")
    assert len(fused.launches()) < len(plain.launches())
    kinds = " ".join(l["kind"] for l in fused.launches())
    assert "dwblock" in kinds, kinds
    for b in (fused, plain):
        if bindings:
            b.reset_state()
    for f in range(2):
        ins = [mlvc_hip.synth_input(config, i, f, s) for i, s in enumerate(fused.in_shapes)]
        for g, p in zip(fused.run(ins), plain.run(ins)):
            assert (g == p).all(), f"frame {f}"
    fused.close()
    plain.close()
