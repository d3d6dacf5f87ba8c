"""GPU parity of single-operator graphs: the "hip" backend (HIP kernels via
the C ABI) against the CPU oracle on identical seeded inputs and weights.

Covers every conv kernel family (MFMA 3x3 s1/s2, 1x1 flat, 1x1 2-D, direct
fallback) with ragged sizes, channel counts that are not multiples of the
tile or chunk, the fused epilogues (LeakyReLU, residual ADD) and the fused
SPACE_TO_DEPTH / CONCAT loads and DEPTH_TO_SPACE stores, plus depthwise and
the standalone pixel-layout and elementwise kernels. Tolerance: max|d| <=
1e-2 and mean|d| <= 1e-3 relative to the oracle output RMS.
"""

import numpy as np
import pytest

import graphs
import mlvc_hip
import mlvc_oracle
from conftest import assert_parity

pytestmark = pytest.mark.gpu


def run_both(tmp_path, model, inputs_shapes, seed=7):
    rng = np.random.default_rng(seed)
    ins = [graphs.half(rng.uniform(-1, 1, s)) for s in inputs_shapes]
    ref = mlvc_oracle.OraclePlan(tmp_path, model)
    want = ref.run(ins)
    gpu = mlvc_hip.Backend(tmp_path, "hip")
    gpu.load(model)
    got = gpu.run(ins)
    launches = gpu.launches()
    gpu.close()
    return got, want, launches


CONV_CASES = [
    # n, ic, h, w, oc, k, stride, pad
    (1, 64, 23, 37, 64, 3, 1, 1),
    (1, 12, 17, 29, 64, 3, 1, 1),
    (1, 3, 9, 11, 16, 3, 1, 1),
    (1, 16, 4, 5, 32, 3, 1, 1),
    (1, 128, 16, 24, 256, 3, 1, 1),
    (1, 64, 20, 33, 12, 3, 1, 1),
    (1, 13, 7, 9, 11, 3, 1, 1),
    (2, 32, 10, 12, 48, 3, 1, 1),
    (1, 64, 23, 37, 128, 3, 2, 1),
    (1, 128, 18, 30, 256, 3, 2, 1),
    (1, 16, 4, 5, 16, 3, 2, 1),
    (1, 3, 7, 9, 8, 3, 2, 1),
    (1, 64, 23, 37, 64, 1, 1, 0),
    (1, 128, 10, 10, 64, 1, 1, 0),
    (1, 256, 8, 9, 512, 1, 1, 0),
    (1, 512, 5, 7, 256, 1, 1, 0),
    (1, 13, 5, 7, 11, 1, 1, 0),
    (1, 16, 9, 9, 8, 5, 1, 2),   # direct fallback
    (1, 8, 8, 10, 16, 2, 2, 0),  # direct fallback
    (1, 16, 6, 7, 8, 3, 1, 0),   # MFMA with pad 0
]


@pytest.mark.parametrize("case", CONV_CASES, ids=lambda c: "n{}_ic{}_{}x{}_oc{}_k{}s{}p{}".format(*c))
def test_conv_geometry(tmp_path, case):
    n, ic, h, w, oc, k, s, p = case
    shapes = graphs.single_conv_graph(tmp_path, "m", n, ic, h, w, oc, k, s, p, seed=sum(case))
    got, want, launches = run_both(tmp_path, "m", shapes)
    assert_parity(got[0], want[0], f"conv {case} via {launches[0]['kind']}")


@pytest.mark.parametrize("epilogue", ["lrelu", "residual"])
@pytest.mark.parametrize("case", [(1, 64, 19, 35, 64, 3, 1, 1), (1, 64, 19, 35, 128, 3, 2, 1), (1, 128, 9, 13, 96, 1, 1, 0)])
def test_conv_epilogues(tmp_path, case, epilogue):
    n, ic, h, w, oc, k, s, p = case
    shapes = graphs.single_conv_graph(tmp_path, "m", n, ic, h, w, oc, k, s, p, epilogue=epilogue, seed=3)
    got, want, launches = run_both(tmp_path, "m", shapes)
    assert len(launches) == 1 and ("lrelu" in launches[0]["kind"] or "residual" in launches[0]["kind"])
    assert_parity(got[0], want[0], f"conv {case} + {epilogue}")


@pytest.mark.parametrize("k,pad", [(3, 1), (1, 0)])
def test_fused_space_to_depth_load(tmp_path, k, pad):
    # Input channels 12 = 3 x 2^2 (frame unshuffle) and 64 = 16 x 4.
    for ic in (12, 64):
        d = tmp_path / f"ic{ic}"
        shapes = graphs.single_conv_graph(d, "m", 1, ic, 14, 22, 32, k, 1, pad, s2d=2, epilogue="lrelu", seed=ic)
        got, want, launches = run_both(d, "m", shapes)
        assert len(launches) == 1 and "+s2d" in launches[0]["kind"], launches
        assert_parity(got[0], want[0], f"s2d-fused conv ic={ic} k={k}")


@pytest.mark.parametrize("k,pad,oc", [(3, 1, 64), (3, 1, 12), (1, 0, 256)])
def test_fused_depth_to_space_store(tmp_path, k, pad, oc):
    shapes = graphs.single_conv_graph(tmp_path, "m", 1, 32, 11, 19, oc, k, 1, pad, d2s=2, epilogue="lrelu", seed=oc)
    got, want, launches = run_both(tmp_path, "m", shapes)
    assert len(launches) == 1 and "+d2s" in launches[0]["kind"], launches
    assert_parity(got[0], want[0], f"d2s-fused conv oc={oc}")


@pytest.mark.parametrize("k,pad", [(1, 0), (3, 1)])
def test_fused_concat_load(tmp_path, k, pad):
    shapes = graphs.single_conv_graph(tmp_path, "m", 1, 128, 12, 20, 64, k, 1, pad, concat_ic=64, epilogue="lrelu")
    got, want, launches = run_both(tmp_path, "m", shapes)
    assert len(launches) == 1 and "+concat" in launches[0]["kind"], launches
    assert_parity(got[0], want[0], "concat-fused conv")


# 3x3 s1 p1 with rows of a multiple of 8 pixels runs the 16-byte row kernel:
# 256x46x80 and 128x92x160 (the residual-block shapes), 8x1x8 (one row, every
# tap at a border), 24x7x16 (two segments a row).
# Two images (n = 2) cover the row kernel's plane -> channel mapping.
@pytest.mark.parametrize("n,c,h,w,k,s,p", [(1, 16, 13, 17, 3, 1, 1), (1, 256, 46, 80, 3, 1, 1), (1, 12, 9, 10, 3, 1, 1),
                                           (1, 64, 15, 21, 3, 2, 1), (1, 32, 11, 11, 5, 1, 2), (1, 128, 92, 160, 3, 1, 1),
                                           (1, 8, 1, 8, 3, 1, 1), (1, 24, 7, 16, 3, 1, 1), (2, 16, 9, 24, 3, 1, 1)])
def test_depthwise(tmp_path, n, c, h, w, k, s, p):
    shapes = graphs.single_conv_graph(tmp_path, "m", n, c, h, w, c, k, s, p, groups=c, seed=c)
    got, want, launches = run_both(tmp_path, "m", shapes)
    assert launches[0]["kind"] == "depthwise"
    st = assert_parity(got[0], want[0], "depthwise")
    if c % 8 == 0 and k == 3 and s == 1:
        # Same seed, same tap order, one fused multiply-add per tap: the
        # reference AVX2 path and the GPU agree bit for bit.
        assert (got[0] == want[0]).all(), st


def test_standalone_layout_and_eltwise(tmp_path, rng):
    # Graph with nothing to fuse into: pixel ops, LeakyReLU and ADD run as
    # their own kernels (graph outputs are never fused away).
    g = graphs.Graph()
    x = g.input("x", [1, 8, 6, 10])
    y = g.input("y", [1, 8, 6, 10])
    a = g.binary("ADD", "a", x, y)
    l = g.leaky_relu("l", a, 0.2)
    u = g.pixel("SPACE_TO_DEPTH", "u", l, 2)
    v = g.pixel("DEPTH_TO_SPACE", "v", u, 2)
    c = g.concat("c", [v, x], 1)
    for t in (a, l, u, v, c):
        g.output(t)
    g.write(tmp_path, "m")
    ins = [graphs.half(rng.uniform(-2, 2, (1, 8, 6, 10))) for _ in range(2)]
    want = mlvc_oracle.OraclePlan(tmp_path, "m").run(ins)
    gpu = mlvc_hip.Backend(tmp_path, "hip")
    gpu.load("m")
    got = gpu.run(ins)
    kinds = [l["kind"] for l in gpu.launches()]
    assert kinds == ["add", "leaky_relu", "space_to_depth", "depth_to_space", "concat"], kinds
    for i, (gg, ww) in enumerate(zip(got, want)):
        assert (gg == ww).all(), f"output {i} differs"  # one rounding per op on both sides


# Block-2 shuffles on aligned rows run the row kernels (D2S: input width
# % 4 == 0; S2D: input width % 16 == 0), the others the per-element kernels:
# the residual-block path's 512-channel shuffle, two images, and widths on
# either side of each condition.
@pytest.mark.parametrize("op,shape", [("DEPTH_TO_SPACE", (1, 512, 12, 16)), ("DEPTH_TO_SPACE", (2, 16, 5, 8)),
                                      ("DEPTH_TO_SPACE", (1, 8, 3, 12)), ("DEPTH_TO_SPACE", (1, 64, 7, 4)),
                                      ("DEPTH_TO_SPACE", (2, 8, 4, 6)), ("SPACE_TO_DEPTH", (1, 128, 12, 32)),
                                      ("SPACE_TO_DEPTH", (2, 4, 4, 16)), ("SPACE_TO_DEPTH", (1, 4, 6, 24))])
def test_standalone_pixel_shuffle(tmp_path, rng, op, shape):
    g = graphs.Graph()
    x = g.input("x", list(shape))
    g.output(g.pixel(op, "y", x, 2))
    g.write(tmp_path, "m")
    ins = [graphs.half(rng.uniform(-2, 2, shape))]
    want = mlvc_oracle.OraclePlan(tmp_path, "m").run(ins)
    gpu = mlvc_hip.Backend(tmp_path, "hip")
    gpu.load("m")
    got = gpu.run(ins)
    assert [l["kind"] for l in gpu.launches()] == [op.lower()]
    gpu.close()
    assert got[0].shape == want[0].shape and (got[0] == want[0]).all()  # a permutation: bit for bit


# ica <= 16 runs the streaming kernel (persistent grid of two workgroups per
# CU): 150x488 has 608 tiles of 4x32, more than the grid, with ragged last
# rows and columns; n = 2 walks tiles of two images.
@pytest.mark.parametrize("s2d,ica,h,w,acts,n", [(2, 12, 14, 40, (True, True), 1), (0, 16, 9, 24, (True, False), 1),
                                                (0, 40, 6, 16, (False, True), 1), (2, 24, 5, 8, (True, True), 1),
                                                (2, 12, 150, 488, (True, True), 1), (2, 12, 10, 72, (True, False), 2),
                                                (0, 8, 7, 40, (False, True), 2)])
def test_fused_conv_pair(tmp_path, monkeypatch, s2d, ica, h, w, acts, n):
    """3x3 conv [+LeakyReLU] -> CONCAT(t, r) -> 1x1 [+LeakyReLU] runs as one
    launch, matches the oracle and equals the unfused schedule bit for bit."""
    rng = np.random.default_rng(ica + h)
    g = graphs.Graph()
    if s2d:
        x0 = g.input("x", [n, ica // 4, 2 * h, 2 * w])
        x = g.pixel("SPACE_TO_DEPTH", "xs", x0, 2)
    else:
        x = g.input("x", [n, ica, h, w])
    r = g.input("r", [n, 64, h, w])
    wa = g.weight_fp16("wa", rng.normal(0, 1 / np.sqrt(9 * ica), (64, ica, 3, 3)))
    ba = g.weight_fp16("ba", rng.normal(0, 0.1, (64,)))
    t = g.conv("t", x, wa, ba, (1, 1), (1, 1, 1, 1))
    if acts[0]:
        t = g.leaky_relu("ta", t, 0.1)
    c = g.concat("cat", [t, r], 1)
    wb = g.weight_fp16("wb", rng.normal(0, 1 / np.sqrt(128), (64, 128, 1, 1)))
    bb = g.weight_fp16("bb", rng.normal(0, 0.1, (64,)))
    y = g.conv("y", c, wb, bb)
    if acts[1]:
        y = g.leaky_relu("ya", y, 0.2)
    g.output(y)
    g.write(tmp_path, "m")
    ins = [graphs.half(rng.uniform(-1, 1, s)) for s in ([n, ica // 4, 2 * h, 2 * w] if s2d else [n, ica, h, w],
                                                        [n, 64, h, w])]
    want = mlvc_oracle.OraclePlan(tmp_path, "m").run(ins)[0]
    fused = mlvc_hip.Backend(tmp_path, "hip")
    fused.load("m")
    kinds = [l["kind"] for l in fused.launches()]
    assert len(kinds) == 1 and kinds[0].startswith("convpair"), kinds
    got = fused.run(ins)[0]
    fused.close()
    assert_parity(got, want, f"conv pair s2d={s2d} ica={ica} {n}x{h}x{w}")
    monkeypatch.setenv("MLVC_HIP_DISABLE_FUSION", "1")
    plain = mlvc_hip.Backend(tmp_path, "hip")
    plain.load("m")
    ref = plain.run(ins)[0]
    plain.close()
    assert (got == ref).all()


# 1x1 conv -> SLICE [0,G) / [G,2G) -> CLIP(gate) -> MUL(clipped, linear): one
# launch with the ReGLU epilogue (the reference's pointwise ReGLU fusion),
# G-channel output; flattened and ragged pixel counts, two images, G = 32,
# 64 and 96 (several 64-row blocks, a partial last output-channel block);
# 640 input channels over few pixels run split K (ranges of 128 channels,
# the ReGLU applied by the kernel that adds the partials).
@pytest.mark.parametrize("ic,g,h,w,n,lo,hi", [(64, 32, 16, 24, 1, -1.0, 6.0), (48, 64, 7, 13, 2, 0.0, 4.0),
                                              (32, 96, 12, 20, 1, -2.0, 2.0), (640, 96, 6, 10, 2, -1.0, 3.0)])
def test_conv_reglu_epilogue(tmp_path, monkeypatch, ic, g, h, w, n, lo, hi):
    rng = np.random.default_rng(ic + g + h)
    gr = graphs.Graph()
    x = gr.input("x", [n, ic, h, w])
    wt = gr.weight_fp16("w", rng.normal(0, 1 / np.sqrt(ic), (2 * g, ic, 1, 1)))
    bt = gr.weight_fp16("b", rng.normal(0, 0.2, (2 * g,)))
    c = gr.conv("c", x, wt, bt)
    i64 = lambda name, v: gr.weight(name, np.array([v], np.int64), graphs.INT64)  # noqa: E731
    gate = gr.node("SLICE", [c, i64("s0", 0), i64("e0", g), i64("a0", 1)], "gate", [n, g, h, w])
    lin = gr.node("SLICE", [c, i64("s1", g), i64("e1", 2 * g), i64("a1", 1)], "lin", [n, g, h, w])
    clipped = gr.node("CLIP", [gate, gr.weight_fp16("lo", np.array([lo])), gr.weight_fp16("hi", np.array([hi]))], "clipped",
                      [n, g, h, w])
    y = gr.node("MUL", [clipped, lin], "y", [n, g, h, w])
    gr.output(y)
    gr.write(tmp_path, "m")
    ins = [graphs.half(rng.uniform(-3, 3, (n, ic, h, w)))]
    want = mlvc_oracle.OraclePlan(tmp_path, "m").run(ins)[0]
    fused = mlvc_hip.Backend(tmp_path, "hip")
    fused.load("m")
    kinds = [l["kind"] for l in fused.launches()]
    assert len(kinds) == 1 and "+reglu" in kinds[0], kinds
    assert ("+split" in kinds[0]) == (ic == 640), kinds
    got = fused.run(ins)[0]
    fused.close()
    assert_parity(got, want, f"conv+reglu ic={ic} g={g} {n}x{h}x{w}")
    monkeypatch.setenv("MLVC_HIP_DISABLE_FUSION", "1")
    plain = mlvc_hip.Backend(tmp_path, "hip")
    plain.load("m")
    ref = plain.run(ins)[0]
    plain.close()
    assert (got == ref).all()


# conv -> CLIP: one launch with the clamp epilogue (the reference's kClamp
# GEMM epilogue), 3x3 and 1x1, with both bounds or only the upper one.
@pytest.mark.parametrize("k,lo,hi", [(3, -0.5, 0.75), (1, None, 0.25), (3, 0.0, 6.0)])
def test_conv_clip_epilogue(tmp_path, monkeypatch, k, lo, hi):
    rng = np.random.default_rng(k + 17)
    n, ic, h, w, oc = 1, 24, 9, 20, 40
    gr = graphs.Graph()
    x = gr.input("x", [n, ic, h, w])
    wt = gr.weight_fp16("w", rng.normal(0, 1 / np.sqrt(ic * k * k), (oc, ic, k, k)))
    bt = gr.weight_fp16("b", rng.normal(0, 0.2, (oc,)))
    p = k // 2
    c = gr.conv("c", x, wt, bt, (1, 1), (p, p, p, p))
    lo_id = gr.weight_fp16("lo", np.array([lo])) if lo is not None else 0
    y = gr.node("CLIP", [c, lo_id, gr.weight_fp16("hi", np.array([hi]))], "y", [n, oc, h, w])
    gr.output(y)
    gr.write(tmp_path, "m")
    ins = [graphs.half(rng.uniform(-2, 2, (n, ic, h, w)))]
    want = mlvc_oracle.OraclePlan(tmp_path, "m").run(ins)[0]
    fused = mlvc_hip.Backend(tmp_path, "hip")
    fused.load("m")
    kinds = [l["kind"] for l in fused.launches()]
    assert len(kinds) == 1 and kinds[0].endswith("+clip"), kinds
    got = fused.run(ins)[0]
    fused.close()
    assert_parity(got, want, f"conv{k}+clip")
    monkeypatch.setenv("MLVC_HIP_DISABLE_FUSION", "1")
    plain = mlvc_hip.Backend(tmp_path, "hip")
    plain.load("m")
    ref = plain.run(ins)[0]
    plain.close()
    assert (got == ref).all()



def test_fill_pattern():
    """The load-time tuner's operand pattern: FP16 values with |v| in [0.5, 1),
    both signs, deterministic in the seed, different across seeds, zeros
    nowhere (the tuner times kernels on it instead of zeroed buffers)."""
    import ctypes as C

    from devmem import Dev

    dev = Dev()
    try:
        L = dev.lib
        L.mlvc_hip_fill_pattern.argtypes = [C.c_void_p, C.c_size_t, C.c_uint, C.c_void_p]
        n = (1 << 20) + 3
        bufs = [dev.alloc(2 * n) for _ in range(3)]
        for p, seed in zip(bufs, (7, 7, 8)):
            dev.check(L.mlvc_hip_fill_pattern(p, 2 * n, seed, None))
        a, b, c = (dev.get(p, (n,), np.uint16) for p in bufs)
        v = a.view(np.float16).astype(np.float32)
        assert np.isfinite(v).all() and (np.abs(v) >= 0.5).all() and (np.abs(v) < 1.0).all()
        assert 0.45 < (v < 0).mean() < 0.55
        assert (a == b).all() and (a != c).mean() > 0.9
        assert len(np.unique(a)) > 1500  # sign x 1024 mantissas, spread over them
        dev.check(L.mlvc_hip_fill_pattern(bufs[0], 0, 1, None))  # empty fill is allowed
        assert L.mlvc_hip_fill_pattern(bufs[0], 3, 1, None) != 0  # odd byte count rejected
    finally:
        dev.close()
