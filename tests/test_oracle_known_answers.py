"""Graph-level pins of the CPU oracle, independent of the reference build.

* Closed-form known answers modelled on the reference's
  tests/unit/cpu_backend_tests.cpp:437-594 (depthwise centre + top-left taps,
  identity 1x1 + LeakyReLU, residual ADD, 3x3 centre tap, wide OC=128 1x1 +
  residual, stride-2 3x3 with taps (0,2) and (2,0)), same input formula and
  tolerances.
* Small-channel layout round trip C=3 and C=11 (cpu_backend_tests.cpp:796-864).
* The CRD pixel shuffle index formula for blocks 2 and 8
  (tests/unit/cutlass_kernel_tests.cpp:43-89) against numpy reshapes, and the
  SPACE_TO_DEPTH -> DEPTH_TO_SPACE round trip.
* Brute-force float64 direct convolution (numpy) for conv + epilogues.
* Fused vs unfused schedules, 1 vs N threads and reset_state determinism
  (cpu_backend_tests.cpp:596-661, 663-794).
"""

import numpy as np
import pytest

import graphs
import mlvc_hip
import mlvc_oracle


def run_oracle(d, inputs, **kw):
    return mlvc_oracle.OraclePlan(d, "m", **kw).run(inputs)


def test_conv_epilogue_known_answers(tmp_path):
    H, W, IC = 4, 5, 16
    g = graphs.Graph()
    x = g.input("x", [1, IC, H, W])
    wdw = np.zeros((16, 1, 3, 3))
    wdw[:, 0, 1, 1] = 1.0
    wdw[:, 0, 0, 0] = 0.25
    dw = g.conv("dw", x, g.weight_fp16("wdw", wdw), g.weight_fp16("bdw", np.full(16, 0.1)), (1, 1), (1, 1, 1, 1), 16)
    eye = np.eye(16).reshape(16, 16, 1, 1)
    c2 = g.conv("c2", dw, g.weight_fp16("w2", eye), 0, (1, 1), (0, 0, 0, 0))
    lr = g.leaky_relu("lrelu", c2, 0.01)
    c3 = g.conv("c3", lr, g.weight_fp16("w2b", eye), 0, (1, 1), (0, 0, 0, 0))
    res = g.binary("ADD", "res", c3, x)
    w3 = np.zeros((16, 16, 3, 3))
    for c in range(16):
        w3[c, c, 1, 1] = 0.5
    sp = g.conv("sp3", res, g.weight_fp16("w3", w3), 0, (1, 1), (1, 1, 1, 1))
    rw = g.input("res_wide", [1, 128, H, W])
    ww = np.zeros((128, 16, 1, 1))
    for oc in range(128):
        ww[oc, oc % 16] = 0.25
    cw = g.conv("c_wide", sp, g.weight_fp16("ww", ww), 0, (1, 1), (0, 0, 0, 0))
    wide = g.binary("ADD", "wide", cw, rw)
    ws2 = np.zeros((16, 16, 3, 3))
    for c in range(16):
        ws2[c, c, 0, 2] = 0.25
        ws2[c, c, 2, 0] = 0.5
    s2 = g.conv("s2", sp, g.weight_fp16("ws2", ws2), 0, (2, 2), (1, 1, 1, 1))
    for t in (sp, wide, s2):
        g.output(t)
    g.write(tmp_path, "m")

    xv = ((np.arange(IC * H * W) % 13) - 6) * 0.25
    rv = ((np.arange(128 * H * W) % 19) - 9) * 0.125
    xh, rh = graphs.half(xv), graphs.half(rv)
    outs = mlvc_oracle.OraclePlan(tmp_path, "m", num_threads=4).run([xh.reshape(1, IC, H, W), rh.reshape(1, 128, H, W)])
    xf = graphs.to_float(xh).reshape(IC, H, W).astype(np.float64)
    dwv = 0.1 + xf.copy()
    dwv[:, 1:, 1:] += 0.25 * xf[:, :-1, :-1]
    lrv = np.where(dwv < 0, dwv * 0.01, dwv)
    spv = 0.5 * (lrv + xf)
    np.testing.assert_allclose(graphs.to_float(outs[0]).reshape(IC, H, W), spv, atol=2e-2)
    widev = 0.25 * spv[np.arange(128) % 16] + graphs.to_float(rh).reshape(128, H, W)
    np.testing.assert_allclose(graphs.to_float(outs[1]).reshape(128, H, W), widev, atol=2e-2)
    s2v = np.zeros((16, 2, 3))
    for oy in range(2):
        for ox in range(3):
            iy, ix = oy * 2 - 1, ox * 2 + 1
            if 0 <= iy < H and 0 <= ix < W:
                s2v[:, oy, ox] += 0.25 * spv[:, iy, ix]
            iy, ix = oy * 2 + 1, ox * 2 - 1
            if 0 <= iy < H and 0 <= ix < W:
                s2v[:, oy, ox] += 0.5 * spv[:, iy, ix]
    np.testing.assert_allclose(graphs.to_float(outs[2]).reshape(16, 2, 3), s2v, atol=2e-2)


@pytest.mark.parametrize("c,h,w", [(3, 9, 11), (11, 5, 7)])
def test_small_channel_layout_roundtrip(tmp_path, c, h, w):
    g = graphs.Graph()
    x = g.input("x", [1, c, h, w])
    b = (0.5 + 0.25 * np.arange(c)) if c == 3 else (-0.25 * np.arange(c))
    y = g.conv("y", x, g.weight_fp16("w", np.eye(c).reshape(c, c, 1, 1)), g.weight_fp16("b", b), (1, 1), (0, 0, 0, 0))
    g.output(y)
    g.write(tmp_path, "m")
    hw = h * w
    idx = np.arange(c * hw).reshape(c, hw)
    ch = idx // hw
    s = idx % hw
    xv = (0.01 * ((ch * 31 + s) % 40) - 0.1) if c == 3 else (0.02 * ((ch * 17 + s) % 25) - 0.2)
    out = run_oracle(tmp_path, [graphs.half(xv).reshape(1, c, h, w)], num_threads=4)[0]
    want = graphs.to_float(graphs.half(xv)) + b[:, None]
    np.testing.assert_allclose(graphs.to_float(out).reshape(c, hw), want, atol=5e-3)


@pytest.mark.parametrize("block", [2, 8])
def test_pixel_shuffle_index_formula(tmp_path, block):
    c_out, h, w = 3, 2, 3
    c_in = c_out * block * block
    g = graphs.Graph()
    x = g.input("x", [1, c_in, h, w])
    d2s = g.pixel("DEPTH_TO_SPACE", "d2s", x, block)
    back = g.pixel("SPACE_TO_DEPTH", "s2d", d2s, block)
    g.output(d2s)
    g.output(back)
    g.write(tmp_path, "m")
    vals = np.arange(c_in * h * w, dtype=np.float32) % 2048  # exact in fp16
    xh = graphs.half(vals).reshape(1, c_in, h, w)
    d, b = run_oracle(tmp_path, [xh])
    # out[c, y*b+dy, x*b+dx] = in[c*b*b + dy*b + dx, y, x]
    want = xh.reshape(c_out, block, block, h, w).transpose(0, 3, 1, 4, 2).reshape(1, c_out, h * block, w * block)
    assert (d == want).all()
    for c in range(c_out):
        for y in range(h):
            for xx in range(w):
                for dy in range(block):
                    for dx in range(block):
                        assert d[0, c, y * block + dy, xx * block + dx] == xh[0, c * block * block + dy * block + dx, y, xx]
    assert (b == xh).all()


def direct_conv64(x, w, b, stride, pad):
    """Float64 direct convolution of fp16-valued tensors (NCHW, groups 1)."""
    n, ic, h, wd = x.shape
    oc, _, kh, kw = w.shape
    xp = np.zeros((n, ic, h + 2 * pad, wd + 2 * pad))
    xp[:, :, pad:pad + h, pad:pad + wd] = x
    oh, ow = (h + 2 * pad - kh) // stride + 1, (wd + 2 * pad - kw) // stride + 1
    y = np.zeros((n, oc, oh, ow)) + b[None, :, None, None]
    for ky in range(kh):
        for kx in range(kw):
            patch = xp[:, :, ky:ky + stride * oh:stride, kx:kx + stride * ow:stride]
            y += np.einsum("nchw,oc->nohw", patch, w[:, :, ky, kx])
    return y


@pytest.mark.parametrize("ic,oc,k,s,p,epi", [(16, 32, 3, 1, 1, "lrelu"), (12, 20, 3, 2, 1, None), (40, 24, 1, 1, 0, "lrelu"),
                                             (7, 5, 3, 1, 1, None)])
def test_conv_against_float64_brute_force(tmp_path, ic, oc, k, s, p, epi):
    n, h, w = 1, 9, 13
    graphs.single_conv_graph(tmp_path, "m", n, ic, h, w, oc, k, s, p, epilogue=epi, seed=ic + oc)
    rng = np.random.default_rng(ic + oc)  # same stream as single_conv_graph
    std = 1.0 / np.sqrt(ic * k * k)
    wt = graphs.to_float(graphs.half(rng.normal(0, std, (oc, ic, k, k)))).astype(np.float64)
    bt = graphs.to_float(graphs.half(rng.normal(0, 0.1, (oc,)))).astype(np.float64)
    xin = graphs.half(np.random.default_rng(1).uniform(-1, 1, (n, ic, h, w)))
    got = graphs.to_float(run_oracle(tmp_path, [xin])[0]).astype(np.float64)
    y = direct_conv64(graphs.to_float(xin).astype(np.float64), wt, bt, s, p)
    y = graphs.to_float(graphs.half(y)).astype(np.float64)
    if epi == "lrelu":
        y = np.where(y < 0, y * 0.01, y)
    rms = np.sqrt(np.mean(y * y))
    assert np.abs(got - y).max() <= 1e-2 * rms
    assert np.abs(got - y).mean() <= 1e-3 * rms


@pytest.fixture(scope="module")
def tiny_model(tmp_path_factory):
    d = tmp_path_factory.mktemp("mlvc_s_tiny")
    mlvc_hip.synth_write("mlvc_s_tiny", d, 0)
    bindings, _ = mlvc_hip.synth_bindings("mlvc_s_tiny")
    return d, bindings


def _frames(d, bindings, frames=3, **kw):
    p = mlvc_oracle.OraclePlan(d, "mlvc_s_tiny", bindings, **kw)
    p.reset_state()
    return [p.run([mlvc_hip.synth_input("mlvc_s_tiny", 0, f, p.in_shapes[0])])[0] for f in range(frames)]


def test_fused_vs_unfused_and_threads_bit_identical(tiny_model):
    d, bindings = tiny_model
    fused = _frames(d, bindings, num_threads=4)
    unfused = _frames(d, bindings, num_threads=4, fusion=False)
    single = _frames(d, bindings, num_threads=1)
    for a, b, c in zip(fused, unfused, single):
        assert (a == b).all() and (a == c).all()


def test_state_semantics(tiny_model):
    d, bindings = tiny_model
    p = mlvc_oracle.OraclePlan(d, "mlvc_s_tiny", bindings)
    x = mlvc_hip.synth_input("mlvc_s_tiny", 0, 0, p.in_shapes[0])
    with pytest.raises(mlvc_oracle.OracleError, match="reset_state"):
        p.run([x])
    p.reset_state()
    f1 = p.run([x])[0]
    f2 = p.run([x])[0]
    assert not (f1 == f2).all()  # the carried reference changes frame 2
    p.reset_state()
    assert (p.run([x])[0] == f1).all()
    assert len(p.out_shapes) == 1 and len(p.in_shapes) == 1  # bound tensors leave run()'s lists


def test_scalar_isa_within_tolerance_of_avx2(tiny_model):
    d, bindings = tiny_model
    a = _frames(d, bindings, isa=0)
    b = _frames(d, bindings, isa=1)
    for x, y in zip(a, b):
        st = mlvc_oracle.parity_stats(x, y)
        assert st["max_rel"] <= 5e-3, st
