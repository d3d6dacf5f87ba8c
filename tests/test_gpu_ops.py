"""GPU parity of the real-model operators and fused kernels (CLIP, SIGMOID,
RECIPROCAL, ROUND, broadcast ADD/SUB/MUL, SLICE, CONCAT, GATHER, ReGLU,
recurrent feature update, y0/y1 quantisation tails).

Kernel level, through the device C ABI: bit-exact against the oracle's
restatement (itself pinned bit-exact against the reference CPU kernels and
numpy semantics in test_oracle_ops.py), on NCHW buffers, with plane sizes on
and off the 16-byte vector path.

Graph level, through the backend C ABI: the operator zoo graph (no convs) is
bit-exact against the oracle; the real-model pattern graphs (convs around
the fused chains, recurrent state) meet the FP16 parity bar frame after frame
and are bit-identical between the fused and unfused GPU schedules.
"""

import ctypes as C

import numpy as np
import pytest

import mlvc_hip
import mlvc_oracle as O
from conftest import assert_parity
from devmem import Dev

pytestmark = pytest.mark.gpu

UNARY = {"clip": 0, "sigmoid": 1, "reciprocal": 2, "round": 3}
BINARY = {"add": 0, "sub": 1, "mul": 2}
_i64x4 = C.c_int64 * 4


class OpsDev(Dev):
    def __init__(self):
        super().__init__()
        L = self.lib
        vp, sz = C.c_void_p, C.c_size_t
        L.mlvc_hip_unary.argtypes = [vp, vp, sz, C.c_int, C.c_float, C.c_float, vp]
        L.mlvc_hip_binary.argtypes = [vp, C.POINTER(C.c_int64), vp, C.POINTER(C.c_int64), vp, C.POINTER(C.c_int64), C.c_int, vp]
        L.mlvc_hip_slice.argtypes = [vp, C.POINTER(C.c_int64), vp, C.POINTER(C.c_int64), C.POINTER(C.c_int64),
                                     C.POINTER(C.c_int64), vp]
        L.mlvc_hip_copy_rows.argtypes = [vp, vp, sz, sz, sz, sz, vp]
        L.mlvc_hip_gather.argtypes = [vp, vp, C.c_int, sz, sz, sz, sz, vp, vp]
        L.mlvc_hip_reglu.argtypes = [vp, vp, C.c_int, C.c_int, sz, C.c_float, C.c_float, vp]
        L.mlvc_hip_feature_update.argtypes = [vp] * 6 + [C.c_int, C.c_int, sz, vp]

    def get16(self, p, shape):
        return self.get(p, shape, np.uint16)


class Y0Desc(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("latent", "prior", "quant_scale", "update_scale0", "update_scale1", "normalized",
                                          "clipped", "y_raw", "concat2", "concat3")] + \
               [("n", C.c_int), ("q", C.c_int), ("hw", C.c_size_t), ("clip_min", C.c_float)]


class Y1Desc(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("normalized", "prior", "quant_scale", "update_scale0", "update_scale1", "concat2",
                                          "clipped", "y_raw", "out")] + [("n", C.c_int), ("q", C.c_int), ("hw", C.c_size_t)]


@pytest.fixture
def dev():
    d = OpsDev()
    yield d
    d.close()


def f16(a):
    return np.asarray(a, np.float32).astype(np.float16).view(np.uint16)


def rand16(rng, shape, lo=-4.0, hi=4.0):
    return f16(rng.uniform(lo, hi, shape))


def to_nhwc(x):
    """[C, HW] planes (N=1) -> the reference kernels' [HW, C] rows."""
    return np.ascontiguousarray(x.reshape(x.shape[0], -1).T).reshape(-1)


def from_nhwc(buf, c):
    return np.ascontiguousarray(buf.reshape(-1, c).T)


# ------------------------------------------------------------------ unary

UNARY_CASES = [("clip", -1.0, 1.0), ("clip", 0.0, np.inf), ("clip", -np.inf, 6.0), ("clip", 2.0, -2.0),
               ("sigmoid", 0, 0), ("reciprocal", 0, 0), ("round", 0, 0)]


@pytest.mark.parametrize("case", UNARY_CASES, ids=[f"{c[0]}_{c[1]}_{c[2]}" for c in UNARY_CASES])
def test_unary_every_half(dev, case):
    op, lo, hi = case
    # All 65536 bit patterns, NaNs and infinities included, plus 3 more so
    # the last group of 8 is partial.
    x = np.concatenate([np.arange(65536, dtype=np.uint32).astype(np.uint16), f16([0.5, -2.5, 3.5])])
    want = O.Ops().unary(np.concatenate([x, np.zeros(5, np.uint16)]), op, lo, hi, 0)[: x.size]
    px, py = dev.put(x), dev.alloc(x.nbytes)
    dev.check(dev.lib.mlvc_hip_unary(px, py, x.size, UNARY[op], lo, hi, None))
    assert np.array_equal(dev.get16(py, x.shape), want)


# ----------------------------------------------------------------- binary

NP_OP = {"add": np.add, "sub": np.subtract, "mul": np.multiply}
BCAST = [([1, 24, 12, 20], [1, 24, 12, 20]), ([1, 24, 12, 20], [1, 1, 1, 1]), ([1, 1, 1, 1], [1, 24, 12, 20]),
         ([1, 24, 12, 20], [1, 24, 1, 1]), ([1, 24, 1, 1], [1, 24, 12, 20]), ([2, 8, 5, 6], [1, 1, 5, 6]),
         ([1, 8, 1, 6], [3, 8, 5, 1]), ([2, 8, 5, 7], [2, 1, 1, 1]), ([1, 1, 1, 7], [4, 3, 2, 7]),
         # W a multiple of 8: the 16-byte row path (full / broadcast operands).
         ([1, 24, 12, 24], [1, 24, 1, 1]), ([1, 1, 1, 1], [1, 8, 3, 16]), ([2, 8, 5, 16], [1, 1, 5, 16]),
         ([1, 8, 1, 16], [3, 8, 5, 1]), ([2, 8, 5, 16], [2, 8, 5, 16])]


@pytest.mark.parametrize("op", ["add", "sub", "mul"])
@pytest.mark.parametrize("shapes", BCAST, ids=[f"{a}x{b}" for a, b in BCAST])
def test_binary_broadcast(dev, shapes, op):
    sa, sb = shapes
    rng = np.random.default_rng(len(sa) + sum(sb))
    a = rng.uniform(-300, 300, sa).astype(np.float16)
    b = rng.uniform(-3, 3, sb).astype(np.float16)
    want = NP_OP[op](a.astype(np.float32), b.astype(np.float32)).astype(np.float16)
    pa, pb, py = dev.put(a.view(np.uint16)), dev.put(b.view(np.uint16)), dev.alloc(want.nbytes)
    dev.check(dev.lib.mlvc_hip_binary(pa, _i64x4(*sa), pb, _i64x4(*sb), py, _i64x4(*want.shape), BINARY[op], None))
    assert np.array_equal(dev.get16(py, want.shape), want.view(np.uint16))


def test_binary_rejects_bad_broadcast(dev):
    p = dev.alloc(64)
    with pytest.raises(mlvc_hip.MlvcError, match="broadcast"):
        dev.check(dev.lib.mlvc_hip_binary(p, _i64x4(1, 2, 1, 1), p, _i64x4(1, 3, 1, 1), p, _i64x4(1, 3, 1, 1), 0, None))


# ------------------------------------------------------------ slice/concat

SLICES = [([1, 12, 6, 10], [1, 4, 6, 10], [0, 4, 0, 0], [1, 1, 1, 1]),
          ([1, 12, 6, 10], [1, 12, 3, 10], [0, 0, 2, 0], [1, 1, 1, 1]),
          ([2, 12, 6, 10], [2, 5, 3, 4], [0, 1, 1, 3], [1, 2, 2, 1]),
          ([2, 6, 8, 9], [1, 6, 4, 3], [1, 0, 7, 8], [1, 1, -2, -3]),
          ([1, 32, 16, 24], [1, 16, 16, 24], [0, 16, 0, 0], [1, 1, 1, 1]),
          ([2, 4, 6, 32], [1, 4, 3, 16], [1, 0, 1, 8], [1, 1, 2, 1])]


@pytest.mark.parametrize("case", SLICES, ids=[str(i) for i in range(len(SLICES))])
def test_slice(dev, case):
    id4, od4, starts, steps = case
    x = np.random.default_rng(sum(id4)).uniform(-2, 2, id4).astype(np.float16).view(np.uint16)
    want = x[np.ix_(*[np.arange(od4[d]) * steps[d] + starts[d] for d in range(4)])]
    px, py = dev.put(x), dev.alloc(want.nbytes)
    dev.check(dev.lib.mlvc_hip_slice(px, _i64x4(*id4), py, _i64x4(*od4), _i64x4(*starts), _i64x4(*steps), None))
    assert np.array_equal(dev.get16(py, od4), want)


def test_slice_rejects_reads_outside(dev):
    p = dev.alloc(1024)
    with pytest.raises(mlvc_hip.MlvcError, match="outside"):
        dev.check(dev.lib.mlvc_hip_slice(p, _i64x4(1, 4, 4, 4), p, _i64x4(1, 4, 4, 3), _i64x4(0, 0, 0, 2), _i64x4(1, 1, 1, 1), None))


CONCATS = [(1, [[1, 3, 4, 5], [1, 5, 4, 5]]), (1, [[2, 8, 4, 4], [2, 16, 4, 4], [2, 8, 4, 4]]),
           (2, [[1, 6, 2, 5], [1, 6, 3, 5]]), (3, [[2, 6, 3, 2], [2, 6, 3, 4]]), (0, [[1, 6, 3, 4], [2, 6, 3, 4]])]


@pytest.mark.parametrize("case", CONCATS, ids=[str(i) for i in range(len(CONCATS))])
def test_concat_pieces(dev, case):
    # One block copy per input, as the backend lowers CONCAT.
    axis, dims = case
    rng = np.random.default_rng(axis)
    xs = [rng.uniform(-2, 2, d).astype(np.float16).view(np.uint16) for d in dims]
    want = np.concatenate(xs, axis=axis)
    after = int(np.prod(want.shape[axis + 1:]))
    rows = int(np.prod(want.shape[:axis]))
    py = dev.alloc(want.nbytes)
    off = 0
    for x in xs:
        row = x.shape[axis] * after
        dev.check(dev.lib.mlvc_hip_copy_rows(dev.put(x), C.c_void_p(py.value + 2 * off * after), rows, row, row,
                                             want.shape[axis] * after, None))
        off += x.shape[axis]
    assert np.array_equal(dev.get16(py, want.shape), want)


# ----------------------------------------------------------------- gather

GATHERS = [([72, 24, 1, 1], 0, [5]), ([72, 16, 1, 1], 0, [-1, 3]), ([2, 12, 5, 8], 1, [3, 0, 11]), ([2, 12, 5, 6], 2, [4]),
           ([2, 12, 5, 6], 3, [0, 5, -2]), ([7, 9], 1, [8, 0])]


@pytest.mark.parametrize("dtype", [np.int32, np.int64])
@pytest.mark.parametrize("case", GATHERS, ids=[str(i) for i in range(len(GATHERS))])
def test_gather(dev, case, dtype):
    shape, axis, idx = case
    x = np.random.default_rng(axis).uniform(-2, 2, shape).astype(np.float16).view(np.uint16)
    want = np.take(x, np.asarray(idx), axis=axis)
    outer, inner = int(np.prod(shape[:axis])), int(np.prod(shape[axis + 1:]))
    py = dev.alloc(want.nbytes)
    dev.check(dev.lib.mlvc_hip_gather(dev.put(x), dev.put(np.asarray(idx, dtype)), int(dtype == np.int64), len(idx), outer,
                                      shape[axis], inner, py, None))
    assert np.array_equal(dev.get16(py, want.shape), want)


# ---------------------------------------------------------- fused kernels

@pytest.mark.parametrize("hw", [16 * 24, 10 * 14])
@pytest.mark.parametrize("g", [32, 12])
def test_reglu(dev, g, hw):
    rng = np.random.default_rng(g + hw)
    x = rand16(rng, (2 * g, hw), -8, 8)
    want = from_nhwc(O.Ops().reglu(to_nhwc(x), hw, g, -1.0, 6.0), g)
    py = dev.alloc(g * hw * 2)
    dev.check(dev.lib.mlvc_hip_reglu(dev.put(x), py, 1, g, hw, -1.0, 6.0, None))
    assert np.array_equal(dev.get16(py, (g, hw)), want)


@pytest.mark.parametrize("outputs", [False, True])
@pytest.mark.parametrize("hw", [16 * 24, 10 * 14])
@pytest.mark.parametrize("ch", [32, 16])
def test_feature_update(dev, ch, hw, outputs):
    rng = np.random.default_rng(ch + hw)
    x = rand16(rng, (3 * ch, hw), -6, 6)
    hist = rand16(rng, (ch, hw), -2, 2)
    scale = rand16(rng, ch, 0.5, 1.5)
    want = O.Ops().feature_update(to_nhwc(x), to_nhwc(hist), scale, hw, ch, outputs=True)
    feat = dev.alloc(2 * ch * hw * 2)
    sc = dev.alloc(ch * hw * 2) if outputs else None
    bl = dev.alloc(ch * hw * 2) if outputs else None
    dev.check(dev.lib.mlvc_hip_feature_update(dev.put(x), dev.put(hist), dev.put(scale), feat, sc, bl, 1, ch, hw, None))
    assert np.array_equal(dev.get16(feat, (2 * ch, hw)), from_nhwc(want[0], 2 * ch))
    if outputs:
        assert np.array_equal(dev.get16(sc, (ch, hw)), from_nhwc(want[1], ch))
        assert np.array_equal(dev.get16(bl, (ch, hw)), from_nhwc(want[2], ch))


def test_feature_update_every_gate(dev):
    """Both gates of the feature update take every non-NaN FP16 value (the
    kernel reads most of them from its table, the rest through the
    arithmetic path), bit for bit against the oracle."""
    ch, hw = 16, 4096
    rng = np.random.default_rng(11)
    allh = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    allh = np.where(np.isnan(allh.view(np.float16)), np.uint16(0), allh).astype(np.uint16)
    x = np.concatenate([rand16(rng, (ch, hw), -4, 4), allh.reshape(ch, hw), rng.permutation(allh).reshape(ch, hw)])
    hist = rand16(rng, (ch, hw), -2, 2)
    scale = rand16(rng, ch, 0.5, 1.5)
    want = O.Ops().feature_update(to_nhwc(x), to_nhwc(hist), scale, hw, ch, outputs=True)
    feat = dev.alloc(2 * ch * hw * 2)
    dev.check(dev.lib.mlvc_hip_feature_update(dev.put(x), dev.put(hist), dev.put(scale), feat, None, None, 1, ch, hw, None))
    got, ref = dev.get16(feat, (2 * ch, hw)), from_nhwc(want[0], 2 * ch)
    same = (got == ref) | (np.isnan(got.view(np.float16)) & np.isnan(ref.view(np.float16)))
    bad = np.argwhere(~same)
    assert bad.size == 0, f"{len(bad)} values differ, first at {bad[:4].tolist()}"


@pytest.mark.parametrize("hw", [8 * 12, 5 * 7])
@pytest.mark.parametrize("q", [16, 8])
def test_quant_tails(dev, q, hw):
    rng = np.random.default_rng(q + hw)
    latent = rand16(rng, (2 * q, hw), -20, 20)
    prior = np.concatenate([rand16(rng, (2 * q, hw), -0.5, 3), rand16(rng, (2 * q, hw), -4, 4)])
    qs = rand16(rng, (2 * q, hw), 0.5, 2)
    us0, us1 = rand16(rng, (q, hw), 0.5, 1.5), rand16(rng, (q, hw), 0.5, 1.5)
    want0 = O.Ops().y0_tail(*[to_nhwc(a) for a in (latent, prior, qs, us0, us1)], 0.11, hw, q)
    outs = [dev.alloc(c * hw * 2) for c in (2 * q, 2 * q, q, 2 * q, 6 * q)]
    d = Y0Desc(*[dev.put(a).value for a in (latent, prior, qs, us0, us1)], *[o.value for o in outs], 1, q, hw, 0.11)
    dev.check(dev.lib.mlvc_hip_y0_tail(C.byref(d), None))
    got0 = [dev.get16(o, (c, hw)) for o, c in zip(outs, (2 * q, 2 * q, q, 2 * q, 6 * q))]
    for g, w, c in zip(got0, want0, (2 * q, 2 * q, q, 2 * q, 6 * q)):
        assert np.array_equal(g, from_nhwc(w, c))
    normalized, clipped, _, concat2, _ = got0
    prior1 = rand16(rng, (2 * q, hw), -4, 4)
    want1 = O.Ops().y1_tail(*[to_nhwc(a) for a in (normalized, prior1, qs, us0, us1, concat2, clipped)], hw, q)
    o1 = [dev.alloc(q * hw * 2), dev.alloc(2 * q * hw * 2)]
    d1 = Y1Desc(*[dev.put(a).value for a in (normalized, prior1, qs, us0, us1, concat2, clipped)], *[o.value for o in o1], 1, q, hw)
    dev.check(dev.lib.mlvc_hip_y1_tail(C.byref(d1), None))
    assert np.array_equal(dev.get16(o1[0], (q, hw)), from_nhwc(want1[0], q))
    assert np.array_equal(dev.get16(o1[1], (2 * q, hw)), from_nhwc(want1[1], 2 * q))


# ------------------------------------------------------------ graph level

def _inputs(shapes, rng, frame):
    ins = []
    for s in shapes:
        if tuple(s) == (1,):
            ins.append(np.array([(7 * frame + 5) % 72], np.int32))
        else:
            ins.append(rng.uniform(-1, 1, s).astype(np.float16).view(np.uint16))
    return ins


def test_ops_zoo_bit_exact(tmp_path, monkeypatch):
    cfg = "ops_zoo_tiny"
    mlvc_hip.synth_write(cfg, tmp_path, 0)
    ref = O.OraclePlan(tmp_path, cfg)
    rng = np.random.default_rng(3)
    ins = _inputs(ref.in_shapes, rng, 0)
    want = ref.run(ins)
    for fused in ("0", "1"):
        monkeypatch.setenv("MLVC_HIP_DISABLE_FUSION", "1" if fused == "0" else "0")
        with mlvc_hip.Backend(tmp_path, "hip") as gpu:
            gpu.load(cfg)
            got = gpu.run(ins)
            assert len(got) == len(want)
            for i, (g, w) in enumerate(zip(got, want)):
                assert np.array_equal(g, w), f"output {i} (fusion {fused})"
            # A row index past the table is rejected before any launch.
            bad = list(ins)
            bad[1] = np.array([72], np.int32)
            with pytest.raises(mlvc_hip.MlvcError, match="GATHER index out of range"):
                gpu.run(bad)
            bad[1] = np.array([-1], np.int32)  # counts from the end
            assert all(np.array_equal(g, w) for g, w in zip(gpu.run(bad), ref.run(bad)))


def _product_close(g, w, what):
    # Outputs formed by products of conv results (ReGLU, the feature update,
    # normalisation). The conv results meet the bar (|d| <= 1e-2 of their
    # RMS), and a product a*b carries |b|*|da|: its RMS is below its
    # factors', so the same absolute error is a larger share of it. The bar
    # for these outputs is |d| <= 5e-2 of their RMS; the mean bar is kept.
    # (The kernels themselves are checked bit for bit above and by the
    # chained ReGLU check.)
    st = O.parity_stats(g, w)
    assert st["finite"] and st["mean_rel"] <= 1e-3 and st["max_rel"] <= 5e-2, f"{what}: {st}"


def _quantised_close(g, w, what):
    # Outputs downstream of ROUND: conv results upstream differ from the
    # oracle's in the last FP16 bits (accumulation order), which moves a few
    # values across a rounding edge; everything else stays within the bar.
    gf, wf = g.view(np.float16).astype(np.float64), w.view(np.float16).astype(np.float64)
    assert np.isfinite(gf).all() and np.isfinite(wf).all(), f"{what}: non-finite values"
    rms = float(np.sqrt(np.mean(wf * wf))) or 1.0
    off = np.abs(gf - wf) > 1e-2 * rms
    assert off.mean() < 0.05, f"{what}: {off.mean():.4f} of values off"


@pytest.mark.parametrize("cfg", ["fused_tiny", "fused_odd_tiny"])
def test_fused_patterns_on_graph_inputs(tmp_path, monkeypatch, cfg):
    # Every fused chain fed straight from graph inputs: identical operands on
    # both sides, so the GPU equals the oracle bit for bit (fused_odd_tiny's
    # 13-channel feature update takes the reference's scalar exp for
    # channels 8..12, one FP16 ulp apart at most from the vector form the
    # GPU uses everywhere).
    mlvc_hip.synth_write(cfg, tmp_path, 0)
    ref = O.OraclePlan(tmp_path, cfg)
    assert ref.steps == 6
    rng = np.random.default_rng(8)
    ins = [rng.uniform(-2, 2, s).astype(np.float16).view(np.uint16) for s in ref.in_shapes]
    want = ref.run(ins)
    for flag in ("0", "1"):
        monkeypatch.setenv("MLVC_HIP_DISABLE_FUSION", flag)
        with mlvc_hip.Backend(tmp_path, "hip") as gpu:
            gpu.load(cfg)
            if flag == "0":
                kinds = sorted(l["kind"] for l in gpu.launches())
                assert kinds == sorted(["reglu", "feature_update", "leaky_relu", "feature_update_outputs", "y0_tail", "y1_tail"])
            got = gpu.run(ins)
            for i, (g, w) in enumerate(zip(got, want)):
                if cfg == "fused_tiny":
                    assert np.array_equal(g, w), f"output {i} (fusion off: {flag})"
                else:
                    assert np.mean(g != w) < 0.02, f"output {i}"
                    if i not in (5, 6, 7, 8):
                        assert_parity(g, w, f"output {i}")


def _check_realops(got, want, what):
    """Outputs of the realops graphs: rin (a conv) to the FP16 bar; rout =
    ReGLU(rin) and between = LeakyReLU(rout) bit for bit against the oracle's
    kernels applied to the GPU's own rin, plus the mean bar; the feature
    update and normalised latent to the product bar; the outputs downstream
    of ROUND to the quantised bar."""
    rin = got[0].reshape(got[0].shape[1], -1)
    g, hw = rin.shape[0] // 2, rin.shape[1]
    rout = O.Ops().reglu(np.ascontiguousarray(rin.T).reshape(-1), hw, g, -1.0, 6.0)
    assert np.array_equal(got[1].reshape(g, hw), rout.reshape(hw, g).T), f"{what}: ReGLU of the GPU's rin"
    between = O.Kernels().leaky_relu(np.ascontiguousarray(got[1]).reshape(-1), 0.01)
    assert np.array_equal(got[2].reshape(-1), between), f"{what}: LeakyReLU of the GPU's ReGLU"
    for i, (gg, w) in enumerate(zip(got, want)):
        if i == 0:
            assert_parity(gg, w, f"{what} output {i}")
        elif i < 5:
            _product_close(gg, w, f"{what} output {i}")
        else:
            _quantised_close(gg, w, f"{what} output {i}")


@pytest.mark.parametrize("cfg", ["realops_tiny", "realops_odd_tiny"])
def test_realops_recurrent(tmp_path, cfg):
    mlvc_hip.synth_write(cfg, tmp_path, 0)
    bindings, frames = mlvc_hip.synth_bindings(cfg)
    ref = O.OraclePlan(tmp_path, cfg, bindings)
    with mlvc_hip.Backend(tmp_path, "hip") as gpu:
        gpu.load(cfg, bindings)
        kinds = [l["kind"] for l in gpu.launches()]
        for k in ("y0_tail", "y1_tail", "feature_update", "feature_update_outputs", "reglu", "gather"):
            assert k in kinds, (k, kinds)
        # The FFN's 1x1 conv takes its ReGLU as an epilogue; the ReGLU of rin
        # (a graph output) stays a kernel of its own.
        assert kinds.count("reglu") == 1 and sum(k.endswith("+reglu") for k in kinds) == 1, kinds
        gpu.reset_state()
        ref.reset_state()
        rng = np.random.default_rng(9)
        for f in range(frames):
            ins = _inputs(gpu.in_shapes, rng, f)
            got, want = gpu.run(ins), ref.run(ins)
            _check_realops(got, want, f"{cfg} frame {f}")


@pytest.mark.parametrize("cfg,max_frames", [("realops_tiny", 3), ("realops_odd_tiny", 2), ("realops_544x960", 2)])
def test_realops_are_the_oracle_gpu_arithmetic(tmp_path, cfg, max_frames):
    """The realops graphs, each side carrying its own recurrent state,
    against the isa-2 oracle plan (its convs summed in the matrix core's
    order, everything else as the reference plan): every output of every
    frame bit for bit, those downstream of ROUND included, so the tolerances
    against the reference order above are summation order alone."""
    mlvc_hip.synth_write(cfg, tmp_path, 0)
    bindings, frames = mlvc_hip.synth_bindings(cfg)
    frames = min(frames, max_frames)
    model = O.OraclePlan(tmp_path, cfg, bindings, isa=2)
    with mlvc_hip.Backend(tmp_path, "hip") as gpu:
        gpu.load(cfg, bindings)
        gpu.reset_state()
        model.reset_state()
        rng = np.random.default_rng(9)
        bad = []
        for f in range(frames):
            ins = _inputs(gpu.in_shapes, rng, f)
            got, want = gpu.run(ins), model.run(ins)
            for i, (g, w) in enumerate(zip(got, want)):
                n = int(np.count_nonzero(g != w))
                print(f"{cfg} frame {f} output {i}: {n} of {g.size} differ from the isa-2 oracle", flush=True)
                if n:
                    bad.append((f, i, n))
        assert not bad, bad


def test_realops_fused_and_unfused_bit_identical(tmp_path, monkeypatch):
    cfg = "realops_tiny"
    mlvc_hip.synth_write(cfg, tmp_path, 0)
    bindings, _ = mlvc_hip.synth_bindings(cfg)
    results = {}
    for flag in ("0", "1"):
        monkeypatch.setenv("MLVC_HIP_DISABLE_FUSION", flag)
        with mlvc_hip.Backend(tmp_path, "hip") as gpu:
            gpu.load(cfg, bindings)
            gpu.reset_state()
            rng = np.random.default_rng(4)
            results[flag] = [gpu.run(_inputs(gpu.in_shapes, rng, f)) for f in range(2)]
            results[flag + "n"] = len(gpu.launches())
    assert results["0n"] < results["1n"]
    for fa, fb in zip(results["0"], results["1"]):
        for a, b in zip(fa, fb):
            assert np.array_equal(a, b)


def test_realops_544x960_two_frames(tmp_path):
    cfg = "realops_544x960"
    mlvc_hip.synth_write(cfg, tmp_path, 0)
    bindings, _ = mlvc_hip.synth_bindings(cfg)
    ref = O.OraclePlan(tmp_path, cfg, bindings)
    with mlvc_hip.Backend(tmp_path, "hip") as gpu:
        gpu.load(cfg, bindings)
        gpu.reset_state()
        ref.reset_state()
        rng = np.random.default_rng(5)
        for f in range(2):
            ins = _inputs(gpu.in_shapes, rng, f)
            got, want = gpu.run(ins), ref.run(ins)
            _check_realops(got, want, f"frame {f}")
