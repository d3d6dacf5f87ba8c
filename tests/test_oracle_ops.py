"""The oracle's restatement of the real-model operators (CLIP, SIGMOID,
RECIPROCAL, ROUND, ADD/SUB/MUL with broadcasting, SLICE, CONCAT, GATHER) and
fused kernels (ReGLU, recurrent feature update, y0/y1 quantisation tails),
pinned three ways:

* bit-exact against the reference CPU kernels compiled from source
  (oracle/_ref: kernels_scalar.cpp, kernels_x86_avx2.cpp), on both ISA paths;
* against numpy semantics fixed by the mathematics where the reference code
  lives in its plan and cannot be built here (the general broadcast fallback
  and GATHER of execution_plan.cpp): numpy broadcasting / take in float32
  with one round-to-nearest-even to FP16;
* known answers (sigmoid(0) = 1/2, round half to even, 1/x of powers of two).
"""

import numpy as np
import pytest

import mlvc_oracle as O

needs_ref = pytest.mark.skipif(not O.ref_available(), reason="reference kernels not built (no checkout)")
ISAS = [0, 1]


def f16(a):
    return np.asarray(a, np.float32).astype(np.float16).view(np.uint16)


def rand16(rng, n, lo=-4.0, hi=4.0):
    return f16(rng.uniform(lo, hi, n))


def all_halves():
    return np.arange(65536, dtype=np.uint32).astype(np.uint16)


def nhwc(x):
    """Logical NCHW array -> the reference's buffer (NHWC when C > 1 and H*W > 1)."""
    x = np.asarray(x)
    if x.ndim == 4 and x.shape[1] > 1 and x.shape[2] * x.shape[3] > 1:
        return np.ascontiguousarray(x.transpose(0, 2, 3, 1)).reshape(-1)
    return np.ascontiguousarray(x).reshape(-1)


def from_nhwc(buf, shape):
    if len(shape) == 4 and shape[1] > 1 and shape[2] * shape[3] > 1:
        n, c, h, w = shape
        return buf.reshape(n, h, w, c).transpose(0, 3, 1, 2)
    return buf.reshape(shape)


# ------------------------------------------------------------------ unary

UNARY_CASES = [("clip", -1.0, 1.0), ("clip", 0.0, np.inf), ("clip", -np.inf, 6.0), ("clip", 2.0, -2.0),
               ("sigmoid", 0, 0), ("reciprocal", 0, 0), ("round", 0, 0)]


@needs_ref
@pytest.mark.parametrize("isa", ISAS)
@pytest.mark.parametrize("case", UNARY_CASES, ids=[f"{c[0]}_{c[1]}_{c[2]}" for c in UNARY_CASES])
def test_unary_every_half_matches_reference(case, isa):
    op, lo, hi = case
    x = all_halves()
    want = O.Ops("ref").unary(x, op, lo, hi, isa)
    got = O.Ops().unary(x, op, lo, hi, isa)
    assert np.array_equal(got, want)


@needs_ref
@pytest.mark.parametrize("threads", [1, 3])
@pytest.mark.parametrize("op", ["sigmoid", "clip"])
def test_unary_scalar_tail_matches_reference(op, threads):
    # 4096-element chunks, then a 5-value tail taking the scalar path.
    rng = np.random.default_rng(1)
    x = rand16(rng, 3 * 4096 + 5, -12, 12)
    x[-3] = 0x7E00  # NaN in the tail
    x[7] = 0x7E00   # NaN in a lane
    want = O.Ops("ref").unary(x, op, -0.5, 0.75, 0, threads)
    got = O.Ops().unary(x, op, -0.5, 0.75, 0)
    assert np.array_equal(got, want)


def test_unary_known_values():
    ops = O.Ops()
    x = f16([0.0, 2.5, -0.5, 3.5, 4.0, -0.25, 1000.0, -1000.0])
    assert np.array_equal(ops.unary(x[:1], "sigmoid", isa=1), f16([0.5]))
    assert np.array_equal(ops.unary(x, "sigmoid")[0:1], f16([0.5]))
    r = ops.unary(x, "round").view(np.float16)
    assert list(r[:4]) == [0.0, 2.0, -0.0, 4.0] and np.signbit(r[2])
    assert ops.unary(f16([4.0, -0.25]), "reciprocal").view(np.float16).tolist() == [0.25, -4.0]
    s = ops.unary(x, "sigmoid").view(np.float16)
    assert s[6] == 1.0 and s[7] == 0.0


def test_sigmoid_polynomial_within_one_ulp():
    # The AVX2 lanes' polynomial sigmoid against float64 sigmoid: after FP16
    # rounding they differ by at most one unit in the last place.
    x = all_halves()
    xf = x.view(np.float16).astype(np.float64)
    ok = np.isfinite(xf)
    got = O.Ops().unary(x, "sigmoid", isa=0).view(np.float16)[ok].astype(np.float64)
    with np.errstate(over="ignore"):
        exact = (1.0 / (1.0 + np.exp(-xf[ok]))).astype(np.float16).astype(np.float64)
    ulp = np.spacing(exact.astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(got - exact) <= ulp)


# ----------------------------------------------------------------- binary

@needs_ref
@pytest.mark.parametrize("isa", ISAS)
@pytest.mark.parametrize("op", ["add", "sub", "mul"])
def test_binary_kernels_match_reference(op, isa):
    rng = np.random.default_rng(2)
    a, b = rand16(rng, 1003, -300, 300), rand16(rng, 1003, -300, 300)
    a[:4] = f16([np.inf, -np.inf, 65504, 0.0])
    b[:4] = f16([1.0, np.inf, 65504, -0.0])
    ref, orc = O.Ops("ref"), O.Ops()
    assert np.array_equal(orc.binary(a, [1003], b, [1003], [1003], op), ref.binary_contiguous(a, b, op, isa))
    s = f16([1.5])[0]
    assert np.array_equal(orc.binary(a, [1003], f16([1.5]), [1], [1003], op), ref.binary_scalar(a, s, op, False, isa))
    assert np.array_equal(orc.binary(f16([1.5]), [1], a, [1003], [1003], op), ref.binary_scalar(a, s, op, True, isa))
    # Channel broadcast over an NHWC [N*H*W, C] buffer.
    shape = [1, 24, 5, 7]
    v = rand16(rng, 24 * 35)
    ch = rand16(rng, 24)
    assert np.array_equal(orc.binary(v, shape, ch, [1, 24, 1, 1], shape, op), ref.binary_channel(v, ch, 35, 24, op, False, isa))
    assert np.array_equal(orc.binary(ch, [1, 24, 1, 1], v, shape, shape, op), ref.binary_channel(v, ch, 35, 24, op, True, isa))


NP_OP = {"add": np.add, "sub": np.subtract, "mul": np.multiply}
BCAST = [
    ([2, 8, 5, 6], [1, 1, 5, 6]),
    ([2, 8, 5, 6], [2, 1, 1, 1]),
    ([1, 8, 1, 6], [3, 8, 5, 1]),
    ([2, 8, 5, 6], [6]),
    ([4, 1, 1], [2, 4, 5, 1]),
    ([2, 8, 5, 6], [1, 8, 5, 6]),
    ([5, 6], [6]),
    ([3, 4, 6], [1, 6]),
]


@pytest.mark.parametrize("op", ["add", "sub", "mul"])
@pytest.mark.parametrize("shapes", BCAST, ids=[f"{a}x{b}" for a, b in BCAST])
def test_binary_broadcast_matches_numpy(shapes, op):
    # execute_binary_broadcast_fallback_nhwc (execution_plan.cpp:170-236)
    # lives in the reference plan, which cannot be built here. Its result is
    # numpy broadcasting in float32 with one RNE rounding, on the logical
    # NCHW arrays; the buffers are the reference's NHWC re-layout.
    a_shape, b_shape = shapes
    rng = np.random.default_rng(len(a_shape) * 7 + len(b_shape))
    a = rng.uniform(-3, 3, a_shape).astype(np.float16)
    b = rng.uniform(-3, 3, b_shape).astype(np.float16)
    want = NP_OP[op](a.astype(np.float32), b.astype(np.float32)).astype(np.float16)
    for lhs_first in (True, False):
        x, y = (a, b) if lhs_first else (b, a)
        w = want if lhs_first else NP_OP[op](b.astype(np.float32), a.astype(np.float32)).astype(np.float16)
        got = O.Ops().binary(nhwc(x.view(np.uint16)), list(x.shape), nhwc(y.view(np.uint16)), list(y.shape), list(w.shape), op)
        assert np.array_equal(from_nhwc(got, w.shape), w.view(np.uint16))


def test_binary_rejects_shapes_that_do_not_broadcast():
    with pytest.raises(O.OracleError):
        O.Ops().binary(np.zeros(6, np.uint16), [6], np.zeros(4, np.uint16), [4], [6], "add")
    with pytest.raises(O.OracleError):
        O.Ops().binary(np.zeros(6, np.uint16), [6], np.zeros(6, np.uint16), [6], [2, 6], "add")


# ------------------------------------------------------------ slice/concat

SLICES = [
    # id4, od4, starts, steps
    ([1, 12, 6, 10], [1, 4, 6, 10], [0, 4, 0, 0], [1, 1, 1, 1]),   # channel slice (contiguous C fast path)
    ([1, 12, 6, 10], [1, 12, 3, 10], [0, 0, 2, 0], [1, 1, 1, 1]),  # pure H slice (block copy)
    ([2, 12, 6, 10], [2, 5, 3, 4], [0, 1, 1, 3], [1, 2, 2, 1]),    # strided channels (element loop)
    ([2, 6, 8, 9], [1, 6, 4, 3], [1, 0, 7, 8], [1, 1, -2, -3]),    # negative steps
    ([1, 3, 1, 1], [1, 2, 1, 1], [0, 1, 0, 0], [1, 1, 1, 1]),
]


@needs_ref
@pytest.mark.parametrize("case", SLICES, ids=[str(i) for i in range(len(SLICES))])
def test_slice_matches_reference_and_numpy(case):
    id4, od4, starts, steps = case
    rng = np.random.default_rng(sum(id4))
    x = rng.uniform(-2, 2, id4).astype(np.float16).view(np.uint16)
    got = O.Ops().slice(nhwc(x), id4, od4, starts, steps)
    assert np.array_equal(got, O.Ops("ref").slice(nhwc(x), id4, od4, starts, steps))
    idx = tuple(np.arange(od4[d]) * steps[d] + starts[d] for d in range(4))
    want = x[np.ix_(*idx)]
    assert np.array_equal(from_nhwc(got, od4), want)


CONCATS = [(1, [[1, 3, 4, 5], [1, 5, 4, 5]]), (1, [[2, 2, 3, 4], [2, 7, 3, 4], [2, 1, 3, 4]]), (2, [[1, 6, 2, 5], [1, 6, 3, 5]]),
           (3, [[2, 6, 3, 2], [2, 6, 3, 4]]), (0, [[1, 6, 3, 4], [2, 6, 3, 4]])]


@needs_ref
@pytest.mark.parametrize("case", CONCATS, ids=[str(i) for i in range(len(CONCATS))])
def test_concat_matches_reference_and_numpy(case):
    axis, dims = case
    rng = np.random.default_rng(axis + len(dims))
    xs = [rng.uniform(-2, 2, d).astype(np.float16).view(np.uint16) for d in dims]
    want = np.concatenate(xs, axis=axis)
    od4 = list(want.shape)
    got = O.Ops().concat([nhwc(x) for x in xs], dims, od4, axis)
    assert np.array_equal(got, O.Ops("ref").concat([nhwc(x) for x in xs], dims, od4, axis))
    assert np.array_equal(from_nhwc(got, od4), want)


# ----------------------------------------------------------------- gather

GATHERS = [([72, 16, 1, 1], 0, [5]), ([72, 16, 1, 1], 0, [-1, 3]), ([2, 12, 5, 6], 1, [3, 0, 11]), ([2, 12, 5, 6], 2, [4]),
           ([2, 12, 5, 6], 3, [0, 5, -2]), ([2, 12, 5, 6], 0, [1]), ([7, 9], 1, [8, 0]), ([7, 9], -2, [6])]


@pytest.mark.parametrize("dtype", [np.int32, np.int64])
@pytest.mark.parametrize("case", GATHERS, ids=[str(i) for i in range(len(GATHERS))])
def test_gather_matches_numpy_take(case, dtype):
    # execute_gather_general (execution_plan.cpp:101-168) lives in the
    # reference plan; its result is numpy.take on the logical array.
    shape, axis, idx = case
    rng = np.random.default_rng(len(shape) + axis)
    x = rng.uniform(-2, 2, shape).astype(np.float16).view(np.uint16)
    want = np.take(x, np.asarray(idx), axis=axis)
    got = O.Ops().gather(nhwc(x), shape, np.asarray(idx, dtype), axis)
    assert np.array_equal(from_nhwc(got, want.shape), want)


def test_gather_rejects_out_of_range_index():
    with pytest.raises(O.OracleError, match="GATHER index out of range"):
        O.Ops().gather(np.zeros(72 * 4, np.uint16), [72, 4, 1, 1], np.asarray([72], np.int32), 0)
    with pytest.raises(O.OracleError, match="GATHER axis out of range"):
        O.Ops().gather(np.zeros(72 * 4, np.uint16), [72, 4, 1, 1], np.asarray([0], np.int32), 4)


# ---------------------------------------------------------- fused kernels

@needs_ref
@pytest.mark.parametrize("isa", ISAS)
@pytest.mark.parametrize("g", [16, 12])
def test_reglu_matches_reference(g, isa):
    rng = np.random.default_rng(g)
    sp = 37
    x = rand16(rng, sp * 2 * g, -8, 8)
    for lo, hi in [(-1.0, 1.0), (0.0, 6.0), (-np.inf, np.inf)]:
        assert np.array_equal(O.Ops().reglu(x, sp, g, lo, hi, isa), O.Ops("ref").reglu(x, sp, g, lo, hi, isa))


@needs_ref
@pytest.mark.parametrize("isa", ISAS)
@pytest.mark.parametrize("n", [32, 24])
def test_conv_reglu_epilogue_matches_reference(n, isa):
    # The plan's CONV -> SLICE -> SLICE -> CLIP -> MUL: the 1x1 GEMM with the
    # kReglu epilogue equals the GEMM's rounded output through ReGLU.
    rng = np.random.default_rng(n)
    m, k = 50, 20
    w = f16(rng.normal(0, 0.3, (n, k, 1, 1)))
    b = f16(rng.normal(0, 0.1, n))
    lhs = rand16(rng, m * k, -1, 1)
    ops = O.Kernels()
    packed = ops.pack_conv(w, b, n, k, 1, 1)
    plain = ops.gemm(m, n, k, lhs, packed, isa=isa)
    got = O.Ops().reglu(plain, m, n // 2, -0.5, 0.5, isa)
    want = O.Ops("ref").gemm_reglu(m, n, k, lhs, packed, -0.5, 0.5, isa)
    assert np.array_equal(got, want)


@needs_ref
@pytest.mark.parametrize("isa", ISAS)
@pytest.mark.parametrize("ch", [16, 13])
@pytest.mark.parametrize("outputs", [False, True])
def test_feature_update_matches_reference(ch, isa, outputs):
    rng = np.random.default_rng(ch + 10 * isa)
    sp = 41
    x = rand16(rng, sp * 3 * ch, -6, 6)
    hist = rand16(rng, sp * ch, -2, 2)
    scale = rand16(rng, ch, 0.5, 1.5)
    got = O.Ops().feature_update(x, hist, scale, sp, ch, outputs, isa)
    want = O.Ops("ref").feature_update(x, hist, scale, sp, ch, outputs, isa)
    for g, w in zip(got if outputs else [got], want if outputs else [want]):
        assert np.array_equal(g, w)


def tail_inputs(rng, sp, q):
    latent = rand16(rng, sp * 2 * q, -20, 20)
    prior = np.concatenate([rand16(rng, sp * 2 * q, -0.5, 3).reshape(sp, 2 * q), rand16(rng, sp * 2 * q, -4, 4).reshape(sp, 2 * q)],
                           axis=1).reshape(-1)
    qs = rand16(rng, sp * 2 * q, 0.5, 2)
    us0, us1 = rand16(rng, sp * q, 0.5, 1.5), rand16(rng, sp * q, 0.5, 1.5)
    return latent, prior, qs, us0, us1


@needs_ref
@pytest.mark.parametrize("isa", ISAS)
@pytest.mark.parametrize("q", [16, 6])
def test_quant_tails_match_reference(q, isa):
    rng = np.random.default_rng(q + isa)
    sp = 29
    latent, prior, qs, us0, us1 = tail_inputs(rng, sp, q)
    got0 = O.Ops().y0_tail(latent, prior, qs, us0, us1, 0.11, sp, q, isa)
    want0 = O.Ops("ref").y0_tail(latent, prior, qs, us0, us1, 0.11, sp, q, isa)
    for g, w in zip(got0, want0):
        assert np.array_equal(g, w)
    normalized, clipped, _, concat2, _ = want0
    prior1 = rand16(rng, sp * 2 * q, -4, 4)
    got1 = O.Ops().y1_tail(normalized, prior1, qs, us0, us1, concat2, clipped, sp, q)
    want1 = O.Ops("ref").y1_tail(normalized, prior1, qs, us0, us1, concat2, clipped, sp, q, isa)
    for g, w in zip(got1, want1):
        assert np.array_equal(g, w)
    # y_raw holds integers (ROUND), and concat3's tail is the prior.
    raw = want0[2].view(np.float16).astype(np.float64)
    assert np.array_equal(raw, np.round(raw))
    assert np.array_equal(want0[4].reshape(sp, 6 * q)[:, 2 * q:], prior.reshape(sp, 4 * q))
