"""Exhaustive FP16 checks of the rounding points shared by every kernel.

LeakyReLU is applied to an FP16 value f as fp16(f * alpha) with the product
rounded to FP32 first (backends/cpu/src/kernels_scalar.cpp:178-192,
elementwise.cu:1-80). hipcc may fold the multiply and the narrowing into
one mixed-precision instruction, so these tests run every FP16 bit pattern
through the standalone LeakyReLU kernel and through the conv LeakyReLU
epilogue, and compare with the oracle bit for bit. ADD is checked bit for bit
on a million random pairs spread over all exponents.
"""

import numpy as np
import pytest

import graphs
import mlvc_hip
import mlvc_oracle

pytestmark = pytest.mark.gpu

ALL = np.arange(65536, dtype=np.uint32).astype(np.uint16)
IS_NAN = np.isnan(ALL.view(np.float16))
FINITE = np.isfinite(ALL.view(np.float16))


def _run(tmp_path, g, ins):
    g.write(tmp_path, "m")
    want = mlvc_oracle.OraclePlan(tmp_path, "m").run(ins)
    gpu = mlvc_hip.Backend(tmp_path, "hip")
    gpu.load("m")
    got = gpu.run(ins)
    kinds = [l["kind"] for l in gpu.launches()]
    gpu.close()
    return got, want, kinds


@pytest.mark.parametrize("alpha", [0.01, 0.1, 0.2, 0.3333])
def test_leaky_relu_every_half(tmp_path, alpha):
    g = graphs.Graph()
    x = g.input("x", [1, 256, 16, 16])
    g.output(g.leaky_relu("l", x, alpha))
    got, want, kinds = _run(tmp_path, g, [ALL.reshape(1, 256, 16, 16)])
    assert kinds == ["leaky_relu"], kinds
    got, want = got[0].reshape(-1), want[0].reshape(-1)
    ok = ~IS_NAN
    bad = np.nonzero(got[ok] != want[ok])[0]
    assert bad.size == 0, f"{bad.size} inputs differ, first {ALL[ok][bad[:8]]}"
    assert np.isnan(got[IS_NAN].view(np.float16)).all()


@pytest.mark.parametrize("alpha", [0.01, 0.2])
def test_conv_leaky_relu_epilogue_every_finite_half(tmp_path, alpha):
    """Identity 1x1 conv (exact in any accumulation order) + fused LeakyReLU:
    the epilogue sees every finite FP16 value once."""
    vals = ALL[FINITE]
    c = 16
    n_pix = (vals.size + c - 1) // c
    side = int(np.ceil(np.sqrt(n_pix)))
    x = np.zeros(c * side * side, np.uint16)
    x[: vals.size] = vals
    # NCHW with the value sequence laid out channel-major.
    x = x.reshape(1, c, side, side)
    g = graphs.Graph()
    xi = g.input("x", [1, c, side, side])
    w = g.weight_fp16("w", np.eye(c, dtype=np.float32).reshape(c, c, 1, 1))
    b = g.weight_fp16("b", np.zeros(c, np.float32))
    y = g.conv("y", xi, w, b)
    g.output(g.leaky_relu("l", y, alpha))
    got, want, kinds = _run(tmp_path, g, [x])
    assert len(kinds) == 1 and "lrelu" in kinds[0], kinds
    bad = np.nonzero(got[0].reshape(-1) != want[0].reshape(-1))[0]
    assert bad.size == 0, f"{bad.size} values differ, first inputs {x.reshape(-1)[bad[:8]]}"


def test_add_random_pairs(tmp_path):
    rng = np.random.default_rng(11)
    shape = (1, 64, 128, 128)
    finite = ALL[FINITE]
    a = rng.choice(finite, size=shape)
    b = rng.choice(finite, size=shape)
    g = graphs.Graph()
    xa, xb = g.input("a", list(shape)), g.input("b", list(shape))
    g.output(g.binary("ADD", "s", xa, xb))
    got, want, kinds = _run(tmp_path, g, [a, b])
    assert kinds == ["add"], kinds
    bad = np.nonzero(got[0] != want[0])
    assert bad[0].size == 0, f"{bad[0].size} sums differ"
