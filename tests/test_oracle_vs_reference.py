"""Pins the CPU oracle against the reference CPU kernels compiled from the
reference's own sources (oracle/_ref, built by oracle/build_ref.sh from
backends/cpu/src/{kernels_scalar,kernels_x86_avx2,thread_pool,cpu_features}.cpp).

Every kernel on the conv-graph path is compared bit for bit on seeded
random inputs, for both ISA paths (AVX2+FMA+F16C and scalar), at ragged
sizes that exercise the 6-row and 16-column tails, the scalar fallback for
N % 16 != 0 inside the AVX2 GEMM, and C % 8 != 0 inside the AVX2 depthwise.
Skipped when the reference checkout is absent (e.g. on the GPU host).
"""

import numpy as np
import pytest

import graphs
import mlvc_oracle

pytestmark = pytest.mark.skipif(not mlvc_oracle.ref_available(), reason="reference kernels not built (no checkout)")


@pytest.fixture(scope="module")
def kernels():
    return mlvc_oracle.Kernels("oracle"), mlvc_oracle.Kernels("ref")


def rnd(rng, n, lo=-1.0, hi=1.0):
    return graphs.half(rng.uniform(lo, hi, n))


@pytest.mark.parametrize("isa", [0, 1])
@pytest.mark.parametrize("m,n,k", [(1, 16, 1), (7, 32, 13), (24, 64, 64), (37, 48, 96), (5, 12, 20), (50, 11, 3),
                                   (130, 128, 256)])
@pytest.mark.parametrize("epi", [0, 1, 2, 3])
def test_gemm_bit_exact(kernels, isa, m, n, k, epi):
    o, r = kernels
    rng = np.random.default_rng(m * 1000 + n * 10 + k + epi)
    lhs = rnd(rng, m * k)
    w = graphs.half(rng.normal(0, 0.3, n * k))
    b = graphs.half(rng.normal(0, 0.2, n))
    po, pr = o.pack_conv(w, b, n, k, 1, 1), r.pack_conv(w, b, n, k, 1, 1)
    assert (po == pr).all()
    res = rnd(rng, m * n) if epi == 3 else None
    args = dict(epi=epi, alpha=0.1, cmin=-0.25, cmax=0.5, residual=res, isa=isa, threads=3)
    assert (o.gemm(m, n, k, lhs, po, **args) == r.gemm(m, n, k, lhs, pr, **args)).all()


@pytest.mark.parametrize("isa", [0, 1])
@pytest.mark.parametrize("ic,ih,iw,oc,k,s,p", [(16, 9, 11, 32, 3, 1, 1), (12, 7, 10, 64, 3, 2, 1), (3, 5, 6, 16, 3, 1, 1),
                                               (13, 6, 7, 12, 3, 1, 1), (8, 8, 10, 16, 2, 2, 0), (4, 9, 9, 8, 5, 1, 2),
                                               (32, 4, 5, 48, 3, 1, 0)])
@pytest.mark.parametrize("epi", [0, 2, 3])
def test_spatial_conv_bit_exact(kernels, isa, ic, ih, iw, oc, k, s, p, epi):
    o, r = kernels
    rng = np.random.default_rng(ic * 100 + oc + k + epi)
    oh, ow = (ih + 2 * p - k) // s + 1, (iw + 2 * p - k) // s + 1
    x = rnd(rng, ih * iw * ic)
    w = graphs.half(rng.normal(0, 0.2, oc * ic * k * k))
    b = graphs.half(rng.normal(0, 0.1, oc))
    po, pr = o.pack_conv(w, b, oc, ic, k, k), r.pack_conv(w, b, oc, ic, k, k)
    assert (po == pr).all()
    res = rnd(rng, oh * ow * oc) if epi == 3 else None
    geo = (1, ic, ih, iw, oc, oh, ow, k, k, s, s, p, p)
    a = o.spatial_conv(x, po, *geo, epi=epi, alpha=0.01, residual=res, isa=isa)
    bb = r.spatial_conv(x, pr, *geo, epi=epi, alpha=0.01, residual=res, isa=isa)
    assert (a == bb).all()


@pytest.mark.parametrize("isa", [0, 1])
@pytest.mark.parametrize("c,h,w,k,s,p", [(16, 5, 7, 3, 1, 1), (12, 4, 9, 3, 1, 1), (256, 6, 8, 3, 1, 1), (8, 7, 9, 3, 2, 1),
                                         (5, 6, 6, 5, 1, 2), (24, 1, 1, 3, 1, 1)])
def test_depthwise_bit_exact(kernels, isa, c, h, w, k, s, p):
    o, r = kernels
    rng = np.random.default_rng(c + h + k)
    oh, ow = (h + 2 * p - k) // s + 1, (w + 2 * p - k) // s + 1
    x = rnd(rng, h * w * c)
    wt = graphs.half(rng.normal(0, 0.3, c * k * k))
    b = graphs.half(rng.normal(0, 0.1, c))
    po, pr = o.pack_depthwise(wt, b, c, k, k), r.pack_depthwise(wt, b, c, k, k)
    assert (po == pr).all()
    geo = (1, c, h, w, oh, ow, k, k, s, s, p, p)
    assert (o.depthwise(x, po, *geo, isa=isa) == r.depthwise(x, pr, *geo, isa=isa)).all()


@pytest.mark.parametrize("isa", [0, 1])
def test_elementwise_bit_exact(kernels, isa):
    o, r = kernels
    rng = np.random.default_rng(5)
    a, b = rnd(rng, 1003, -4, 4), rnd(rng, 1003, -4, 4)
    assert (o.leaky_relu(a, 0.01, isa) == r.leaky_relu(a, 0.01, isa)).all()
    assert (o.add(a, b, isa) == r.add(a, b, isa)).all()


@pytest.mark.parametrize("c,h,w,block", [(8, 3, 5, 2), (12, 4, 4, 2), (64, 2, 3, 8), (3, 6, 10, 2)])
def test_pixel_shuffle_and_layout_bit_exact(kernels, c, h, w, block):
    o, r = kernels
    rng = np.random.default_rng(c * h)
    if c % (block * block) == 0:
        x = rnd(rng, c * h * w)
        assert (o.depth_to_space(x, 1, c, h, w, block) == r.depth_to_space(x, 1, c, h, w, block)).all()
    if h % block == 0 and w % block == 0:
        x = rnd(rng, c * h * w)
        assert (o.space_to_depth(x, 1, c, h, w, block) == r.space_to_depth(x, 1, c, h, w, block)).all()
    x = rnd(rng, c * h * w)
    assert (o.nchw_to_nhwc(x, 1, c, h * w) == r.nchw_to_nhwc(x, 1, c, h * w)).all()
    assert (o.nhwc_to_nchw(x, 1, h * w, c) == r.nhwc_to_nchw(x, 1, h * w, c)).all()


def test_fp16_conversion_matches_reference(kernels):
    o, r = kernels
    for hbits in range(0, 65536, 7):
        a, b = o.half_to_float(hbits), r.half_to_float(hbits)
        assert (np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32)) or (np.isnan(a) and np.isnan(b))
    rng = np.random.default_rng(9)
    fs = np.concatenate([rng.normal(0, 10, 3000), rng.normal(0, 1e-5, 2000), [65504, 65520, 65519.99, 1e-8, 6e-8, -0.0]])
    for f in fs.astype(np.float32):
        assert o.float_to_half(float(f)) == r.float_to_half(float(f))
