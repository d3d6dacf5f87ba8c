"""mlvc_hip_conv_launch_noalloc (the conv launch that allocates nothing: the
FP32 partials of a split-K conv live in the library's static device array)
against mlvc_hip_conv_launch with a caller workspace, through the device C
ABI: bit-identical outputs on two calls in a row, the second with a smaller
input (the array keeps the first call's partials), a conv that is not split,
and the error for a split set by hand whose partials exceed the array. Each
result is also checked against a float64 product at the FP16 bar.
"""

import ctypes as C

import numpy as np
import pytest

import mlvc_hip
from conftest import MAX_REL, MEAN_REL
from devmem import Dev
from test_conv_candidates import ConvDesc

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 512 * 128 * 128 * 4


def _bind(lib):
    pd = C.POINTER(ConvDesc)
    lib.mlvc_hip_conv_plan.argtypes = [pd]
    for fn in (lib.mlvc_hip_conv_packed_bytes, lib.mlvc_hip_conv_bias_len, lib.mlvc_hip_conv_workspace_bytes):
        fn.argtypes = [pd]
        fn.restype = C.c_size_t
    lib.mlvc_hip_conv_pack.argtypes = [pd, C.c_void_p, C.c_void_p]
    lib.mlvc_hip_conv_launch.argtypes = [pd, C.c_void_p]
    lib.mlvc_hip_conv_launch_noalloc.argtypes = [pd, C.c_void_p]


def _conv(dev, n, ic, h, w, oc, epilogue, seed):
    """A planned 1x1 conv with its operands in device memory; returns the
    descriptor, the float64 reference output (before FP16 rounding of the
    epilogue) and the output shape."""
    lib = dev.lib
    rng = np.random.default_rng(seed)
    d = ConvDesc(n=n, ic=ic, ih=h, iw=w, oc=oc, oh=h, ow=w, kh=1, kw=1, stride_h=1, stride_w=1, pad_h=0, pad_w=0,
                 epilogue=epilogue, alpha=0.01)
    dev.check(lib.mlvc_hip_conv_plan(C.byref(d)))
    x = rng.uniform(-1, 1, (n, ic, h, w)).astype(np.float16)
    wt = rng.normal(0, 1 / np.sqrt(ic), (oc, ic, 1, 1)).astype(np.float16)
    bias = rng.normal(0, 0.1, oc).astype(np.float16)
    packed = np.zeros(lib.mlvc_hip_conv_packed_bytes(C.byref(d)), np.uint8)
    dev.check(lib.mlvc_hip_conv_pack(C.byref(d), wt.view(np.uint16).ctypes.data, packed.ctypes.data))
    b32 = np.zeros(lib.mlvc_hip_conv_bias_len(C.byref(d)), np.float32)
    b32[:oc] = bias.astype(np.float32)
    d.x = dev.put(x.view(np.uint16))
    d.packed_w = dev.put(packed)
    d.bias = dev.put(b32)
    want = np.einsum("oc,nchw->nohw", wt[:, :, 0, 0].astype(np.float64), x.astype(np.float64))
    want += bias.astype(np.float64)[None, :, None, None]
    if epilogue == 2:  # residual
        r = rng.uniform(-1, 1, (n, oc, h, w)).astype(np.float16)
        d.residual = dev.put(r.view(np.uint16))
        want = want + r.astype(np.float64)
    elif epilogue == 1:  # LeakyReLU
        want = np.where(want < 0, want * 0.01, want)
    return d, want, (n, oc, h, w)


def _both(dev, d, shape):
    """Output of mlvc_hip_conv_launch (with a workspace) and of
    mlvc_hip_conv_launch_noalloc on the same descriptor."""
    lib = dev.lib
    nbytes = int(np.prod(shape)) * 2
    d.y = dev.alloc(nbytes)
    ws = lib.mlvc_hip_conv_workspace_bytes(C.byref(d))
    d.workspace = dev.alloc(ws) if ws else None
    d.workspace_bytes = ws
    dev.check(lib.mlvc_hip_conv_launch(C.byref(d), None))
    a = dev.get(d.y, shape, np.uint16)
    d.y = dev.alloc(nbytes)
    d.workspace, d.workspace_bytes = None, 0
    dev.check(lib.mlvc_hip_conv_launch_noalloc(C.byref(d), None))
    return a, dev.get(d.y, shape, np.uint16)


def _bar(got, want):
    g = got.view(np.float16).astype(np.float64)
    rms = np.sqrt(np.mean(want ** 2))
    err = np.abs(g - want) / rms
    assert err.max() <= MAX_REL and err.mean() <= MEAN_REL, (err.max(), err.mean())


def test_noalloc_matches_the_workspace_launch():
    dev = Dev()
    _bind(dev.lib)
    try:
        # 1: 1x1 1024 -> 256 at 46x80 (8 splits of 128 channels, 30 MB of
        # partials); 2: a smaller input right after it, 1x1 600 -> 64 over two
        # images of 6x10 with a residual (5 splits, the last of 88 channels).
        for n, ic, h, w, oc, epi, splits in ((1, 1024, 46, 80, 256, 1, 8), (2, 600, 6, 10, 64, 2, 5)):
            d, want, shape = _conv(dev, n, ic, h, w, oc, epi, seed=ic)
            assert d.ksplit == splits, d.ksplit
            assert dev.lib.mlvc_hip_conv_workspace_bytes(C.byref(d)) <= SCRATCH_BYTES
            a, b = _both(dev, d, shape)
            assert np.array_equal(a, b), f"{ic}->{oc}: {np.count_nonzero(a != b)} outputs differ"
            _bar(b, want)
        # A conv that is not split runs unchanged.
        d, want, shape = _conv(dev, 1, 64, 16, 24, 32, 0, seed=3)
        assert d.ksplit <= 1
        a, b = _both(dev, d, shape)
        assert np.array_equal(a, b)
        _bar(b, want)
    finally:
        dev.close()


def test_noalloc_rejects_partials_beyond_its_array():
    dev = Dev()
    _bind(dev.lib)
    try:
        # 1x1 1024 -> 1024 at 64x64: planned as 2 splits (exactly the 32 MiB
        # the array holds); 8 splits set by hand need 128 MiB.
        d, _, shape = _conv(dev, 1, 1024, 64, 64, 1024, 0, seed=9)
        assert d.ksplit == 2 and dev.lib.mlvc_hip_conv_workspace_bytes(C.byref(d)) == SCRATCH_BYTES
        d.ksplit, d.split_c = 8, 128
        d.y = dev.alloc(int(np.prod(shape)) * 2)
        assert dev.lib.mlvc_hip_conv_launch_noalloc(C.byref(d), None) == -1
        msg = dev.lib.mlvc_hip_last_error().decode()
        assert "no-allocation launch holds" in msg and str(SCRATCH_BYTES) in msg, msg
    finally:
        dev.close()
