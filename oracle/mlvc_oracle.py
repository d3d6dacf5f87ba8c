"""ctypes binding of the CPU oracle (oracle/liboracle.so) and of the
reference CPU kernels built from source (oracle/_ref/libmlvc_ref_kernels.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the parity reference and the CPU baseline. The
product never imports this module.
"""

from __future__ import annotations

import ctypes as C
import pathlib

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
ORACLE_LIB = HERE / "liboracle.so"
REF_LIB = HERE / "_ref" / "libmlvc_ref_kernels.so"

_u16p = C.POINTER(C.c_uint16)
_u8p = C.POINTER(C.c_uint8)
_i64p = C.POINTER(C.c_int64)


class OracleError(RuntimeError):
    pass


def _kernel_api(lib: C.CDLL, prefix: str) -> None:
    f = lambda name: getattr(lib, prefix + name)  # noqa: E731
    f("last_error").restype = C.c_char_p
    f("pack_conv").argtypes = [_u16p, _u16p, C.c_int, C.c_int, C.c_int, C.c_int, _u16p, C.c_size_t]
    f("pack_depthwise").argtypes = [_u16p, _u16p, C.c_int, C.c_int, C.c_int, _u16p, C.c_size_t]
    f("gemm_nhwc").argtypes = [C.c_size_t, C.c_size_t, C.c_size_t, _u16p, _u16p, _u16p, C.c_int, C.c_float, C.c_float,
                               C.c_float, _u16p, C.c_int, C.c_int]
    f("spatial_conv_nhwc").argtypes = [_u16p, _u16p, _u16p] + [C.c_int] * 14 + [C.c_float, _u16p, C.c_int, C.c_int]
    f("depthwise_nhwc").argtypes = [_u16p, _u16p, _u16p] + [C.c_int] * 14
    f("leaky_relu").argtypes = [_u16p, _u16p, C.c_size_t, C.c_float, C.c_int]
    f("add").argtypes = [_u16p, _u16p, _u16p, C.c_size_t, C.c_int]
    f("depth_to_space_nhwc").argtypes = [_u16p, _u16p] + [C.c_int] * 5
    f("space_to_depth_nhwc").argtypes = [_u16p, _u16p] + [C.c_int] * 5
    f("nchw_to_nhwc").argtypes = [_u16p, _u16p, C.c_size_t, C.c_size_t, C.c_size_t]
    f("nhwc_to_nchw").argtypes = [_u16p, _u16p, C.c_size_t, C.c_size_t, C.c_size_t]
    f("float_to_half").argtypes = [C.c_float]
    f("float_to_half").restype = C.c_uint16
    f("half_to_float").argtypes = [C.c_uint16]
    f("half_to_float").restype = C.c_float


_oracle = None
_ref = None


def oracle_lib() -> C.CDLL:
    global _oracle
    if _oracle is None:
        if not ORACLE_LIB.exists():
            raise OracleError(f"{ORACLE_LIB} is not built; run `python mlvc.cpp_amd/build.py`")
        lib = C.CDLL(str(ORACLE_LIB))
        _kernel_api(lib, "oracle_")
        lib.oracle_packed_conv_elems.restype = C.c_size_t
        lib.oracle_packed_conv_elems.argtypes = [C.c_int] * 4
        lib.oracle_packed_depthwise_elems.restype = C.c_size_t
        lib.oracle_packed_depthwise_elems.argtypes = [C.c_int] * 3
        lib.oracle_load.restype = C.c_void_p
        lib.oracle_load.argtypes = [C.c_char_p, C.c_char_p, _i64p, C.c_int, C.c_int, C.c_int, C.c_int]
        lib.oracle_free.argtypes = [C.c_void_p]
        lib.oracle_reset_state.argtypes = [C.c_void_p]
        lib.oracle_thread_count.argtypes = [C.c_void_p]
        lib.oracle_step_count.argtypes = [C.c_void_p]
        lib.oracle_io_count.argtypes = [C.c_void_p, C.c_int]
        lib.oracle_io_shape.argtypes = [C.c_void_p, C.c_int, C.c_int, _i64p, C.POINTER(C.c_int)]
        lib.oracle_run.argtypes = [C.c_void_p, C.POINTER(_u16p), C.POINTER(_u16p)]
        lib.oracle_yuv420_to_model.argtypes = [_u8p] + [C.c_int] * 5 + [C.c_float, _u16p]
        lib.oracle_model_to_yuv420.argtypes = [_u16p] + [C.c_int] * 7 + [C.c_float, _u8p]
        lib.oracle_frame_padding.argtypes = [C.c_int] * 4 + [C.POINTER(C.c_int)]
        _oracle = lib
    return _oracle


def ref_available() -> bool:
    return REF_LIB.exists()


def ref_lib() -> C.CDLL:
    global _ref
    if _ref is None:
        if not REF_LIB.exists():
            raise OracleError(f"{REF_LIB} is not built (needs the reference checkout)")
        lib = C.CDLL(str(REF_LIB))
        _kernel_api(lib, "ref_")
        lib.ref_prepare_model_input.argtypes = [_u8p] + [C.c_int] * 4 + [C.c_float, _u16p, C.POINTER(C.c_int)]
        lib.ref_prepare_model_output.argtypes = [_u16p] + [C.c_int] * 4 + [C.c_float, C.POINTER(C.c_int), _u8p]
        _ref = lib
    return _ref


def _p(a) -> C.POINTER(C.c_uint16):
    return None if a is None else a.ctypes.data_as(_u16p)


class Kernels:
    """Kernel-level entry points (NHWC buffers) of the oracle or reference."""

    def __init__(self, which: str = "oracle"):
        self.lib = oracle_lib() if which == "oracle" else ref_lib()
        self.prefix = "oracle_" if which == "oracle" else "ref_"

    def _call(self, name, *args):
        rc = getattr(self.lib, self.prefix + name)(*args)
        if rc != 0:
            raise OracleError(getattr(self.lib, self.prefix + "last_error")().decode())

    def pack_conv(self, w, b, oc, ic, kh, kw):
        n = oracle_lib().oracle_packed_conv_elems(oc, ic, kh, kw)
        out = np.zeros(n, np.uint16)
        self._call("pack_conv", _p(w), _p(b), oc, ic, kh, kw, _p(out), n)
        return out

    def pack_depthwise(self, w, b, c, kh, kw):
        n = oracle_lib().oracle_packed_depthwise_elems(c, kh, kw)
        out = np.zeros(n, np.uint16)
        self._call("pack_depthwise", _p(w), _p(b), c, kh, kw, _p(out), n)
        return out

    def gemm(self, m, n, k, lhs, packed, epi=0, alpha=0.01, cmin=0.0, cmax=0.0, residual=None, isa=0, threads=2):
        out = np.zeros(m * n, np.uint16)
        self._call("gemm_nhwc", m, n, k, _p(lhs), _p(packed), _p(out), epi, alpha, cmin, cmax, _p(residual), isa,
                   threads)
        return out

    def spatial_conv(self, x, packed, n, ic, ih, iw, oc, oh, ow, kh, kw, sh, sw, ph, pw, epi=0, alpha=0.01,
                     residual=None, isa=0, threads=2):
        out = np.zeros(n * oh * ow * oc, np.uint16)
        self._call("spatial_conv_nhwc", _p(x), _p(packed), _p(out), n, ic, ih, iw, oc, oh, ow, kh, kw, sh, sw, ph, pw,
                   epi, alpha, _p(residual), isa, threads)
        return out

    def depthwise(self, x, packed, n, c, ih, iw, oh, ow, kh, kw, sh, sw, ph, pw, isa=0, threads=2):
        out = np.zeros(n * oh * ow * c, np.uint16)
        self._call("depthwise_nhwc", _p(x), _p(packed), _p(out), n, c, ih, iw, oh, ow, kh, kw, sh, sw, ph, pw, isa,
                   threads)
        return out

    def leaky_relu(self, x, alpha, isa=0):
        out = np.zeros_like(x)
        self._call("leaky_relu", _p(x), _p(out), x.size, alpha, isa)
        return out

    def add(self, a, b, isa=0):
        out = np.zeros_like(a)
        self._call("add", _p(a), _p(b), _p(out), a.size, isa)
        return out

    def depth_to_space(self, x, n, c, h, w, block):
        out = np.zeros_like(x)
        self._call("depth_to_space_nhwc", _p(x), _p(out), n, c, h, w, block)
        return out

    def space_to_depth(self, x, n, c, h, w, block):
        out = np.zeros_like(x)
        self._call("space_to_depth_nhwc", _p(x), _p(out), n, c, h, w, block)
        return out

    def nchw_to_nhwc(self, x, n, c, hw):
        out = np.zeros_like(x)
        self._call("nchw_to_nhwc", _p(x), _p(out), n, c, hw)
        return out

    def nhwc_to_nchw(self, x, n, hw, c):
        out = np.zeros_like(x)
        self._call("nhwc_to_nchw", _p(x), _p(out), n, hw, c)
        return out

    def float_to_half(self, f: float) -> int:
        return int(getattr(self.lib, self.prefix + "float_to_half")(f))

    def half_to_float(self, h: int) -> float:
        return float(getattr(self.lib, self.prefix + "half_to_float")(h))


class OraclePlan:
    """Graph-level oracle: the reference CpuExecutionPlan restated."""

    def __init__(self, model_dir, model_name: str, bindings=(), num_threads: int = 0, isa: int = 0,
                 fusion: bool = True):
        lib = oracle_lib()
        flat = (C.c_int64 * max(1, 2 * len(bindings)))(*[v for b in bindings for v in b])
        h = lib.oracle_load(str(model_dir).encode(), model_name.encode(), flat, len(bindings), num_threads, isa,
                            1 if fusion else 0)
        if not h:
            raise OracleError(lib.oracle_last_error().decode())
        self._lib, self._h = lib, h
        self.in_shapes = [self._shape(0, i) for i in range(lib.oracle_io_count(h, 0))]
        self.out_shapes = [self._shape(1, i) for i in range(lib.oracle_io_count(h, 1))]

    def _shape(self, is_out, i):
        s = (C.c_int64 * 4)()
        r = C.c_int()
        if self._lib.oracle_io_shape(self._h, is_out, i, s, C.byref(r)) != 0:
            raise OracleError(self._lib.oracle_last_error().decode())
        return tuple(int(s[j]) for j in range(r.value))

    @property
    def threads(self) -> int:
        return self._lib.oracle_thread_count(self._h)

    @property
    def steps(self) -> int:
        return self._lib.oracle_step_count(self._h)

    def reset_state(self) -> None:
        if self._lib.oracle_reset_state(self._h) != 0:
            raise OracleError(self._lib.oracle_last_error().decode())

    def run(self, inputs) -> list[np.ndarray]:
        # FP16 inputs as uint16 bits; INT32 control inputs pass as raw bytes.
        ins = [np.ascontiguousarray(a).view(np.uint16) if np.asarray(a).dtype == np.int32
               else np.ascontiguousarray(a, dtype=np.uint16) for a in inputs]
        if len(ins) != len(self.in_shapes):
            raise OracleError("graph input count mismatch")
        outs = [np.empty(s, np.uint16) for s in self.out_shapes]
        ip = (_u16p * len(ins))(*[_p(a) for a in ins])
        op = (_u16p * len(outs))(*[_p(a) for a in outs])
        if self._lib.oracle_run(self._h, ip, op) != 0:
            raise OracleError(self._lib.oracle_last_error().decode())
        return outs

    def close(self) -> None:
        if self._h:
            self._lib.oracle_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---- codec I/O (frame <-> model image), I420 frames as flat uint8 arrays

def yuv_frame_bytes(w: int, h: int) -> int:
    return w * h + 2 * (w // 2) * (h // 2)


def _check(lib, prefix, rc):
    if rc != 0:
        raise OracleError(getattr(lib, prefix + "last_error")().decode())


def frame_padding(w: int, h: int, mw: int, mh: int) -> tuple:
    """(left, right, top, bottom, rotated) of core/src/yuv.cpp:325-337."""
    lib = oracle_lib()
    pad = (C.c_int * 5)()
    _check(lib, "oracle_", lib.oracle_frame_padding(w, h, mw, mh, pad))
    return tuple(pad)


def yuv_to_model(yuv: np.ndarray, w: int, h: int, mw: int, mh: int, rotated: int, pixel_range: float) -> np.ndarray:
    """I420 frame -> FP16 bits [3, mh, mw]."""
    lib = oracle_lib()
    yuv = np.ascontiguousarray(yuv, np.uint8)
    out = np.zeros((3, mh, mw), np.uint16)
    _check(lib, "oracle_", lib.oracle_yuv420_to_model(yuv.ctypes.data_as(_u8p), w, h, mw, mh, rotated,
                                                       pixel_range, out.ctypes.data_as(_u16p)))
    return out


def model_to_yuv(x: np.ndarray, w: int, h: int, pad: tuple, pixel_range: float) -> np.ndarray:
    """FP16 bits [3, mh, mw] -> I420 frame; pad = (left, right, top, bottom, rotated)."""
    lib = oracle_lib()
    x = np.ascontiguousarray(x, np.uint16)
    mh, mw = x.shape[-2], x.shape[-1]
    out = np.zeros(yuv_frame_bytes(w, h), np.uint8)
    _check(lib, "oracle_", lib.oracle_model_to_yuv420(x.ctypes.data_as(_u16p), w, h, mw, mh, pad[0], pad[2], pad[4],
                                                       pixel_range, out.ctypes.data_as(_u8p)))
    return out


def ref_prepare_model_input(yuv: np.ndarray, w: int, h: int, mw: int, mh: int, pixel_range: float):
    """The reference's prepare_model_input (core/src/yuv.cpp): (image, pad)."""
    lib = ref_lib()
    yuv = np.ascontiguousarray(yuv, np.uint8)
    out = np.zeros((3, mh, mw), np.uint16)
    pad = (C.c_int * 5)()
    _check(lib, "ref_", lib.ref_prepare_model_input(yuv.ctypes.data_as(_u8p), w, h, mw, mh, pixel_range,
                                                     out.ctypes.data_as(_u16p), pad))
    return out, tuple(pad)


def ref_prepare_model_output(x: np.ndarray, w: int, h: int, pad: tuple, pixel_range: float) -> np.ndarray:
    """The reference's prepare_model_output_into (core/src/yuv.cpp)."""
    lib = ref_lib()
    x = np.ascontiguousarray(x, np.uint16)
    mh, mw = x.shape[-2], x.shape[-1]
    out = np.zeros(yuv_frame_bytes(w, h), np.uint8)
    cpad = (C.c_int * 5)(*pad)
    _check(lib, "ref_", lib.ref_prepare_model_output(x.ctypes.data_as(_u16p), w, h, mw, mh, pixel_range, cpad,
                                                      out.ctypes.data_as(_u8p)))
    return out


# ---- operators of the real-model graphs (NHWC buffers, raw FP16 bits)

_i32p = C.POINTER(C.c_int32)
_ip = C.POINTER(C.c_int)
UNARY = {"clip": 0, "sigmoid": 1, "reciprocal": 2, "round": 3}
BINARY = {"add": 0, "sub": 1, "mul": 2}
_ops_bound = set()


def _bind_ops(lib, prefix):
    if prefix in _ops_bound:
        return
    f = lambda name: getattr(lib, prefix + name)  # noqa: E731
    f("slice_nhwc").argtypes = [_u16p, _u16p, _ip, _ip, _ip, _ip]
    f("concat_nhwc").argtypes = [C.POINTER(_u16p), _ip, C.c_int, _u16p, _ip, C.c_int]
    f("reglu_nhwc").argtypes = [_u16p, _u16p, C.c_size_t, C.c_size_t, C.c_float, C.c_float, C.c_int]
    f("feature_update_nhwc").argtypes = [_u16p] * 6 + [C.c_size_t, C.c_size_t, C.c_int]
    f("y0_tail_nhwc").argtypes = [_u16p] * 10 + [C.c_float, C.c_size_t, C.c_size_t, C.c_int]
    if prefix == "oracle_":
        f("unary").argtypes = [_u16p, _u16p, C.c_size_t, C.c_int, C.c_float, C.c_float, C.c_int]
        f("binary").argtypes = [_u16p, _i64p, C.c_int, _u16p, _i64p, C.c_int, _u16p, _i64p, C.c_int, C.c_int]
        f("gather").argtypes = [_u16p, _i64p, C.c_int, _i32p, _i64p, C.c_size_t, C.c_int, _u16p]
        f("y1_tail_nhwc").argtypes = [_u16p] * 9 + [C.c_size_t, C.c_size_t]
    else:
        f("unary").argtypes = [_u16p, _u16p, C.c_size_t, C.c_int, C.c_float, C.c_float, C.c_int, C.c_int]
        f("binary_contiguous").argtypes = [_u16p, _u16p, _u16p, C.c_size_t, C.c_int, C.c_int]
        f("binary_scalar").argtypes = [_u16p, C.c_uint16, _u16p, C.c_size_t, C.c_int, C.c_int, C.c_int]
        f("binary_channel").argtypes = [_u16p, _u16p, _u16p, C.c_size_t, C.c_size_t, C.c_int, C.c_int, C.c_int]
        f("gemm_reglu_nhwc").argtypes = [C.c_size_t, C.c_size_t, C.c_size_t, _u16p, _u16p, _u16p, C.c_float, C.c_float,
                                         C.c_int, C.c_int]
        f("y1_tail_nhwc").argtypes = [_u16p] * 9 + [C.c_size_t, C.c_size_t, C.c_int]
    _ops_bound.add(prefix)


class Ops:
    """Kernel-level operators of the oracle ("oracle") or of the reference
    kernels built from source ("ref"), on NHWC FP16 buffers."""

    def __init__(self, which: str = "oracle"):
        self.lib = oracle_lib() if which == "oracle" else ref_lib()
        self.prefix = "oracle_" if which == "oracle" else "ref_"
        _bind_ops(self.lib, self.prefix)

    def _call(self, name, *args):
        _check(self.lib, self.prefix, getattr(self.lib, self.prefix + name)(*args))

    @staticmethod
    def _u16(a):
        return np.ascontiguousarray(a, np.uint16)

    def unary(self, x, op, lo=0.0, hi=0.0, isa=0, threads=1):
        x = self._u16(x)
        out = np.zeros_like(x)
        extra = (isa, threads) if self.prefix == "ref_" else (isa,)
        self._call("unary", _p(x), _p(out), x.size, UNARY[op], lo, hi, *extra)
        return out

    def binary(self, a, a_shape, b, b_shape, out_shape, op):
        """Oracle only: the reference plan's full ADD/SUB/MUL dispatch."""
        a, b = self._u16(a), self._u16(b)
        out = np.zeros(int(np.prod(out_shape)), np.uint16)
        sa, sb, so = (np.asarray(s, np.int64) for s in (a_shape, b_shape, out_shape))
        self._call("binary", _p(a), sa.ctypes.data_as(_i64p), len(sa), _p(b), sb.ctypes.data_as(_i64p), len(sb), _p(out),
                   so.ctypes.data_as(_i64p), len(so), BINARY[op])
        return out

    def binary_contiguous(self, a, b, op, isa=0):
        a, b = self._u16(a), self._u16(b)
        out = np.zeros_like(a)
        self._call("binary_contiguous", _p(a), _p(b), _p(out), a.size, BINARY[op], isa)
        return out

    def binary_scalar(self, vec, scalar, op, scalar_lhs, isa=0):
        vec = self._u16(vec)
        out = np.zeros_like(vec)
        self._call("binary_scalar", _p(vec), int(scalar), _p(out), vec.size, BINARY[op], int(scalar_lhs), isa)
        return out

    def binary_channel(self, vec, chan, spatial, channels, op, chan_lhs, isa=0):
        vec, chan = self._u16(vec), self._u16(chan)
        out = np.zeros_like(vec)
        self._call("binary_channel", _p(vec), _p(chan), _p(out), spatial, channels, BINARY[op], int(chan_lhs), isa)
        return out

    def slice(self, x, id4, od4, starts, steps):
        x = self._u16(x)
        out = np.zeros(int(np.prod(od4)), np.uint16)
        arr = [(C.c_int * 4)(*v) for v in (id4, od4, starts, steps)]
        self._call("slice_nhwc", _p(x), _p(out), *arr)
        return out

    def concat(self, xs, dims, od4, axis):
        xs = [self._u16(x) for x in xs]
        out = np.zeros(int(np.prod(od4)), np.uint16)
        ptrs = (_u16p * len(xs))(*[_p(x) for x in xs])
        flat = (C.c_int * (4 * len(dims)))(*[v for d in dims for v in d])
        self._call("concat_nhwc", ptrs, flat, len(xs), _p(out), (C.c_int * 4)(*od4), axis)
        return out

    def gather(self, data, shape, idx, axis):
        """Oracle only (the reference's gather lives in its plan)."""
        data = self._u16(data)
        shape = np.asarray(shape, np.int64)
        idx = np.asarray(idx)
        i32 = idx.astype(np.int32) if idx.dtype == np.int32 else None
        i64 = None if i32 is not None else np.ascontiguousarray(idx, np.int64)
        rank = len(shape)
        ax = axis + rank if axis < 0 else axis
        dim = int(shape[ax]) if 0 <= ax < rank else 1
        out = np.zeros(int(np.prod(shape)) // dim * idx.size, np.uint16)
        self._call("gather", _p(data), shape.ctypes.data_as(_i64p), rank,
                   None if i32 is None else i32.ctypes.data_as(_i32p), None if i64 is None else i64.ctypes.data_as(_i64p),
                   idx.size, axis, _p(out))
        return out

    def reglu(self, x, spatial, g, lo, hi, isa=0):
        x = self._u16(x)
        out = np.zeros(spatial * g, np.uint16)
        self._call("reglu_nhwc", _p(x), _p(out), spatial, g, lo, hi, isa)
        return out

    def gemm_reglu(self, m, n, k, lhs, packed, lo, hi, isa=0, threads=2):
        out = np.zeros(m * (n // 2), np.uint16)
        self._call("gemm_reglu_nhwc", m, n, k, _p(self._u16(lhs)), _p(packed), _p(out), lo, hi, isa, threads)
        return out

    def feature_update(self, x, hist, scale, spatial, ch, outputs=False, isa=0):
        x, hist, scale = self._u16(x), self._u16(hist), self._u16(scale)
        feat = np.zeros(spatial * 2 * ch, np.uint16)
        sc = np.zeros(spatial * ch, np.uint16) if outputs else None
        bl = np.zeros(spatial * ch, np.uint16) if outputs else None
        self._call("feature_update_nhwc", _p(x), _p(hist), _p(scale), _p(sc), _p(bl), _p(feat), spatial, ch, isa)
        return (feat, sc, bl) if outputs else feat

    def y0_tail(self, latent, prior, qs, us0, us1, clip_min, spatial, q, isa=0):
        ins = [self._u16(a) for a in (latent, prior, qs, us0, us1)]
        outs = [np.zeros(spatial * c, np.uint16) for c in (2 * q, 2 * q, q, 2 * q, 6 * q)]
        self._call("y0_tail_nhwc", *[_p(a) for a in ins], *[_p(a) for a in outs], clip_min, spatial, q, isa)
        return outs  # normalized, clipped, y_raw, concat2, concat3

    def y1_tail(self, normalized, prior, qs, us0, us1, concat2, clipped, spatial, q, isa=0):
        ins = [self._u16(a) for a in (normalized, prior, qs, us0, us1, concat2, clipped)]
        outs = [np.zeros(spatial * q, np.uint16), np.zeros(spatial * 2 * q, np.uint16)]
        extra = (isa,) if self.prefix == "ref_" else ()
        self._call("y1_tail_nhwc", *[_p(a) for a in ins], *[_p(a) for a in outs], spatial, q, *extra)
        return outs  # y_raw, out


def mfma_step(a: np.ndarray, b: np.ndarray, c: np.ndarray) -> np.ndarray:
    """The isa-2 model of one v_mfma_f32_32x32x16_f16 step per case: a, b
    [n, 16] raw binary16, c [n] float32 -> [n] float32 = c + sum a*b as the
    matrix core sums it."""
    lib = oracle_lib()
    lib.oracle_mfma_step.argtypes = [C.c_void_p] * 4 + [C.c_size_t]
    a = np.ascontiguousarray(a, np.uint16)
    b = np.ascontiguousarray(b, np.uint16)
    c = np.ascontiguousarray(c, np.float32)
    out = np.zeros(c.shape, np.float32)
    if lib.oracle_mfma_step(a.ctypes.data, b.ctypes.data, c.ctypes.data, out.ctypes.data, c.size) != 0:
        raise OracleError(lib.oracle_last_error().decode())
    return out


def parity_stats(got: np.ndarray, want: np.ndarray) -> dict:
    """max|d|/RMS(want) and mean|d|/RMS(want) over FP16 tensors (raw bits)."""
    g = got.view(np.float16).astype(np.float64)
    w = want.view(np.float16).astype(np.float64)
    rms = float(np.sqrt(np.mean(w * w)))
    d = np.abs(g - w)
    scale = rms if rms > 0 else 1.0
    return {"max_rel": float(d.max() / scale), "mean_rel": float(d.mean() / scale), "rms": rms,
            "finite": bool(np.isfinite(g).all())}
