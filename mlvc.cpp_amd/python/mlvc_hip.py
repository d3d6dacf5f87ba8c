"""ctypes binding of the MI355X backend's C ABI (include/mlvc_hip_backend.h
and include/mlvc_hip_device.h).

`Backend` mirrors mlvc::InferenceBackend (reference
runtime/include/mlvc/runtime/backend.hpp:48-63): load(model, bindings),
run(inputs) -> outputs, reset_state(). Tensors are numpy uint16 arrays of
raw binary16 values in NCHW order. Errors raise MlvcError with the library's
message. The libraries must have been built (python mlvc.cpp_amd/build.py);
nothing here falls back to another implementation.
"""

from __future__ import annotations

import ctypes as C
import json
import pathlib

import numpy as np

LIB_DIR = pathlib.Path(__file__).resolve().parent.parent / "lib"
BACKEND_LIB = LIB_DIR / "libmlvc_hip.so"
DEVICE_LIB = LIB_DIR / "libmlvc_hip_device.so"

_i64p = C.POINTER(C.c_int64)
_u16p = C.POINTER(C.c_uint16)


class MlvcError(RuntimeError):
    pass


_lib = None
_dev = None


def _load(path: pathlib.Path) -> C.CDLL:
    if not path.exists():
        raise MlvcError(f"{path} is not built; run `python mlvc.cpp_amd/build.py`")
    return C.CDLL(str(path))


def backend_lib() -> C.CDLL:
    global _lib
    if _lib is None:
        lib = _load(BACKEND_LIB)
        lib.mlvc_backend_last_error.restype = C.c_char_p
        lib.mlvc_backend_name.restype = C.c_char_p
        lib.mlvc_backend_create.argtypes = [C.c_char_p, C.c_char_p, C.c_int, C.c_int, C.POINTER(C.c_void_p)]
        lib.mlvc_backend_destroy.argtypes = [C.c_void_p]
        lib.mlvc_backend_name.argtypes = [C.c_void_p]
        lib.mlvc_backend_load.argtypes = [C.c_void_p, C.c_char_p, _i64p, C.c_int]
        lib.mlvc_backend_io_count.argtypes = [C.c_void_p, C.c_int, C.POINTER(C.c_int)]
        lib.mlvc_backend_io_shape.argtypes = [C.c_void_p, C.c_int, C.c_int, _i64p, C.POINTER(C.c_int)]
        lib.mlvc_backend_run.argtypes = [C.c_void_p, C.POINTER(C.c_void_p), C.POINTER(_u16p)]
        lib.mlvc_backend_io_dtype.argtypes = [C.c_void_p, C.c_int, C.c_int, C.POINTER(C.c_int)]
        _u8pp = C.POINTER(C.POINTER(C.c_uint8))
        lib.mlvc_backend_configure_codec_io.argtypes = [C.c_void_p] + [C.c_int] * 4 + [C.c_float] + [C.c_int] * 5 + [
            C.c_size_t]
        lib.mlvc_backend_codec_slot_count.argtypes = [C.c_void_p, C.POINTER(C.c_size_t)]
        lib.mlvc_backend_encoder_input_yuv.argtypes = [C.c_void_p, C.c_size_t, _u8pp, _u8pp, _u8pp]
        lib.mlvc_backend_decoder_output_yuv.argtypes = [C.c_void_p, C.c_size_t, _u8pp, _u8pp, _u8pp]
        lib.mlvc_backend_submit_encoder.argtypes = [C.c_void_p, C.c_size_t, C.c_int]
        lib.mlvc_backend_submit_decoder.argtypes = [C.c_void_p, C.c_size_t, C.c_int]
        lib.mlvc_backend_codec_tensor_count.argtypes = [C.c_void_p, C.c_size_t, C.c_int, C.POINTER(C.c_int)]
        lib.mlvc_backend_encoder_output.argtypes = [C.c_void_p, C.c_size_t, C.c_int, C.POINTER(C.c_void_p),
                                                    C.POINTER(C.c_size_t)]
        lib.mlvc_backend_decoder_input.argtypes = [C.c_void_p, C.c_size_t, C.c_int, C.POINTER(C.c_void_p),
                                                   C.POINTER(C.c_size_t)]
        lib.mlvc_backend_wait_codec_slot.argtypes = [C.c_void_p, C.c_size_t]
        lib.mlvc_frame_padding.argtypes = [C.c_int] * 4 + [C.POINTER(C.c_int)]
        lib.mlvc_backend_reset_state.argtypes = [C.c_void_p]
        lib.mlvc_backend_available.argtypes = [C.c_char_p, C.c_size_t]
        lib.mlvc_hip_backend_upload_inputs.argtypes = [C.c_void_p, C.POINTER(C.c_void_p)]
        lib.mlvc_hip_backend_time_frames.argtypes = [C.c_void_p, C.c_int, C.POINTER(C.c_float)]
        lib.mlvc_hip_backend_time_frames_each.argtypes = [C.c_void_p, C.c_int, C.c_size_t, C.POINTER(C.c_float)]
        lib.mlvc_hip_backend_download_outputs.argtypes = [C.c_void_p, C.POINTER(_u16p)]
        lib.mlvc_hip_backend_launch_count.argtypes = [C.c_void_p, C.POINTER(C.c_int)]
        lib.mlvc_hip_backend_launch_info.argtypes = [C.c_void_p, C.c_int, C.c_char_p, C.c_size_t, C.c_char_p,
                                                     C.c_size_t, C.POINTER(C.c_double), C.POINTER(C.c_double)]
        lib.mlvc_hip_backend_time_launch.argtypes = [C.c_void_p, C.c_int, C.c_int, C.POINTER(C.c_float)]
        lib.mlvc_hip_backend_time_launch_cold.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_size_t,
                                                          C.POINTER(C.c_float)]
        lib.mlvc_synth_configs.argtypes = [C.c_char_p, C.c_size_t]
        lib.mlvc_synth_write.argtypes = [C.c_char_p, C.c_char_p, C.c_uint64]
        lib.mlvc_synth_input.argtypes = [C.c_char_p, C.c_int, C.c_int, C.c_uint64, _u16p, C.c_size_t]
        lib.mlvc_synth_bindings.argtypes = [C.c_char_p, _i64p, C.c_int, C.POINTER(C.c_int), C.POINTER(C.c_int)]
        lib.mlvc_aot_inspect.argtypes = [C.c_char_p, C.c_char_p, C.POINTER(C.c_int), C.POINTER(C.c_int),
                                         C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]
        lib.mlvc_model_config_json.argtypes = [C.c_char_p, C.c_char_p, C.c_size_t]
        lib.mlvc_model_verify_bundle.argtypes = [C.c_char_p]
        _lib = lib
    return _lib


def device_lib() -> C.CDLL:
    global _dev
    if _dev is None:
        _dev = _load(DEVICE_LIB)
        _dev.mlvc_hip_last_error.restype = C.c_char_p
    return _dev


def conv_variants() -> list[str]:
    """Names of the conv tile variants (index order); index 0 is the direct fallback."""
    lib = device_lib()
    lib.mlvc_hip_conv_variant_name.restype = C.c_char_p
    lib.mlvc_hip_conv_variant_name.argtypes = [C.c_int]
    names = []
    while True:
        name = lib.mlvc_hip_conv_variant_name(len(names)).decode()
        if name == "invalid":
            return names
        names.append(name)


def _check(rc: int) -> None:
    if rc != 0:
        raise MlvcError(backend_lib().mlvc_backend_last_error().decode())


def _ptrs(arrays):
    arr = (_u16p * len(arrays))()
    for i, a in enumerate(arrays):
        arr[i] = a.ctypes.data_as(_u16p)
    return arr


def _vptrs(arrays):
    arr = (C.c_void_p * len(arrays))()
    for i, a in enumerate(arrays):
        arr[i] = a.ctypes.data
    return arr


def frame_padding(width: int, height: int, model_width: int, model_height: int) -> tuple:
    """(left, right, top, bottom, rotated): frame_padding of core/src/yuv.cpp:325-337."""
    pad = (C.c_int * 5)()
    _check(backend_lib().mlvc_frame_padding(width, height, model_width, model_height, pad))
    return tuple(pad)


def yuv_frame_bytes(width: int, height: int) -> int:
    return width * height + 2 * (width // 2) * (height // 2)


def available_backends() -> list[str]:
    buf = C.create_string_buffer(4096)
    _check(backend_lib().mlvc_backend_available(buf, len(buf)))
    return [s for s in buf.value.decode().split(",") if s]


class Backend:
    """An mlvc::InferenceBackend created through the registry."""

    def __init__(self, model_dir: str | pathlib.Path, backend_name: str = "hip", device_id: int = 0,
                 num_threads: int = 0):
        self._lib = backend_lib()
        h = C.c_void_p()
        _check(self._lib.mlvc_backend_create(backend_name.encode(), str(model_dir).encode(), device_id, num_threads,
                                             C.byref(h)))
        self._h = h
        self.in_shapes: list[tuple[int, ...]] = []
        self.out_shapes: list[tuple[int, ...]] = []

    @property
    def name(self) -> str:
        return self._lib.mlvc_backend_name(self._h).decode()

    def close(self) -> None:
        if self._h:
            self._lib.mlvc_backend_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def _shapes(self, is_output: int) -> list[tuple[int, ...]]:
        n = C.c_int()
        _check(self._lib.mlvc_backend_io_count(self._h, is_output, C.byref(n)))
        out = []
        for i in range(n.value):
            s = (C.c_int64 * 4)()
            r = C.c_int()
            _check(self._lib.mlvc_backend_io_shape(self._h, is_output, i, s, C.byref(r)))
            out.append(tuple(int(s[j]) for j in range(r.value)))
        return out

    def load(self, model_name: str, bindings=()) -> None:
        flat = (C.c_int64 * max(1, 2 * len(bindings)))(*[v for b in bindings for v in b])
        _check(self._lib.mlvc_backend_load(self._h, model_name.encode(), flat, len(bindings)))
        self.in_shapes = self._shapes(0)
        self.out_shapes = self._shapes(1)
        self.in_dtypes = []
        for i in range(len(self.in_shapes)):
            t = C.c_int()
            _check(self._lib.mlvc_backend_io_dtype(self._h, 0, i, C.byref(t)))
            self.in_dtypes.append(np.int32 if t.value == 1 else np.uint16)

    def _check_inputs(self, inputs):
        """FP16 inputs as uint16 bit patterns; INT32 control inputs as int32."""
        if len(inputs) != len(self.in_shapes):
            raise MlvcError("graph input count mismatch")
        arrs = []
        for a, s, t in zip(inputs, self.in_shapes, self.in_dtypes):
            a = np.ascontiguousarray(a, dtype=t)
            if a.size != int(np.prod(s)):
                raise MlvcError("graph input shape mismatch")
            arrs.append(a)
        return arrs

    def run(self, inputs) -> list[np.ndarray]:
        arrs = self._check_inputs(inputs)
        outs = [np.empty(s, dtype=np.uint16) for s in self.out_shapes]
        _check(self._lib.mlvc_backend_run(self._h, _vptrs(arrs), _ptrs(outs)))
        return outs

    # ---- BufferedCodecBackend (backend.hpp:64-96) ----
    def configure_codec_io(self, width: int, height: int, model_width: int, model_height: int,
                           pixel_range: float = 1.0, padding=None, slots: int = 2) -> tuple:
        """padding = (left, right, top, bottom, rotated); default frame_padding()."""
        pad = padding if padding is not None else frame_padding(width, height, model_width, model_height)
        _check(self._lib.mlvc_backend_configure_codec_io(self._h, width, height, model_width, model_height,
                                                         pixel_range, *[int(v) for v in pad], slots))
        self.codec = (width, height)
        return pad

    def codec_slot_count(self) -> int:
        n = C.c_size_t()
        _check(self._lib.mlvc_backend_codec_slot_count(self._h, C.byref(n)))
        return n.value

    def _frame(self, fn, slot: int, writable: bool) -> np.ndarray:
        y, u, v = (C.POINTER(C.c_uint8)(), C.POINTER(C.c_uint8)(), C.POINTER(C.c_uint8)())
        _check(fn(self._h, slot, C.byref(y), C.byref(u), C.byref(v)))
        w, h = self.codec
        n = yuv_frame_bytes(w, h)
        # The three planes are contiguous in the slot's pinned buffer.
        a = np.ctypeslib.as_array(y, shape=(n,))
        a.flags.writeable = writable
        return a

    def encoder_input_yuv(self, slot: int) -> np.ndarray:
        """Writable view of the slot's pinned I420 frame (Y, U, V back to back)."""
        return self._frame(self._lib.mlvc_backend_encoder_input_yuv, slot, True)

    def decoder_output_yuv(self, slot: int) -> np.ndarray:
        return self._frame(self._lib.mlvc_backend_decoder_output_yuv, slot, False)

    def submit_encoder(self, slot: int, shifted_q: int) -> None:
        _check(self._lib.mlvc_backend_submit_encoder(self._h, slot, shifted_q))

    def submit_decoder(self, slot: int, shifted_q: int) -> None:
        _check(self._lib.mlvc_backend_submit_decoder(self._h, slot, shifted_q))

    def wait_codec_slot(self, slot: int) -> None:
        _check(self._lib.mlvc_backend_wait_codec_slot(self._h, slot))

    def _tensors(self, slot: int, decoder: bool) -> list[np.ndarray]:
        n = C.c_int()
        _check(self._lib.mlvc_backend_codec_tensor_count(self._h, slot, int(decoder), C.byref(n)))
        fn = self._lib.mlvc_backend_decoder_input if decoder else self._lib.mlvc_backend_encoder_output
        out = []
        for i in range(n.value):
            p, nb = C.c_void_p(), C.c_size_t()
            _check(fn(self._h, slot, i, C.byref(p), C.byref(nb)))
            a = np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_uint16)), shape=(nb.value // 2,))
            a.flags.writeable = decoder
            out.append(a)
        return out

    def encoder_outputs(self, slot: int) -> list[np.ndarray]:
        """Views of the slot's pinned external outputs (FP16 bits, flat, graph order)."""
        return self._tensors(slot, False)

    def decoder_inputs(self, slot: int) -> list[np.ndarray]:
        """Writable views of the slot's pinned external inputs other than q_index_shifted."""
        return self._tensors(slot, True)

    def reset_state(self) -> None:
        _check(self._lib.mlvc_backend_reset_state(self._h))

    # ---- device-resident measurement helpers ("hip" backend only) ----
    def upload_inputs(self, inputs) -> None:
        arrs = self._check_inputs(inputs)
        _check(self._lib.mlvc_hip_backend_upload_inputs(self._h, _vptrs(arrs)))

    def time_frames(self, frames: int) -> float:
        ms = C.c_float()
        _check(self._lib.mlvc_hip_backend_time_frames(self._h, frames, C.byref(ms)))
        return ms.value

    def time_frames_each(self, frames: int, flush_bytes: int = 0) -> np.ndarray:
        """Per-frame GPU ms of `frames` back-to-back replays; flush_bytes > 0
        evicts the caches with a device copy before each (untimed)."""
        ms = np.zeros(frames, dtype=np.float32)
        _check(self._lib.mlvc_hip_backend_time_frames_each(
            self._h, frames, flush_bytes, ms.ctypes.data_as(C.POINTER(C.c_float))))
        return ms

    def download_outputs(self) -> list[np.ndarray]:
        outs = [np.empty(s, dtype=np.uint16) for s in self.out_shapes]
        _check(self._lib.mlvc_hip_backend_download_outputs(self._h, _ptrs(outs)))
        return outs

    def launches(self) -> list[dict]:
        n = C.c_int()
        _check(self._lib.mlvc_hip_backend_launch_count(self._h, C.byref(n)))
        out = []
        for i in range(n.value):
            name = C.create_string_buffer(256)
            kind = C.create_string_buffer(256)
            fl, by = C.c_double(), C.c_double()
            _check(self._lib.mlvc_hip_backend_launch_info(self._h, i, name, 256, kind, 256, C.byref(fl), C.byref(by)))
            out.append({"index": i, "name": name.value.decode(), "kind": kind.value.decode(),
                        "flops": fl.value, "bytes": by.value})
        return out

    def time_launch(self, index: int, reps: int) -> float:
        ms = C.c_float()
        _check(self._lib.mlvc_hip_backend_time_launch(self._h, index, reps, C.byref(ms)))
        return ms.value

    def time_launch_cold(self, index: int, reps: int, flush_bytes: int) -> np.ndarray:
        """Per-launch GPU ms of `reps` single launches of kernel `index`, each
        after a device copy of flush_bytes / 2 that evicts L2 and the MALL."""
        ms = np.zeros(reps, dtype=np.float32)
        _check(self._lib.mlvc_hip_backend_time_launch_cold(
            self._h, index, reps, flush_bytes, ms.ctypes.data_as(C.POINTER(C.c_float))))
        return ms


# ---- seeded synthetic graphs ----------------------------------------------

def synth_configs() -> list[str]:
    buf = C.create_string_buffer(4096)
    _check(backend_lib().mlvc_synth_configs(buf, len(buf)))
    return buf.value.decode().split(",")


def synth_write(config: str, out_dir: str | pathlib.Path, seed: int = 0) -> None:
    _check(backend_lib().mlvc_synth_write(config.encode(), str(out_dir).encode(), seed))


def synth_input(config: str, index: int, frame: int, shape, seed: int = 0) -> np.ndarray:
    a = np.empty(shape, dtype=np.uint16)
    _check(backend_lib().mlvc_synth_input(config.encode(), index, frame, seed, a.ctypes.data_as(_u16p), a.size))
    return a


def synth_bindings(config: str) -> tuple[list[tuple[int, int]], int]:
    pairs = (C.c_int64 * 16)()
    n, frames = C.c_int(), C.c_int()
    _check(backend_lib().mlvc_synth_bindings(config.encode(), pairs, 8, C.byref(n), C.byref(frames)))
    return [(int(pairs[2 * i]), int(pairs[2 * i + 1])) for i in range(n.value)], frames.value


def aot_inspect(model_dir, model_name: str) -> dict:
    """Loads and validates aot/<model>/graph.pb without touching a GPU."""
    nodes, tensors = C.c_int(), C.c_int()
    arena, weights = C.c_uint64(), C.c_uint64()
    _check(backend_lib().mlvc_aot_inspect(str(model_dir).encode(), model_name.encode(), C.byref(nodes),
                                          C.byref(tensors), C.byref(arena), C.byref(weights)))
    return {"nodes": nodes.value, "tensors": tensors.value, "arena_bytes": arena.value,
            "weights_bytes": weights.value}


def model_config(model_dir) -> dict:
    """ModelConfig of a model directory: metadata.pb checked against model_bundle.pb and validated
    (reference core/src/model.cpp:150-183), plus the derived feature/latent/hyperprior sizes."""
    buf = C.create_string_buffer(8192)
    _check(backend_lib().mlvc_model_config_json(str(model_dir).encode(), buf, len(buf)))
    return json.loads(buf.value.decode())


def verify_bundle(model_dir) -> None:
    """Checks every artifact listed in model_bundle.pb for presence, size and SHA-256."""
    _check(backend_lib().mlvc_model_verify_bundle(str(model_dir).encode()))


def bundle_info(model_dir) -> dict:
    """model_bundle.pb of a location: profile, model_version, width, height, artifacts [{path, size}]."""
    n = 1 << 16
    while True:
        buf = C.create_string_buffer(n)
        rc = backend_lib().mlvc_model_bundle_json(str(model_dir).encode(), buf, len(buf))
        if rc == 0:
            return json.loads(buf.value.decode())
        if "buffer too small" not in backend_lib().mlvc_backend_last_error().decode() or n >= 1 << 24:
            _check(rc)
        n *= 4


def embedded_profiles() -> list[str]:
    """Profiles of the linked embedded model image (empty when none is linked)."""
    buf = C.create_string_buffer(1 << 16)
    _check(backend_lib().mlvc_model_embedded_profiles(buf, len(buf)))
    return [p for p in buf.value.decode().split("\n") if p]


def default_model_location() -> str:
    """'embedded:mlvc-psnr-v1' if embedded, else the first embedded profile's location, else ''."""
    buf = C.create_string_buffer(4096)
    _check(backend_lib().mlvc_model_default_location(buf, len(buf)))
    return buf.value.decode()
