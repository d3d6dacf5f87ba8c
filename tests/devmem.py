"""Device buffers for GPU tests through the device C ABI
(include/mlvc_hip_device.h)."""

import ctypes as C

import numpy as np

import mlvc_hip


class Dev:
    """Device buffers through the device C ABI (include/mlvc_hip_device.h)."""

    def __init__(self):
        self.lib = mlvc_hip.device_lib()
        L = self.lib
        L.mlvc_hip_malloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        L.mlvc_hip_free.argtypes = [C.c_void_p]
        L.mlvc_hip_memcpy_h2d.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]
        L.mlvc_hip_memcpy_d2h.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]
        L.mlvc_hip_stream_synchronize.argtypes = [C.c_void_p]
        L.mlvc_hip_yuv420_to_model.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p] + [C.c_int] * 5 + [C.c_void_p]
        L.mlvc_hip_model_to_yuv420.argtypes = [C.c_void_p, C.c_void_p] + [C.c_int] * 7 + [C.c_float, C.c_void_p]
        self.bufs = []

    def check(self, rc):
        if rc != 0:
            raise mlvc_hip.MlvcError(self.lib.mlvc_hip_last_error().decode())

    def alloc(self, nbytes):
        p = C.c_void_p()
        self.check(self.lib.mlvc_hip_malloc(C.byref(p), max(nbytes, 16)))
        self.bufs.append(p)
        return p

    def put(self, a):
        a = np.ascontiguousarray(a)
        p = self.alloc(a.nbytes)
        self.check(self.lib.mlvc_hip_memcpy_h2d(p, a.ctypes.data, a.nbytes, None))
        return p

    def get(self, p, shape, dtype):
        a = np.empty(shape, dtype)
        self.check(self.lib.mlvc_hip_stream_synchronize(None))
        self.check(self.lib.mlvc_hip_memcpy_d2h(a.ctypes.data, p, a.nbytes, None))
        self.check(self.lib.mlvc_hip_stream_synchronize(None))
        return a

    def close(self):
        for p in self.bufs:
            self.lib.mlvc_hip_free(p)
        self.bufs = []
