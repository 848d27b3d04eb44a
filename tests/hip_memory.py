"""Device memory for the caller's side of the C ABI in GPU tests (plumbing):
hipMalloc / hipMemcpy / hipFree of the system HIP runtime through ctypes."""

import ctypes

import numpy as np


class Hip:
    def __init__(self):
        self.lib = ctypes.CDLL("libamdhip64.so")
        self.lib.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
        self.lib.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        self.lib.hipFree.argtypes = [ctypes.c_void_p]
        self.lib.hipDeviceSynchronize.argtypes = []
        self.held = []

    def alloc(self, nbytes):
        p = ctypes.c_void_p()
        assert self.lib.hipMalloc(ctypes.byref(p), max(int(nbytes), 1)) == 0
        self.held.append(p.value)
        return p.value

    def upload(self, array):
        a = np.ascontiguousarray(array)
        p = self.alloc(a.nbytes)
        if a.nbytes:
            assert self.lib.hipMemcpy(ctypes.c_void_p(p), a.ctypes.data_as(ctypes.c_void_p), a.nbytes, 1) == 0
        return p

    def download(self, ptr, shape, dtype):
        out = np.empty(shape, dtype=dtype)
        if out.nbytes:
            assert self.lib.hipMemcpy(out.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(ptr), out.nbytes, 2) == 0
        return out

    def free_all(self):
        assert self.lib.hipDeviceSynchronize() == 0
        for p in self.held:
            self.lib.hipFree(ctypes.c_void_p(p))
        self.held = []
