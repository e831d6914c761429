"""A device buffer for tests that drive the device-pointer entry points."""
import ctypes as C

import numpy as np

from autoresearch_amd import engine


class DevBuf:
    """A device buffer from the HIP runtime libfgpt.so is linked against
    (test plumbing only: the step under test takes device pointers)."""

    hip = None

    def __init__(self, arr):
        if DevBuf.hip is None:
            engine.load_library()
            DevBuf.hip = C.CDLL("libamdhip64.so.7")
        self.nbytes = arr.nbytes
        self.dtype = arr.dtype
        self.p = C.c_void_p()
        assert DevBuf.hip.hipMalloc(C.byref(self.p), C.c_size_t(self.nbytes)) == 0
        self.put(arr)

    def put(self, arr):
        a = np.ascontiguousarray(arr, dtype=self.dtype)
        assert DevBuf.hip.hipMemcpy(self.p, a.ctypes.data_as(C.c_void_p), C.c_size_t(self.nbytes), 1) == 0
        # a pageable hipMemcpy may return before its DMA lands, and the null
        # stream it runs on is not ordered against the engine's non-blocking
        # stream: wait for the device before the buffer is handed over
        assert DevBuf.hip.hipDeviceSynchronize() == 0

    def get(self):
        out = np.empty(self.nbytes // self.dtype.itemsize, self.dtype)
        assert DevBuf.hip.hipDeviceSynchronize() == 0
        assert DevBuf.hip.hipMemcpy(out.ctypes.data_as(C.c_void_p), self.p, C.c_size_t(self.nbytes), 2) == 0
        return out

    @property
    def ptr(self):
        return self.p.value

    def free(self):
        DevBuf.hip.hipFree(self.p)
