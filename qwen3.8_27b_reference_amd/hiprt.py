"""Minimal ctypes access to the HIP runtime that libqk.so itself links (/opt/rocm libamdhip64),
for device buffers, copies, streams and events in tests and the benchmark.  Plumbing only.

torch is deliberately not used: its wheel bundles a second HIP/HSA runtime, and two runtimes in
one process do not share device allocations.
"""
import ctypes
import os

import numpy as np

_CANDIDATES = ["/opt/rocm/lib/libamdhip64.so.7", "/opt/rocm/lib/libamdhip64.so", "libamdhip64.so.7"]

H2D, D2H, D2D = 1, 2, 3


class HipError(RuntimeError):
    pass


class Hip:
    def __init__(self):
        last = None
        for c in _CANDIDATES:
            try:
                self.lib = ctypes.CDLL(c, mode=ctypes.RTLD_GLOBAL)
                break
            except OSError as e:  # pragma: no cover - depends on the image
                last = e
        else:
            raise HipError(f"cannot load libamdhip64: {last}")
        L = self.lib
        vp, sz = ctypes.c_void_p, ctypes.c_size_t
        L.hipMalloc.argtypes = [ctypes.POINTER(vp), sz]
        L.hipFree.argtypes = [vp]
        L.hipMemcpy.argtypes = [vp, vp, sz, ctypes.c_int]
        L.hipMemcpyAsync.argtypes = [vp, vp, sz, ctypes.c_int, vp]
        L.hipMemset.argtypes = [vp, ctypes.c_int, sz]
        L.hipMemsetAsync.argtypes = [vp, ctypes.c_int, sz, vp]
        L.hipStreamCreate.argtypes = [ctypes.POINTER(vp)]
        L.hipStreamDestroy.argtypes = [vp]
        L.hipStreamSynchronize.argtypes = [vp]
        L.hipEventCreate.argtypes = [ctypes.POINTER(vp)]
        L.hipEventDestroy.argtypes = [vp]
        L.hipEventRecord.argtypes = [vp, vp]
        L.hipEventSynchronize.argtypes = [vp]
        L.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), vp, vp]
        L.hipGetDeviceCount.argtypes = [ctypes.POINTER(ctypes.c_int)]
        L.hipDeviceGetAttribute.argtypes = [ctypes.POINTER(ctypes.c_int), ctypes.c_int, ctypes.c_int]
        L.hipGetErrorString.restype = ctypes.c_char_p
        L.hipGetErrorString.argtypes = [ctypes.c_int]
        L.hipMemGetInfo.argtypes = [ctypes.POINTER(sz), ctypes.POINTER(sz)]
        L.hipStreamBeginCapture.argtypes = [vp, ctypes.c_int]
        L.hipStreamEndCapture.argtypes = [vp, ctypes.POINTER(vp)]
        L.hipGraphInstantiate.argtypes = [ctypes.POINTER(vp), vp, vp, ctypes.c_char_p, sz]
        L.hipGraphLaunch.argtypes = [vp, vp]
        L.hipGraphExecDestroy.argtypes = [vp]
        L.hipGraphDestroy.argtypes = [vp]
        L.hipDeviceSynchronize.argtypes = []

    def _ck(self, rc, what):
        if rc != 0:
            raise HipError(f"{what}: {self.lib.hipGetErrorString(rc).decode()} ({rc})")

    def device_count(self):
        n = ctypes.c_int(0)
        rc = self.lib.hipGetDeviceCount(ctypes.byref(n))
        return n.value if rc == 0 else 0

    def attribute(self, attr, dev=0):
        v = ctypes.c_int(0)
        self._ck(self.lib.hipDeviceGetAttribute(ctypes.byref(v), attr, dev), "hipDeviceGetAttribute")
        return v.value

    def mem_info(self):
        free, total = ctypes.c_size_t(), ctypes.c_size_t()
        self._ck(self.lib.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)), "hipMemGetInfo")
        return free.value, total.value

    def malloc(self, nbytes):
        p = ctypes.c_void_p()
        self._ck(self.lib.hipMalloc(ctypes.byref(p), max(int(nbytes), 1)), f"hipMalloc({nbytes})")
        return p.value

    def free(self, p):
        self._ck(self.lib.hipFree(p), "hipFree")

    def htod(self, dst, a):
        a = np.ascontiguousarray(a)
        self._ck(self.lib.hipMemcpy(dst, a.ctypes.data, a.nbytes, H2D), "hipMemcpy H2D")

    def dtoh(self, a, src):
        self._ck(self.lib.hipMemcpy(a.ctypes.data, src, a.nbytes, D2H), "hipMemcpy D2H")
        return a

    def dtod(self, dst, src, nbytes):
        self._ck(self.lib.hipMemcpy(dst, src, nbytes, D2D), "hipMemcpy D2D")

    def memset(self, p, value, nbytes):
        self._ck(self.lib.hipMemset(p, value, nbytes), "hipMemset")

    def sync(self):
        self._ck(self.lib.hipDeviceSynchronize(), "hipDeviceSynchronize")

    def stream_create(self):
        s = ctypes.c_void_p()
        self._ck(self.lib.hipStreamCreate(ctypes.byref(s)), "hipStreamCreate")
        return s.value

    def stream_sync(self, s):
        self._ck(self.lib.hipStreamSynchronize(s), "hipStreamSynchronize")

    def stream_destroy(self, s):
        self._ck(self.lib.hipStreamDestroy(s), "hipStreamDestroy")

    def event_create(self):
        e = ctypes.c_void_p()
        self._ck(self.lib.hipEventCreate(ctypes.byref(e)), "hipEventCreate")
        return e.value

    def event_record(self, e, stream=0):
        self._ck(self.lib.hipEventRecord(e, stream), "hipEventRecord")

    def event_sync(self, e):
        self._ck(self.lib.hipEventSynchronize(e), "hipEventSynchronize")

    def elapsed_ms(self, e0, e1):
        ms = ctypes.c_float()
        self._ck(self.lib.hipEventElapsedTime(ctypes.byref(ms), e0, e1), "hipEventElapsedTime")
        return ms.value

    def event_destroy(self, e):
        self._ck(self.lib.hipEventDestroy(e), "hipEventDestroy")

    # -- graphs (capture on a non-default stream) ---------------------------------------------
    def begin_capture(self, stream):
        self._ck(self.lib.hipStreamBeginCapture(stream, 0), "hipStreamBeginCapture")  # global mode

    def end_capture(self, stream):
        g = ctypes.c_void_p()
        self._ck(self.lib.hipStreamEndCapture(stream, ctypes.byref(g)), "hipStreamEndCapture")
        ex = ctypes.c_void_p()
        self._ck(self.lib.hipGraphInstantiate(ctypes.byref(ex), g, None, None, 0), "hipGraphInstantiate")
        return g.value, ex.value

    def graph_launch(self, exec_, stream):
        self._ck(self.lib.hipGraphLaunch(exec_, stream), "hipGraphLaunch")

    def graph_destroy(self, graph, exec_):
        self._ck(self.lib.hipGraphExecDestroy(exec_), "hipGraphExecDestroy")
        self._ck(self.lib.hipGraphDestroy(graph), "hipGraphDestroy")


class Buf:
    """A device allocation with numpy upload/download helpers."""

    def __init__(self, hip, nbytes):
        self.hip = hip
        self.nbytes = int(nbytes)
        self.ptr = hip.malloc(self.nbytes)

    @classmethod
    def of(cls, hip, a):
        a = np.ascontiguousarray(a)
        b = cls(hip, a.nbytes)
        hip.htod(b.ptr, a)
        return b

    def get(self, dtype, shape=None):
        a = np.empty(self.nbytes // np.dtype(dtype).itemsize, dtype)
        self.hip.sync()
        self.hip.dtoh(a, self.ptr)
        return a if shape is None else a.reshape(shape)

    def fill_nan(self):
        a = np.full(self.nbytes // 4, np.nan, np.float32)
        self.hip.htod(self.ptr, a)

    def close(self):
        if self.ptr:
            self.hip.free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
