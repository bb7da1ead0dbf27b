"""Device memory, streams and events through the HIP runtime the library
links (libamdhip64 from ROCm), for tests and benchmarks that drive the C ABI
from Python. Using the library's own runtime keeps one HIP runtime per
process (a second copy, such as the one bundled with a framework, would see
no device once this one is initialised).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import hip as _hip

_rt = None
H2D, D2H, D2D = 1, 2, 3


def rt():
    global _rt
    if _rt is None:
        _hip.lib()                        # resolves libamdhip64 via the library's rpath
        R = C.CDLL("libamdhip64.so.7")
        vp, sz, i = C.c_void_p, C.c_size_t, C.c_int
        for name, res, args in [
            ("hipMalloc", i, [C.POINTER(vp), sz]), ("hipFree", i, [vp]),
            ("hipMemcpy", i, [vp, vp, sz, i]), ("hipMemset", i, [vp, i, sz]),
            ("hipDeviceSynchronize", i, []), ("hipStreamSynchronize", i, [vp]),
            ("hipEventCreate", i, [C.POINTER(vp)]), ("hipEventDestroy", i, [vp]),
            ("hipEventRecord", i, [vp, vp]), ("hipEventSynchronize", i, [vp]),
            ("hipEventElapsedTime", i, [C.POINTER(C.c_float), vp, vp]),
            ("hipGetErrorString", C.c_char_p, [i]), ("hipGetDeviceCount", i, [C.POINTER(i)]),
            ("hipMemGetInfo", i, [C.POINTER(sz), C.POINTER(sz)]),
            ("hipMemcpyAsync", i, [vp, vp, sz, i, vp]),
            ("hipStreamBeginCapture", i, [vp, i]), ("hipStreamEndCapture", i, [vp, C.POINTER(vp)]),
            ("hipGraphInstantiate", i, [C.POINTER(vp), vp, vp, vp, sz]), ("hipGraphLaunch", i, [vp, vp]),
            ("hipGraphExecDestroy", i, [vp]), ("hipGraphDestroy", i, [vp]),
        ]:
            fn = getattr(R, name)
            fn.restype, fn.argtypes = res, args
        _rt = R
    return _rt


def check(rc, what="hip"):
    if rc:
        raise RuntimeError(f"{what}: {rt().hipGetErrorString(rc).decode()}")


def device_count() -> int:
    n = C.c_int(0)
    rc = rt().hipGetDeviceCount(C.byref(n))
    return n.value if rc == 0 else 0


def synchronize():
    check(rt().hipDeviceSynchronize(), "hipDeviceSynchronize")


def mem_info():
    free, total = C.c_size_t(), C.c_size_t()
    check(rt().hipMemGetInfo(C.byref(free), C.byref(total)), "hipMemGetInfo")
    return free.value, total.value


class Buf:
    """An owned device allocation with typed copies to and from numpy."""

    def __init__(self, nbytes: int, dtype=np.uint8, shape=None):
        self.nbytes = int(nbytes)
        self.dtype = np.dtype(dtype)
        self.shape = shape if shape is not None else (self.nbytes // self.dtype.itemsize,)
        p = C.c_void_p()
        check(rt().hipMalloc(C.byref(p), max(self.nbytes, 1)), f"hipMalloc({self.nbytes})")
        self.ptr = p.value

    @classmethod
    def empty(cls, shape, dtype=np.float32):
        shape = (shape,) if isinstance(shape, int) else tuple(shape)
        return cls(int(np.prod(shape)) * np.dtype(dtype).itemsize, dtype, shape)

    @classmethod
    def of(cls, a: np.ndarray):
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes, a.dtype, a.shape)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        check(rt().hipMemcpy(self.ptr, a.ctypes.data, a.nbytes, H2D), "hipMemcpy H2D")

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        check(rt().hipDeviceSynchronize(), "hipDeviceSynchronize")
        check(rt().hipMemcpy(out.ctypes.data, self.ptr, out.nbytes, D2H), "hipMemcpy D2H")
        return out

    def zero(self):
        check(rt().hipMemset(self.ptr, 0, self.nbytes), "hipMemset")

    def data_ptr(self) -> int:
        return self.ptr

    def free(self):
        if self.ptr:
            rt().hipFree(self.ptr)
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def copy_async(dst: int, src: int, nbytes: int, kind: int, stream):
    check(rt().hipMemcpyAsync(dst, src, nbytes, kind, stream), "hipMemcpyAsync")


class Graph:
    """Work issued on one stream by `fn()` captured into a HIP graph
    (relaxed capture mode) and replayed with launch(). The captured calls
    must issue only kernels, event records and copies between device
    buffers on that stream: nothing that waits on the host."""

    def __init__(self, stream, fn):
        self.stream = stream
        self.graph = C.c_void_p()
        self.exec = C.c_void_p()
        check(rt().hipStreamBeginCapture(stream, 2), "hipStreamBeginCapture")
        try:
            fn()
        finally:
            rc = rt().hipStreamEndCapture(stream, C.byref(self.graph))
        check(rc, "hipStreamEndCapture")
        check(rt().hipGraphInstantiate(C.byref(self.exec), self.graph, None, None, 0), "hipGraphInstantiate")

    def launch(self):
        check(rt().hipGraphLaunch(self.exec, self.stream), "hipGraphLaunch")

    def free(self):
        if self.exec:
            rt().hipGraphExecDestroy(self.exec)
            self.exec = C.c_void_p()
        if self.graph:
            rt().hipGraphDestroy(self.graph)
            self.graph = C.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Event:
    def __init__(self):
        e = C.c_void_p()
        check(rt().hipEventCreate(C.byref(e)), "hipEventCreate")
        self.e = e.value

    def record(self, stream=None):
        check(rt().hipEventRecord(self.e, stream), "hipEventRecord")

    def synchronize(self):
        check(rt().hipEventSynchronize(self.e), "hipEventSynchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        check(rt().hipEventElapsedTime(C.byref(ms), self.e, end.e), "hipEventElapsedTime")
        return ms.value

    def __del__(self):
        try:
            if self.e:
                rt().hipEventDestroy(self.e)
        except Exception:
            pass
