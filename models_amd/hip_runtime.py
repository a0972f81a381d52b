"""Device memory, copies and events through the HIP runtime that libjmodels_attn.so itself links.

The attention library links /opt/rocm's ``libamdhip64.so.7``; loading a second HIP runtime into
the same process (for example the one bundled with a PyTorch wheel, which has the same soname)
leaves one of them without devices. Tests and the benchmark therefore allocate device buffers and
time kernels through this thin ctypes layer over the runtime already loaded with the library.
"""

from __future__ import annotations

import ctypes
from typing import Optional

import numpy as np

from . import attention

_hip: Optional[ctypes.CDLL] = None

H2D = 1
D2H = 2
D2D = 3


def hip() -> ctypes.CDLL:
    global _hip
    if _hip is None:
        attention.load_library()  # resolves libamdhip64.so.7 through the library's RUNPATH
        lib = ctypes.CDLL("libamdhip64.so.7", mode=ctypes.RTLD_GLOBAL)
        vp, sz, i32 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
        sig = {
            "hipMalloc": [ctypes.POINTER(vp), sz],
            "hipFree": [vp],
            "hipMemcpy": [vp, vp, sz, i32],
            "hipMemcpyAsync": [vp, vp, sz, i32, vp],
            "hipMemset": [vp, i32, sz],
            "hipDeviceSynchronize": [],
            "hipStreamSynchronize": [vp],
            "hipEventCreate": [ctypes.POINTER(vp)],
            "hipEventDestroy": [vp],
            "hipEventRecord": [vp, vp],
            "hipEventSynchronize": [vp],
            "hipEventElapsedTime": [ctypes.POINTER(ctypes.c_float), vp, vp],
            "hipSetDevice": [i32],
            "hipStreamBeginCapture": [vp, i32],
            "hipStreamEndCapture": [vp, ctypes.POINTER(vp)],
            "hipGraphInstantiate": [ctypes.POINTER(vp), vp, vp, vp, sz],
            "hipGraphLaunch": [vp, vp],
            "hipGraphExecDestroy": [vp],
            "hipGraphDestroy": [vp],
        }
        for name, args in sig.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = i32
        lib.hipGetErrorString.argtypes = [i32]
        lib.hipGetErrorString.restype = ctypes.c_char_p
        _hip = lib
    return _hip


def check(err: int, what: str) -> None:
    if err != 0:
        raise RuntimeError(f"{what}: {hip().hipGetErrorString(err).decode()}")


class DeviceArray:
    """A device allocation holding ``count`` elements of ``dtype`` (float32 by default)."""

    def __init__(self, count: int, dtype=np.float32):
        self.dtype = np.dtype(dtype)
        self.count = int(count)
        self.nbytes = self.count * self.dtype.itemsize
        p = ctypes.c_void_p()
        check(hip().hipMalloc(ctypes.byref(p), max(self.nbytes, 1)), "hipMalloc")
        self.ptr = p.value

    @classmethod
    def from_host(cls, array: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(array)
        d = cls(a.size, a.dtype)
        d.upload(a)
        return d

    def upload(self, array: np.ndarray, offset_elems: int = 0) -> None:
        a = np.ascontiguousarray(array, dtype=self.dtype)
        assert offset_elems + a.size <= self.count
        check(hip().hipMemcpy(self.ptr + offset_elems * self.dtype.itemsize, a.ctypes.data,
                              a.nbytes, H2D), "hipMemcpy H2D")

    def download(self, count: Optional[int] = None, offset_elems: int = 0) -> np.ndarray:
        count = self.count - offset_elems if count is None else count
        out = np.empty(count, self.dtype)
        check(hip().hipMemcpy(out.ctypes.data, self.ptr + offset_elems * self.dtype.itemsize,
                              out.nbytes, D2H), "hipMemcpy D2H")
        return out

    def zero(self) -> None:
        check(hip().hipMemset(self.ptr, 0, self.nbytes), "hipMemset")

    def at(self, offset_elems: int) -> int:
        """Device address of element ``offset_elems``."""
        return self.ptr + offset_elems * self.dtype.itemsize

    def free(self) -> None:
        if self.ptr:
            check(hip().hipFree(self.ptr), "hipFree")
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Event:
    """hipEvent_t recorded on a given stream (the attention context's stream for kernel timing)."""

    def __init__(self):
        e = ctypes.c_void_p()
        check(hip().hipEventCreate(ctypes.byref(e)), "hipEventCreate")
        self.handle = e.value

    def record(self, stream: int) -> None:
        check(hip().hipEventRecord(self.handle, stream or None), "hipEventRecord")

    def synchronize(self) -> None:
        check(hip().hipEventSynchronize(self.handle), "hipEventSynchronize")

    def elapsed_ms(self, later: "Event") -> float:
        ms = ctypes.c_float()
        check(hip().hipEventElapsedTime(ctypes.byref(ms), self.handle, later.handle),
              "hipEventElapsedTime")
        return float(ms.value)

    def __del__(self):
        try:
            if self.handle:
                hip().hipEventDestroy(self.handle)
        except Exception:
            pass


class Graph:
    """A HIP graph captured from the work a callable enqueues on ``stream``.

    Capture records launches without running them; the callable must not allocate, synchronize
    or memset (run it once eagerly first so every scratch buffer already exists)."""

    RELAXED = 2  # hipStreamCaptureModeRelaxed

    def __init__(self, stream: int, enqueue):
        check(hip().hipStreamBeginCapture(stream, self.RELAXED), "hipStreamBeginCapture")
        graph = ctypes.c_void_p()
        try:
            enqueue()
        finally:
            check(hip().hipStreamEndCapture(stream, ctypes.byref(graph)), "hipStreamEndCapture")
        self.graph = graph.value
        exe = ctypes.c_void_p()
        check(hip().hipGraphInstantiate(ctypes.byref(exe), self.graph, None, None, 0),
              "hipGraphInstantiate")
        self.exec = exe.value
        self.stream = stream

    def launch(self) -> None:
        check(hip().hipGraphLaunch(self.exec, self.stream), "hipGraphLaunch")

    def destroy(self) -> None:
        if getattr(self, "exec", None):
            hip().hipGraphExecDestroy(self.exec)
            self.exec = None
        if getattr(self, "graph", None):
            hip().hipGraphDestroy(self.graph)
            self.graph = None


def device_synchronize() -> None:
    check(hip().hipDeviceSynchronize(), "hipDeviceSynchronize")
