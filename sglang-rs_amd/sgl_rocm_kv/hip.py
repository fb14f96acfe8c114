"""Minimal HIP runtime plumbing over ctypes: device memory, copies, streams
and events for the binding's users (tests, bench, smoke).

It loads the same ``libamdhip64.so.7`` that ``libsgl_rocm_kv.so`` links, so
pointers, streams and events are shared with the library. It deliberately
does not use torch: torch ships its own copy of the HIP runtime, and two
runtimes in one process would not share device pointers.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_ROCM_LIB = os.environ.get("ROCM_PATH", "/opt/rocm") + "/lib/libamdhip64.so.7"

_H2D, _D2H, _D2D = 1, 2, 3


class HipError(RuntimeError):
    def __init__(self, call: str, code: int, text: str):
        super().__init__(f"{call} failed: {text} ({code})")
        self.call, self.code = call, code


def _load():
    lib = ctypes.CDLL(_ROCM_LIB if os.path.exists(_ROCM_LIB) else "libamdhip64.so.7",
                      mode=ctypes.RTLD_GLOBAL)
    vp, sz, i32 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
    sig = {
        "hipGetDeviceCount": [ctypes.POINTER(i32)],
        "hipSetDevice": [i32],
        "hipGetDevice": [ctypes.POINTER(i32)],
        "hipMalloc": [ctypes.POINTER(vp), sz],
        "hipFree": [vp],
        "hipHostMalloc": [ctypes.POINTER(vp), sz, ctypes.c_uint],
        "hipHostFree": [vp],
        "hipMemcpy": [vp, vp, sz, i32],
        "hipMemcpyAsync": [vp, vp, sz, i32, vp],
        "hipMemset": [vp, i32, sz],
        "hipMemsetAsync": [vp, i32, sz, vp],
        "hipDeviceSynchronize": [],
        "hipStreamCreate": [ctypes.POINTER(vp)],
        "hipStreamDestroy": [vp],
        "hipStreamSynchronize": [vp],
        "hipStreamWaitEvent": [vp, vp, ctypes.c_uint],
        "hipEventCreate": [ctypes.POINTER(vp)],
        "hipEventDestroy": [vp],
        "hipEventRecord": [vp, vp],
        "hipEventSynchronize": [vp],
        "hipEventElapsedTime": [ctypes.POINTER(ctypes.c_float), vp, vp],
        "hipMemGetInfo": [ctypes.POINTER(sz), ctypes.POINTER(sz)],
    }
    for name, args in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = i32
    lib.hipGetErrorString.argtypes = [i32]
    lib.hipGetErrorString.restype = ctypes.c_char_p
    return lib


_lib = None


def lib():
    global _lib
    if _lib is None:
        _lib = _load()
    return _lib


def check(code: int, call: str):
    if code != 0:
        raise HipError(call, code, lib().hipGetErrorString(code).decode())


def device_count() -> int:
    n = ctypes.c_int(0)
    code = lib().hipGetDeviceCount(ctypes.byref(n))
    return n.value if code == 0 else 0


def set_device(d: int):
    check(lib().hipSetDevice(d), "hipSetDevice")


def synchronize():
    check(lib().hipDeviceSynchronize(), "hipDeviceSynchronize")


def mem_info():
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    check(lib().hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)), "hipMemGetInfo")
    return free.value, total.value


class DeviceBuffer:
    """An owned device allocation (hipMalloc) of ``nbytes`` bytes."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        check(lib().hipMalloc(ctypes.byref(p), max(self.nbytes, 1)), "hipMalloc")
        self.ptr = p.value

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray, offset: int = 0):
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes, "upload past the end of the buffer"
        check(lib().hipMemcpy(self.ptr + offset, a.ctypes.data, a.nbytes, _H2D), "hipMemcpy")

    def download(self, nbytes: int | None = None, offset: int = 0, dtype=np.uint8) -> np.ndarray:
        n = self.nbytes - offset if nbytes is None else int(nbytes)
        assert offset + n <= self.nbytes, "download past the end of the buffer"
        out = np.empty(n, dtype=np.uint8)
        check(lib().hipMemcpy(out.ctypes.data, self.ptr + offset, n, _D2H), "hipMemcpy")
        return out.view(dtype)

    def fill(self, byte: int, nbytes: int | None = None, offset: int = 0):
        n = self.nbytes - offset if nbytes is None else int(nbytes)
        check(lib().hipMemset(self.ptr + offset, byte, n), "hipMemset")

    def free(self):
        if self.ptr:
            check(lib().hipFree(self.ptr), "hipFree")
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class PinnedBuffer:
    """Page-locked host memory (hipHostMalloc) for the staging hop."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        check(lib().hipHostMalloc(ctypes.byref(p), max(self.nbytes, 1), 0), "hipHostMalloc")
        self.ptr = p.value

    def array(self) -> np.ndarray:
        return np.ctypeslib.as_array((ctypes.c_uint8 * self.nbytes).from_address(self.ptr))

    def free(self):
        if self.ptr:
            check(lib().hipHostFree(self.ptr), "hipHostFree")
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def memcpy_async(dst: int, src: int, nbytes: int, kind: str, stream: "Stream | None" = None):
    k = {"h2d": _H2D, "d2h": _D2H, "d2d": _D2D}[kind]
    check(lib().hipMemcpyAsync(dst, src, nbytes, k, stream.handle if stream else None),
          "hipMemcpyAsync")


class Stream:
    """A HIP stream at the default priority."""

    def __init__(self):
        s = ctypes.c_void_p()
        check(lib().hipStreamCreate(ctypes.byref(s)), "hipStreamCreate")
        self.handle = s.value

    def synchronize(self):
        check(lib().hipStreamSynchronize(self.handle), "hipStreamSynchronize")

    def wait(self, event: "Event"):
        check(lib().hipStreamWaitEvent(self.handle, event.handle, 0), "hipStreamWaitEvent")

    def destroy(self):
        if self.handle:
            check(lib().hipStreamDestroy(self.handle), "hipStreamDestroy")
            self.handle = None


class Event:
    def __init__(self):
        e = ctypes.c_void_p()
        check(lib().hipEventCreate(ctypes.byref(e)), "hipEventCreate")
        self.handle = e.value

    def record(self, stream: Stream | None = None):
        check(lib().hipEventRecord(self.handle, stream.handle if stream else None), "hipEventRecord")

    def synchronize(self):
        check(lib().hipEventSynchronize(self.handle), "hipEventSynchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        check(lib().hipEventElapsedTime(ctypes.byref(ms), self.handle, end.handle),
              "hipEventElapsedTime")
        return ms.value

    def destroy(self):
        if self.handle:
            check(lib().hipEventDestroy(self.handle), "hipEventDestroy")
            self.handle = None
