"""Minimal HIP runtime plumbing for the host side: device buffers, copies, streams, events.

decide's device layer (crates/decide-metal/src/device.rs) owns the device,
the queue and the buffers the engine binds; this is the same role over the
HIP runtime that libdecide_hip.so itself links (libamdhip64.so.7 from
/opt/rocm), bound with ctypes. Using that one runtime keeps every launch,
allocation and timing event in a single HIP instance.
"""

from __future__ import annotations

import ctypes
from ctypes import POINTER, byref, c_char_p, c_float, c_int, c_size_t, c_uint, c_uint32, c_void_p

import numpy as np

from . import _lib

H2D, D2H, D2D = 1, 2, 3

_rt = None


def rt() -> ctypes.CDLL:
    """The HIP runtime that libdecide_hip.so is linked against."""
    global _rt
    if _rt is not None:
        return _rt
    _lib.load()  # pulls in its libamdhip64.so.7; dlopen by soname returns that same copy
    r = ctypes.CDLL("libamdhip64.so.7", mode=ctypes.RTLD_GLOBAL)
    sig = {
        "hipGetDeviceCount": (c_int, [POINTER(c_int)]),
        "hipSetDevice": (c_int, [c_int]),
        "hipMalloc": (c_int, [POINTER(c_void_p), c_size_t]),
        "hipFree": (c_int, [c_void_p]),
        "hipMemcpy": (c_int, [c_void_p, c_void_p, c_size_t, c_int]),
        "hipMemcpyAsync": (c_int, [c_void_p, c_void_p, c_size_t, c_int, c_void_p]),
        "hipMemset": (c_int, [c_void_p, c_int, c_size_t]),
        "hipDeviceSynchronize": (c_int, []),
        "hipStreamCreate": (c_int, [POINTER(c_void_p)]),
        "hipStreamDestroy": (c_int, [c_void_p]),
        "hipStreamSynchronize": (c_int, [c_void_p]),
        "hipEventCreate": (c_int, [POINTER(c_void_p)]),
        "hipEventCreateWithFlags": (c_int, [POINTER(c_void_p), c_uint32]),
        "hipEventDestroy": (c_int, [c_void_p]),
        "hipEventRecord": (c_int, [c_void_p, c_void_p]),
        "hipEventSynchronize": (c_int, [c_void_p]),
        "hipEventElapsedTime": (c_int, [POINTER(c_float), c_void_p, c_void_p]),
        "hipGetErrorString": (c_char_p, [c_int]),
        "hipGetLastError": (c_int, []),
        "hipStreamBeginCapture": (c_int, [c_void_p, c_int]),
        "hipStreamEndCapture": (c_int, [c_void_p, POINTER(c_void_p)]),
        "hipGraphInstantiate": (c_int, [POINTER(c_void_p), c_void_p, c_void_p, c_void_p, c_size_t]),
        "hipGraphLaunch": (c_int, [c_void_p, c_void_p]),
        "hipGraphExecDestroy": (c_int, [c_void_p]),
        "hipGraphDestroy": (c_int, [c_void_p]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(r, name)
        fn.restype = res
        fn.argtypes = args
    _rt = r
    return r


class HipError(RuntimeError):
    pass


def check(e: int, what: str = "hip") -> None:
    if e != 0:
        raise HipError(f"{what}: {rt().hipGetErrorString(e).decode()} ({e})")


def device_count() -> int:
    n = c_int(0)
    e = rt().hipGetDeviceCount(byref(n))
    return n.value if e == 0 else 0


def available() -> bool:
    return device_count() > 0


def synchronize() -> None:
    check(rt().hipDeviceSynchronize(), "hipDeviceSynchronize")


class DeviceArray:
    """A device buffer with a numpy shape and dtype. ``data_ptr()`` is its device address."""

    def __init__(self, shape, dtype):
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = c_void_p()
        check(rt().hipMalloc(byref(p), max(self.nbytes, 1)), f"hipMalloc({self.nbytes})")
        self.ptr = p.value

    @classmethod
    def from_numpy(cls, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        if d.nbytes:
            check(rt().hipMemcpy(d.ptr, a.ctypes.data, d.nbytes, H2D), "hipMemcpy H2D")
        return d

    @classmethod
    def full(cls, shape, dtype, value) -> "DeviceArray":
        return cls.from_numpy(np.full(shape, value, dtype=dtype))

    def data_ptr(self) -> int:
        return self.ptr

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        if self.nbytes:
            check(rt().hipMemcpy(out.ctypes.data, self.ptr, self.nbytes, D2H), "hipMemcpy D2H")
        return out

    def copy_from(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.nbytes == self.nbytes
        check(rt().hipMemcpy(self.ptr, a.ctypes.data, self.nbytes, H2D), "hipMemcpy H2D")

    def copy_(self, other: "DeviceArray") -> None:
        assert other.nbytes == self.nbytes
        check(rt().hipMemcpy(self.ptr, other.ptr, self.nbytes, D2D), "hipMemcpy D2D")

    def zero_(self) -> None:
        check(rt().hipMemset(self.ptr, 0, self.nbytes), "hipMemset")

    def free(self) -> None:
        if self.ptr:
            rt().hipFree(self.ptr)
            self.ptr = None

    def __del__(self):  # pragma: no cover
        try:
            self.free()
        except Exception:
            pass


class Stream:
    """A HIP stream at the default priority (``handle`` is the hipStream_t as an int)."""

    def __init__(self):
        h = c_void_p()
        check(rt().hipStreamCreate(byref(h)), "hipStreamCreate")
        self.handle = h.value

    def synchronize(self) -> None:
        check(rt().hipStreamSynchronize(self.handle), "hipStreamSynchronize")

    def destroy(self) -> None:
        if self.handle:
            rt().hipStreamDestroy(self.handle)
            self.handle = None


# hipEventDisableSystemFence: the event's record skips the system-scope fence (an L2 write-back and
# invalidate) that a default event performs, which would stall the stream and leave the next kernel a cold L2.
EVENT_DISABLE_SYSTEM_FENCE = 0x20000000


class Event:
    """A HIP event. ``timing=True`` makes a timing-only event (no system-scope fence on record): for
    timestamps between kernels of one stream, read after a default event later on that stream completes."""

    def __init__(self, timing: bool = False):
        h = c_void_p()
        if timing:
            check(rt().hipEventCreateWithFlags(byref(h), EVENT_DISABLE_SYSTEM_FENCE), "hipEventCreateWithFlags")
        else:
            check(rt().hipEventCreate(byref(h)), "hipEventCreate")
        self.handle = h.value

    def record(self, stream: int = 0) -> None:
        check(rt().hipEventRecord(self.handle, stream), "hipEventRecord")

    def synchronize(self) -> None:
        check(rt().hipEventSynchronize(self.handle), "hipEventSynchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = c_float()
        check(rt().hipEventElapsedTime(byref(ms), self.handle, end.handle), "hipEventElapsedTime")
        return float(ms.value)

    def destroy(self) -> None:
        if self.handle:
            rt().hipEventDestroy(self.handle)
            self.handle = None
