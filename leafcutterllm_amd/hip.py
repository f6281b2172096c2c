"""Minimal ctypes binding of the HIP runtime (the same libamdhip64 the product
library links): device buffers, streams and events for callers that hand the
library device pointers (lcmoe_forward_dev) and time it."""
from __future__ import annotations

import ctypes as C
import os

_ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
_rt = None


def rt() -> C.CDLL:
    global _rt
    if _rt is None:
        _rt = C.CDLL(os.path.join(_ROCM, "lib", "libamdhip64.so"))
        vp, i32, sz = C.c_void_p, C.c_int, C.c_size_t
        for name, res, args in [
            ("hipMalloc", i32, [C.POINTER(vp), sz]), ("hipFree", i32, [vp]),
            ("hipMemcpy", i32, [vp, vp, sz, i32]), ("hipMemset", i32, [vp, i32, sz]),
            ("hipDeviceSynchronize", i32, []), ("hipStreamCreate", i32, [C.POINTER(vp)]),
            ("hipStreamDestroy", i32, [vp]), ("hipStreamSynchronize", i32, [vp]),
            ("hipEventCreate", i32, [C.POINTER(vp)]), ("hipEventDestroy", i32, [vp]),
            ("hipEventRecord", i32, [vp, vp]), ("hipEventSynchronize", i32, [vp]),
            ("hipEventElapsedTime", i32, [C.POINTER(C.c_float), vp, vp]),
            ("hipGetDeviceCount", i32, [C.POINTER(i32)]),
            ("hipGetErrorString", C.c_char_p, [i32]),
            ("hipMemGetInfo", i32, [C.POINTER(sz), C.POINTER(sz)]),
        ]:
            fn = getattr(_rt, name)
            fn.restype = res
            fn.argtypes = args
    return _rt


H2D, D2H = 1, 2


def _check(err: int, what: str) -> None:
    if err != 0:
        raise RuntimeError(f"{what}: {rt().hipGetErrorString(err).decode()}")


def device_count() -> int:
    n = C.c_int(0)
    err = rt().hipGetDeviceCount(C.byref(n))
    return n.value if err == 0 else 0


class DeviceBuffer:
    def __init__(self, nbytes: int):
        self.nbytes = nbytes
        p = C.c_void_p()
        _check(rt().hipMalloc(C.byref(p), max(nbytes, 256)), "hipMalloc")
        self.ptr = p.value

    def upload(self, arr) -> "DeviceBuffer":
        assert arr.nbytes <= self.nbytes
        _check(rt().hipMemcpy(self.ptr, arr.ctypes.data, arr.nbytes, H2D), "hipMemcpy H2D")
        return self

    def download(self, arr):
        assert arr.nbytes <= self.nbytes
        _check(rt().hipMemcpy(arr.ctypes.data, self.ptr, arr.nbytes, D2H), "hipMemcpy D2H")
        return arr

    def free(self) -> None:
        if self.ptr:
            rt().hipFree(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    def __init__(self):
        p = C.c_void_p()
        _check(rt().hipStreamCreate(C.byref(p)), "hipStreamCreate")
        self.ptr = p.value

    def synchronize(self) -> None:
        _check(rt().hipStreamSynchronize(self.ptr), "hipStreamSynchronize")


class Event:
    def __init__(self):
        p = C.c_void_p()
        _check(rt().hipEventCreate(C.byref(p)), "hipEventCreate")
        self.ptr = p.value

    def record(self, stream: Stream) -> None:
        _check(rt().hipEventRecord(self.ptr, stream.ptr), "hipEventRecord")

    def elapsed_ms(self, later: "Event") -> float:
        _check(rt().hipEventSynchronize(later.ptr), "hipEventSynchronize")
        t = C.c_float()
        _check(rt().hipEventElapsedTime(C.byref(t), self.ptr, later.ptr), "hipEventElapsedTime")
        return float(t.value)
