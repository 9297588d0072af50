"""Minimal ctypes access to HIP runtime events (for timing kernels on a given stream)."""

from __future__ import annotations

import ctypes

_hip = None


def _lib():
    global _hip
    if _hip is None:
        for name in ("libamdhip64.so", "libamdhip64.so.7", "/opt/rocm/lib/libamdhip64.so"):
            try:
                _hip = ctypes.CDLL(name)
                break
            except OSError:
                continue
        if _hip is None:
            raise RuntimeError("libamdhip64.so not found")
        p = ctypes.c_void_p
        _hip.hipEventCreate.argtypes = [ctypes.POINTER(p)]
        _hip.hipEventCreate.restype = ctypes.c_int
        _hip.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(p), ctypes.c_uint]
        _hip.hipEventCreateWithFlags.restype = ctypes.c_int
        _hip.hipEventDestroy.argtypes = [p]
        _hip.hipEventDestroy.restype = ctypes.c_int
        _hip.hipEventSynchronize.argtypes = [p]
        _hip.hipEventSynchronize.restype = ctypes.c_int
        _hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), p, p]
        _hip.hipEventElapsedTime.restype = ctypes.c_int
    return _hip


HIP_EVENT_DISABLE_TIMING = 0x2


class EventArray:
    """n hipEvent_t handles in a C array (pass ``.ptr`` where a void** is expected).

    ``timing=False`` creates them with hipEventDisableTiming (ordering only).
    """

    def __init__(self, n: int, timing: bool = True):
        L = _lib()
        self.n = n
        self.arr = (ctypes.c_void_p * n)()
        for i in range(n):
            h = ctypes.c_void_p()
            if timing:
                rc = L.hipEventCreate(ctypes.byref(h))
            else:
                rc = L.hipEventCreateWithFlags(ctypes.byref(h), HIP_EVENT_DISABLE_TIMING)
            if rc != 0:
                raise RuntimeError(f"hipEventCreate failed ({rc})")
            self.arr[i] = h.value
        self.ptr = ctypes.cast(self.arr, ctypes.c_void_p).value

    def elapsed_ms(self, i: int, j: int) -> float:
        L = _lib()
        L.hipEventSynchronize(self.arr[j])
        ms = ctypes.c_float()
        rc = L.hipEventElapsedTime(ctypes.byref(ms), self.arr[i], self.arr[j])
        if rc != 0:
            raise RuntimeError(f"hipEventElapsedTime failed ({rc})")
        return float(ms.value)

    def close(self) -> None:
        L = _lib()
        for i in range(self.n):
            if self.arr[i]:
                L.hipEventDestroy(self.arr[i])
                self.arr[i] = None
