"""HIP-event timing on the device's own stream (the stream every dwim_* call
queues on), through libamdhip64 directly."""
from __future__ import annotations

import ctypes

_hip = None


def hip() -> ctypes.CDLL:
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so")
        _hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        _hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        _hip.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        _hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        _hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
    return _hip


class Event:
    def __init__(self):
        h = ctypes.c_void_p()
        if hip().hipEventCreate(ctypes.byref(h)) != 0:
            raise RuntimeError("hipEventCreate failed")
        self.h = h.value

    def record(self, stream: int):
        if hip().hipEventRecord(self.h, stream) != 0:
            raise RuntimeError("hipEventRecord failed")

    def synchronize(self):
        hip().hipEventSynchronize(self.h)

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        end.synchronize()
        if hip().hipEventElapsedTime(ctypes.byref(ms), self.h, end.h) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return ms.value

    def __del__(self):
        if _hip is not None and getattr(self, "h", None):
            _hip.hipEventDestroy(self.h)
