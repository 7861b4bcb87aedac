"""HIP events over ctypes, for timing work queued on a backend's stream
(`mfh_stream`).

Uses the same libamdhip64 the backend library links, so stream and event
handles are shared with it.  Plumbing for benches and drivers; no compute.
"""
from __future__ import annotations

import ctypes
import ctypes.util

_hip = None


def hip() -> ctypes.CDLL:
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("/opt/rocm/lib/libamdhip64.so.7")
        P, PP = ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)
        sigs = {
            "hipEventCreate": [PP],
            "hipEventDestroy": [P],
            "hipEventRecord": [P, P],
            "hipEventSynchronize": [P],
            "hipEventElapsedTime": [ctypes.POINTER(ctypes.c_float), P, P],
            "hipStreamSynchronize": [P],
            "hipGetErrorString": [ctypes.c_int],
        }
        for name, args in sigs.items():
            fn = getattr(_hip, name)
            fn.argtypes = args
            fn.restype = ctypes.c_char_p if name == "hipGetErrorString" else ctypes.c_int
    return _hip


def check(err: int, what: str) -> None:
    if err:
        raise RuntimeError(f"{what} failed: {hip().hipGetErrorString(err).decode()} ({err})")


class Event:
    def __init__(self):
        h = ctypes.c_void_p()
        check(hip().hipEventCreate(ctypes.byref(h)), "hipEventCreate")
        self.handle = h.value

    def record(self, stream: int) -> None:
        check(hip().hipEventRecord(self.handle, stream), "hipEventRecord")

    def synchronize(self) -> None:
        check(hip().hipEventSynchronize(self.handle), "hipEventSynchronize")

    def elapsed_ms(self, start: "Event") -> float:
        ms = ctypes.c_float(0)
        check(hip().hipEventElapsedTime(ctypes.byref(ms), start.handle, self.handle),
              "hipEventElapsedTime")
        return float(ms.value)

    def __del__(self):
        try:
            if self.handle:
                hip().hipEventDestroy(self.handle)
        except Exception:
            pass


def stream_synchronize(stream: int) -> None:
    check(hip().hipStreamSynchronize(stream), "hipStreamSynchronize")
