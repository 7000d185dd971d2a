"""ctypes binding of libvtq_probe.so: measurement helpers used by bench.py
(a hand-written read-only stream kernel).  Not part of the quantized-linear
boundary."""
from __future__ import annotations

import ctypes
import os

from . import LIB_DIR, load_library

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        load_library()  # torch first, then the HIP libraries: one HIP runtime per process
        path = os.path.join(LIB_DIR, "libvtq_probe.so")
        if not os.path.exists(path):
            raise ImportError(f"{path} is missing (run __graft_entry__.build())")
        L = ctypes.CDLL(path)
        L.vtqp_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_void_p,
                                       ctypes.c_void_p]
        L.vtqp_stream_read.restype = ctypes.c_int
        _lib = L
    return _lib


def stream_read(ptr: int, nbytes: int, workgroups: int, sink_ptr: int, stream: int) -> None:
    """Launch a read-only stream of `nbytes` (a multiple of 16) at device
    address `ptr` with `workgroups` workgroups of 256 threads on `stream`."""
    rc = lib().vtqp_stream_read(ptr, nbytes, workgroups, sink_ptr, stream)
    if rc != 0:
        raise RuntimeError(f"vtqp_stream_read: hipError {rc}")
