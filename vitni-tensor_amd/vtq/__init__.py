"""vtq -- Python host mirror of vitni-tensor's quantized linear API over libvtq.

The functions keep the reference's names, argument meaning and error
behaviour (src/ops/quant.rs, src/model/forward_quantized.rs:663-785):
``x`` is ``[batch, in_feat]`` float32, ``w`` the GGUF block bytes of
``W[out_feat, in_feat]``, ``y_out`` ``[batch, out_feat]`` float32 written in
place.  A failing call raises the exception that mirrors the reference's
``Error`` variant (src/error.rs:7-63) with the reference's message.

All compute runs in libvtq on the GPU.  If libvtq.so is missing or no GPU is
present the calls raise; there is no CPU fallback in this package.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(os.path.dirname(_HERE), "lib")
LIB_PATH = os.path.join(LIB_DIR, "libvtq.so")

# GGUF tensor type tags (src/model/gguf.rs:127-139)
F32, F16, Q4_0, Q5_0, Q8_0, Q4_K, Q6_K = 0, 1, 2, 6, 8, 12, 14
TYPE_NAMES = {F32: "F32", F16: "F16", Q4_0: "Q4_0", Q5_0: "Q5_0", Q8_0: "Q8_0", Q4_K: "Q4_K", Q6_K: "Q6_K"}
BLOCK = {Q4_0: (32, 18), Q5_0: (32, 22), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210)}

REGIME_INTEGER = 0       # std-parallel build: integer Q4_K
REGIME_FLOAT_FUSED = 1   # default build: float-fused Q4_K

OK, E_INTERNAL, E_GPU, E_NOT_IMPLEMENTED, E_INVALID_ARGUMENT = 0, 1, 2, 3, 4
E_MALFORMED, E_TRUNCATED, E_OVERFLOW, E_SHAPE_MISMATCH, E_INVALID_SHAPE = 5, 6, 7, 8, 9


class VtqError(Exception):
    """Base of the mirrored vitni_tensor::error::Error variants."""

    code = -1

    def __init__(self, message: str):
        super().__init__(message)
        self.message = message


class Internal(VtqError):
    """Error::Internal(&'static str) -- shape and length violations."""

    code = E_INTERNAL


class GpuError(VtqError):
    """Error::GpuError -- a HIP call failed."""

    code = E_GPU


class NotImplementedDtype(VtqError):
    """Error::NotImplemented -- dtype (or size) not supported."""

    code = E_NOT_IMPLEMENTED


class InvalidArgument(VtqError):
    """Null pointer / context misuse (ruled out by Rust's types in the reference)."""

    code = E_INVALID_ARGUMENT


class Malformed(VtqError):
    """Error::Malformed -- a GGUF file that violates the format."""

    code = E_MALFORMED


class Truncated(VtqError):
    """Error::Truncated -- a GGUF file that ends before a field."""

    code = E_TRUNCATED


class Overflow(VtqError):
    """Error::Overflow -- a GGUF length or offset whose arithmetic overflows."""

    code = E_OVERFLOW


class ShapeMismatch(VtqError):
    """Error::ShapeMismatch -- a norm weight whose length is not the model dimension."""

    code = E_SHAPE_MISMATCH


class InvalidShape(VtqError):
    """Error::InvalidShape -- an empty prompt, or prompt + new tokens past seq_len."""

    code = E_INVALID_SHAPE


_ERRORS = {c.code: c for c in (Internal, GpuError, NotImplementedDtype, InvalidArgument, Malformed, Truncated,
                               Overflow, ShapeMismatch, InvalidShape)}


def error_class(code: int):
    """The exception class of a libvtq / libvtq_runtime status code."""
    return _ERRORS.get(code, GpuError)

_lib: Optional[ctypes.CDLL] = None


def load_library(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load libvtq.so (built in-tree by ``make -C vitni-tensor_amd``)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise ImportError(f"libvtq.so not built: {path} is missing (run __graft_entry__.build())")
    # One HIP runtime per process: torch's ROCm wheel loads its own
    # libamdhip64 (NEEDED "libamdhip64.so", SONAME libamdhip64.so.7).  Loading
    # torch first lets libvtq's NEEDED libamdhip64.so.7 resolve to that same
    # copy by SONAME; the other order would map a second runtime into the
    # process and the second one would find no device.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(path)
    vp, sz, i = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
    lib.vtq_create.argtypes = [i, ctypes.POINTER(vp)]
    lib.vtq_create.restype = i
    lib.vtq_destroy.argtypes = [vp]
    lib.vtq_destroy.restype = None
    lib.vtq_last_error.argtypes = [vp]
    lib.vtq_last_error.restype = ctypes.c_char_p
    lib.vtq_version.argtypes = []
    lib.vtq_version.restype = ctypes.c_char_p
    host_sig = [vp, vp, sz, vp, sz, vp, sz, sz, sz, sz]
    for name in ("vtq_linear_q4_k_integer", "vtq_linear_q6_k_integer", "vtq_linear_q4_k_fused", "vtq_linear_q4_0"):
        f = getattr(lib, name)
        f.argtypes = host_sig
        f.restype = i
    lib.vtq_linear.argtypes = [vp, i, i, vp, sz, vp, sz, vp, sz, sz, sz, sz]
    lib.vtq_linear.restype = i
    lib.vtq_release_weights.argtypes = [vp, vp]
    lib.vtq_release_weights.restype = i
    lib.vtq_linear_device.argtypes = [vp, i, i, vp, vp, sz, vp, sz, sz, sz, vp]
    lib.vtq_linear_device.restype = i
    _lib = lib
    return lib


EXPORTED = (
    "vtq_create", "vtq_destroy", "vtq_last_error", "vtq_version", "vtq_linear",
    "vtq_linear_q4_k_integer", "vtq_linear_q6_k_integer", "vtq_linear_q4_k_fused",
    "vtq_linear_q4_0", "vtq_release_weights", "vtq_linear_device", "vtq_linear_device_noalloc",
)


class Context:
    """One libvtq context (one HIP device, used by one thread at a time).

    Host-pointer calls cache the weight bytes on the device keyed by the
    array's address and length, as the reference's weights are immutable
    views into a GGUF blob.  Call release_weights() before reusing or freeing
    a weight array whose bytes change.
    """

    def __init__(self, device: int = 0):
        self.lib = load_library()
        h = ctypes.c_void_p()
        rc = self.lib.vtq_create(int(device), ctypes.byref(h))
        if rc != OK:
            raise GpuError(f"vtq_create({device}) failed with status {rc}: no usable HIP device")
        self.handle = h
        self.device = device

    def close(self) -> None:
        if getattr(self, "handle", None):
            self.lib.vtq_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def _check(self, rc: int) -> None:
        if rc == OK:
            return
        msg = self.lib.vtq_last_error(self.handle).decode(errors="replace")
        raise _ERRORS.get(rc, VtqError)(msg)

    # -- host-pointer calls -------------------------------------------------

    @staticmethod
    def _f32(a: np.ndarray, name: str) -> np.ndarray:
        if not isinstance(a, np.ndarray) or a.dtype != np.float32 or not a.flags.c_contiguous:
            raise TypeError(f"{name} must be a C-contiguous float32 numpy array")
        return a

    @staticmethod
    def _u8(a) -> np.ndarray:
        if isinstance(a, (bytes, bytearray)):
            a = np.frombuffer(a, dtype=np.uint8)
        if not isinstance(a, np.ndarray) or a.dtype != np.uint8 or not a.flags.c_contiguous:
            raise TypeError("w must be a C-contiguous uint8 numpy array or bytes")
        return a

    def _host(self, fn, x, w, y_out, batch, in_feat, out_feat):
        x = self._f32(x, "x")
        y_out = self._f32(y_out, "y_out")
        w = self._u8(w)
        if not y_out.flags.writeable:
            raise TypeError("y_out must be writeable")
        rc = fn(self.handle, x.ctypes.data, x.size, w.ctypes.data, w.size, y_out.ctypes.data, y_out.size,
                batch, in_feat, out_feat)
        self._check(rc)

    def linear_q4_k_integer(self, x, w_q4k, y_out, batch, in_feat, out_feat):
        """src/ops/quant.rs:936-980"""
        self._host(self.lib.vtq_linear_q4_k_integer, x, w_q4k, y_out, batch, in_feat, out_feat)

    def linear_q6_k_integer(self, x, w_q6k, y_out, batch, in_feat, out_feat):
        """src/ops/quant.rs:1060-1096"""
        self._host(self.lib.vtq_linear_q6_k_integer, x, w_q6k, y_out, batch, in_feat, out_feat)

    def linear_q4_k_fused(self, x, w_q4k, y_out, batch, in_feat, out_feat):
        """src/ops/quant.rs:1433-1453"""
        self._host(self.lib.vtq_linear_q4_k_fused, x, w_q4k, y_out, batch, in_feat, out_feat)

    def linear_q4_0(self, x, w_q4, y_out, batch, in_feat, out_feat):
        """src/ops/quant.rs:1529-1565 (linear_q4_0_cpu)"""
        self._host(self.lib.vtq_linear_q4_0, x, w_q4, y_out, batch, in_feat, out_feat)

    def linear(self, ggml_type, regime, x, w, y_out, batch, in_feat, out_feat):
        """src/model/forward_quantized.rs:663-785 (linear_dispatch), any batch."""
        x = self._f32(x, "x")
        y_out = self._f32(y_out, "y_out")
        w = self._u8(w)
        rc = self.lib.vtq_linear(self.handle, int(ggml_type), int(regime), x.ctypes.data, x.size, w.ctypes.data,
                                 w.size, y_out.ctypes.data, y_out.size, batch, in_feat, out_feat)
        self._check(rc)

    def linear_dispatch(self, x, w, ggml_type, in_feat, out_feat, regime=REGIME_INTEGER):
        """The reference's linear_dispatch shape: batch 1, returns a new y."""
        y = np.zeros(out_feat, dtype=np.float32)
        self.linear(ggml_type, regime, x, w, y, 1, in_feat, out_feat)
        return y

    def release_weights(self, w=None):
        ptr = None if w is None else self._u8(w).ctypes.data
        self._check(self.lib.vtq_release_weights(self.handle, ptr))

    # -- device-pointer call ------------------------------------------------

    def linear_device(self, ggml_type, regime, x_ptr, w_ptr, w_len, y_ptr, batch, in_feat, out_feat, stream=None):
        """Enqueue on `stream` (int handle or None); pointers are device addresses."""
        rc = self.lib.vtq_linear_device(self.handle, int(ggml_type), int(regime), x_ptr, w_ptr, w_len, y_ptr,
                                        batch, in_feat, out_feat, stream)
        self._check(rc)


def row_bytes(ggml_type: int, in_feat: int) -> int:
    if ggml_type == F32:
        return 4 * in_feat
    numel, nbytes = BLOCK[ggml_type]
    return (in_feat // numel) * nbytes
