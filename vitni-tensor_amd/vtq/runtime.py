"""ctypes bindings of libvtq_runtime (include/vtq_runtime.h): the reference's
quantized decode (inference::run_quantized) with every linear on the GPU."""
from __future__ import annotations

import ctypes
import os

import numpy as np

from . import LIB_DIR, load_library, error_class

_rt = None


def lib() -> ctypes.CDLL:
    global _rt
    if _rt is None:
        load_library()  # torch first, then libvtq: one HIP runtime per process
        path = os.path.join(LIB_DIR, "libvtq_runtime.so")
        if not os.path.exists(path):
            raise ImportError(f"{path} is missing (run __graft_entry__.build())")
        L = ctypes.CDLL(path)
        vp, sz, i = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
        L.vtqrt_load.argtypes = [i, vp, sz, ctypes.POINTER(vp)]
        L.vtqrt_load.restype = i
        L.vtqrt_free.argtypes = [vp]
        L.vtqrt_free.restype = None
        L.vtqrt_last_error.argtypes = [vp]
        L.vtqrt_last_error.restype = ctypes.c_char_p
        L.vtqrt_dims.argtypes = [vp, vp]
        L.vtqrt_dims.restype = i
        L.vtqrt_run.argtypes = [vp, i, ctypes.c_char_p, vp, vp, i, i, vp, vp, vp, vp]
        L.vtqrt_run.restype = i
        L.vtqrt_parse.argtypes = [vp, sz, i, vp, ctypes.c_char_p, sz]
        L.vtqrt_parse.restype = i
        L.vtqrt_run_recorded.argtypes = [vp, i, ctypes.c_char_p, vp, vp, i, i, i, vp, vp, sz, vp, sz,
                                         ctypes.POINTER(sz), ctypes.POINTER(sz), vp]
        L.vtqrt_run_recorded.restype = i
        L.vtqrt_blake3.argtypes = [vp, sz, vp]
        L.vtqrt_blake3.restype = None
        L.vtqrt_rms_norm_device.argtypes = [vp, vp, sz, ctypes.c_float, vp, vp]
        L.vtqrt_rms_norm_device.restype = i
        L.vtqrt_transcendentals_device.argtypes = [vp, sz, vp, vp]
        L.vtqrt_transcendentals_device.restype = i
        L.vtqrt_set_prompt_mode.argtypes = [vp, i]
        L.vtqrt_set_prompt_mode.restype = i
        _rt = L
    return _rt


def blake3(data) -> bytes:
    d = np.ascontiguousarray(np.frombuffer(bytes(data), dtype=np.uint8) if isinstance(data, (bytes, bytearray))
                             else data, dtype=np.uint8)
    out = (ctypes.c_uint8 * 32)()
    lib().vtqrt_blake3(d.ctypes.data if d.size else None, d.size, out)
    return bytes(out)


def parse(blob, level=0):
    """vtqrt_parse on the host (no GPU needed): GgufFile::parse (level 0), or
    with Config / QuantizedWeights (level 1).  (status, message, dims):
    status 0 is Ok, else the include/vtq.h code of the reference's Error
    variant; dims (level 1, status 0) is (dim, hidden, layers, heads,
    kv_heads, vocab, seq_len)."""
    b = np.ascontiguousarray(np.frombuffer(bytes(blob), dtype=np.uint8) if isinstance(blob, (bytes, bytearray))
                             else blob, dtype=np.uint8)
    dims = np.zeros(7, dtype=np.int32)
    err = ctypes.create_string_buffer(256)
    rc = lib().vtqrt_parse(b.ctypes.data if b.size else None, b.size, level, dims.ctypes.data, err, len(err))
    return rc, err.value.decode(), tuple(int(d) for d in dims) if rc == 0 and level == 1 else None


def rms_norm_device(x_ptr, w_ptr, n, eps, y_ptr, stream=None) -> None:
    """vtqrt_rms_norm_device: enqueue rms_norm_slice on device pointers."""
    rc = lib().vtqrt_rms_norm_device(x_ptr, w_ptr, n, float(eps), y_ptr, stream)
    if rc != 0:
        raise RuntimeError(f"vtqrt_rms_norm_device failed with status {rc}")


def transcendentals_device(x_ptr, n, y_ptr, stream=None) -> None:
    """vtqrt_transcendentals_device: y[7i + k] = f_k(x[i]) on the device."""
    rc = lib().vtqrt_transcendentals_device(x_ptr, n, y_ptr, stream)
    if rc != 0:
        raise RuntimeError(f"vtqrt_transcendentals_device failed with status {rc}")


PROMPT_BATCHED, PROMPT_STEPWISE = 0, 1  # vtqrt_set_prompt_mode (include/vtq_runtime.h)
RECORD_OPS = 1
RECORD_ACTIVATIONS = 2


class OpRecord(ctypes.Structure):
    """vtqrt_op_record: one PerOp receipt entry."""
    _fields_ = [("op_index", ctypes.c_uint32), ("layer", ctypes.c_uint32), ("op_name", ctypes.c_char * 16),
                ("input_hash", ctypes.c_uint8 * 32), ("params_hash", ctypes.c_uint8 * 32),
                ("output_hash", ctypes.c_uint8 * 32)]

    def key(self):
        return (self.op_index, self.layer, self.op_name, bytes(self.input_hash), bytes(self.params_hash),
                bytes(self.output_hash))


class ActRecord(ctypes.Structure):
    """vtqrt_act_record: one activation-checkpoint receipt entry."""
    _fields_ = [("act_index", ctypes.c_uint32), ("token_index", ctypes.c_uint32), ("layer", ctypes.c_uint32),
                ("checkpoint", ctypes.c_char * 16), ("tensor_hash", ctypes.c_uint8 * 32)]

    def key(self):
        return (self.act_index, self.token_index, self.layer, self.checkpoint, bytes(self.tensor_hash))


class Model:
    """A GGUF model uploaded to one GPU (vtqrt_load)."""

    def __init__(self, blob, device: int = 0):
        self.digest_v1 = None
        self.handle = None
        b = np.ascontiguousarray(np.frombuffer(blob, dtype=np.uint8) if isinstance(blob, (bytes, bytearray))
                                 else blob, dtype=np.uint8)
        self.handle = ctypes.c_void_p()
        rc = lib().vtqrt_load(device, b.ctypes.data, b.size, ctypes.byref(self.handle))
        if rc:
            msg = lib().vtqrt_last_error(self.handle).decode()
            lib().vtqrt_free(self.handle)
            self.handle = None
            raise error_class(rc)(msg)
        dims = np.zeros(7, dtype=np.int32)
        lib().vtqrt_dims(self.handle, dims.ctypes.data)
        self.dim, self.hidden, self.layers, self.heads, self.kv_heads, self.vocab, self.seq_len = map(int, dims)

    def run(self, prompt, n_new, weights_hash: bytes, regime=0, model_id="vitni-receipt", want_logits=True,
            stepwise=False):
        """(generated tokens, v2 digest hex, logits [steps][vocab] or None);
        digest_v1 then holds the frozen v1 digest of the same cert.  The
        prompt goes through in one batched pass unless stepwise (one step per
        position, run_quantized's loop); both give the same bits."""
        rc = lib().vtqrt_set_prompt_mode(self.handle, PROMPT_STEPWISE if stepwise else PROMPT_BATCHED)
        if rc:
            raise error_class(rc)(lib().vtqrt_last_error(self.handle).decode())
        prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
        wh = np.frombuffer(bytes(weights_hash), dtype=np.uint8).copy()
        tokens = np.zeros(max(1, n_new), dtype=np.uint32)
        logits = np.zeros((prompt.size + n_new) * self.vocab, dtype=np.float32) if want_logits else None
        digest = (ctypes.c_uint8 * 32)()
        digest_v1 = (ctypes.c_uint8 * 32)()
        rc = lib().vtqrt_run(self.handle, regime, model_id.encode(), wh.ctypes.data, prompt.ctypes.data, prompt.size,
                             n_new, None if logits is None else logits.ctypes.data, tokens.ctypes.data, digest,
                             digest_v1)
        if rc:
            raise error_class(rc)(lib().vtqrt_last_error(self.handle).decode())
        self.digest_v1 = bytes(digest_v1).hex()
        if logits is not None:
            logits = logits.reshape(prompt.size + n_new, self.vocab)
        return tokens[:n_new], bytes(digest).hex(), logits

    def run_recorded(self, prompt, n_new, weights_hash: bytes, flags=RECORD_OPS | RECORD_ACTIVATIONS, regime=0,
                     model_id="vitni-receipt"):
        """run_quantized with per-op / activation receipts:
        (generated tokens, v2 digest hex, [OpRecord], [ActRecord])."""
        prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
        wh = np.frombuffer(bytes(weights_hash), dtype=np.uint8).copy()
        tokens = np.zeros(max(1, n_new), dtype=np.uint32)
        steps = prompt.size + n_new
        ops = (OpRecord * max(1, steps * (9 * self.layers + 2)))()
        acts = (ActRecord * max(1, steps * (2 * self.layers + 3)))()
        n_ops, n_acts = ctypes.c_size_t(), ctypes.c_size_t()
        digest = (ctypes.c_uint8 * 32)()
        rc = lib().vtqrt_run_recorded(self.handle, regime, model_id.encode(), wh.ctypes.data, prompt.ctypes.data,
                                      prompt.size, n_new, flags, tokens.ctypes.data, ops, len(ops), acts, len(acts),
                                      ctypes.byref(n_ops), ctypes.byref(n_acts), digest)
        if rc:
            raise error_class(rc)(lib().vtqrt_last_error(self.handle).decode())
        return tokens[:n_new], bytes(digest).hex(), list(ops[:n_ops.value]), list(acts[:n_acts.value])

    def close(self):
        if getattr(self, "handle", None):
            lib().vtqrt_free(self.handle)
            self.handle = None

    def __del__(self):
        self.close()
