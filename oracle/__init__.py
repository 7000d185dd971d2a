"""ctypes bindings of the CPU oracle (libvtq_oracle.so).

TEST INFRASTRUCTURE, NOT PRODUCT.  Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg import this module, always as the checker or the
reported CPU baseline; libvtq never calls it.  See vtq_oracle.h for what each
function restates (reference file:line on every declaration).
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libvtq_oracle.so")

_lib = None


class OracleError(Exception):
    def __init__(self, code, message):
        super().__init__(f"[{code}] {message}")
        self.code = code
        self.message = message


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} missing (run `make -C oracle` or __graft_entry__.build())")
    L = ctypes.CDLL(LIB_PATH)
    vp, sz, i, f = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_float
    msgp = ctypes.POINTER(ctypes.c_char_p)
    L.vtqo_f16_to_f32.argtypes = [ctypes.c_uint16]
    L.vtqo_f16_to_f32.restype = f
    L.vtqo_f16_to_f32_bits.argtypes = [ctypes.c_uint16]
    L.vtqo_f16_to_f32_bits.restype = ctypes.c_uint32
    L.vtqo_f32_to_f16.argtypes = [f]
    L.vtqo_f32_to_f16.restype = ctypes.c_uint16
    L.vtqo_fixed_tree.argtypes = [vp, sz]
    L.vtqo_fixed_tree.restype = f
    for name in ("vtqo_canonical_chunk", "vtqo_canonical_dot", "vtqo_canonical_dot_regime2"):
        getattr(L, name).argtypes = [vp, vp, sz]
        getattr(L, name).restype = f
    L.vtqo_canonical_combine.argtypes = [vp, sz]
    L.vtqo_canonical_combine.restype = f
    for name in ("vtqo_dequantize_q4_0", "vtqo_dequantize_q5_0", "vtqo_dequantize_q8_0", "vtqo_dequantize_q4_k",
                 "vtqo_dequantize_q6_k"):
        getattr(L, name).argtypes = [vp, sz, vp, msgp]
        getattr(L, name).restype = i
    for name in ("vtqo_quantize_q4_0", "vtqo_quantize_q8_0"):
        getattr(L, name).argtypes = [vp, sz, vp, msgp]
        getattr(L, name).restype = i
    L.vtqo_quantize_block_q8.argtypes = [vp, sz, vp]
    L.vtqo_quantize_block_q8.restype = None
    for name in ("vtqo_dot_q4k_q8_block", "vtqo_dot_q6k_q8_block"):
        getattr(L, name).argtypes = [vp, vp, sz]
        getattr(L, name).restype = f
    for name in ("vtqo_integer_dot_q4k", "vtqo_canonical_dot_q4k_fused", "vtqo_canonical_dot_q6k_fused"):
        getattr(L, name).argtypes = [vp, vp, sz, sz, vp, msgp]
        getattr(L, name).restype = i
    for name in ("vtqo_linear_q4_k_integer", "vtqo_linear_q6_k_integer", "vtqo_linear_q4_k_fused",
                 "vtqo_linear_q6_k_fused"):
        getattr(L, name).argtypes = [vp, vp, sz, vp, sz, sz, sz, i, msgp]
        getattr(L, name).restype = i
    for name in ("vtqo_linear_q4_k_cpu", "vtqo_linear_q6_k_cpu", "vtqo_linear_q4_0_cpu"):
        getattr(L, name).argtypes = [vp, sz, vp, sz, vp, sz, sz, sz, sz, msgp]
        getattr(L, name).restype = i
    L.vtqo_linear_dispatch.argtypes = [i, i, vp, sz, vp, sz, vp, sz, sz, sz, sz, i, msgp]
    L.vtqo_linear_dispatch.restype = i
    L.vtqo_matmul_f32.argtypes = [vp, vp, vp, sz, sz, sz]
    L.vtqo_matmul_f32.restype = None
    # end-to-end decode (vtq_oracle_e2e.h)
    for name in ("vtqo_expf", "vtqo_sinf", "vtqo_cosf", "vtqo_sqrtf"):
        getattr(L, name).argtypes = [f]
        getattr(L, name).restype = f
    L.vtqo_powf.argtypes = [f, f]
    L.vtqo_powf.restype = f
    L.vtqo_run_quantized_recorded.argtypes = [vp, i, ctypes.c_char_p, vp, vp, i, i, i, i, vp, vp, sz, vp, sz,
                                              ctypes.POINTER(sz), ctypes.POINTER(sz), vp, msgp]
    L.vtqo_run_quantized_recorded.restype = i
    L.vtqo_rms_norm.argtypes = [vp, vp, i, f, vp]
    L.vtqo_rms_norm.restype = None
    L.vtqo_softmax.argtypes = [vp, i]
    L.vtqo_softmax.restype = None
    L.vtqo_argmax.argtypes = [vp, i]
    L.vtqo_argmax.restype = ctypes.c_uint32
    L.vtqo_blake3_hash.argtypes = [vp, sz, vp]
    L.vtqo_blake3_hash.restype = None
    L.vtqo_transcendental_hash.argtypes = [vp]
    L.vtqo_transcendental_hash.restype = sz
    L.vtqo_digest_v2.argtypes = [i, vp, vp, vp, i, vp, vp, vp, vp]
    L.vtqo_digest_v2.restype = None
    L.vtqo_model_load.argtypes = [vp, sz, ctypes.POINTER(vp), msgp]
    L.vtqo_model_load.restype = i
    L.vtqo_model_free.argtypes = [vp]
    L.vtqo_model_free.restype = None
    L.vtqo_model_dims.argtypes = [vp, vp]
    L.vtqo_model_dims.restype = None
    L.vtqo_run_quantized.argtypes = [vp, i, ctypes.c_char_p, vp, vp, i, i, i, vp, vp, vp, vp, msgp]
    L.vtqo_run_quantized.restype = i
    L.vtqo_gguf_parse.argtypes = [vp, sz, i, msgp]
    L.vtqo_gguf_parse.restype = i
    L.vtqo_digest_v1_full.argtypes = [i, vp, vp, vp, i, vp, vp, vp, sz, vp, sz, vp, vp]
    L.vtqo_digest_v1_full.restype = None
    _lib = L
    return L


def _ptr(a):
    return None if a is None else a.ctypes.data


def _f32(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a


def _u8(a):
    if isinstance(a, (bytes, bytearray)):
        a = np.frombuffer(a, dtype=np.uint8)
    return np.ascontiguousarray(a, dtype=np.uint8)


def _check(rc, msg):
    if rc != 0:
        raise OracleError(rc, msg.value.decode() if msg.value else "")


def f16_to_f32(h: int) -> np.float32:
    return np.float32(lib().vtqo_f16_to_f32(h))


def f16_to_f32_bits(h: int) -> int:
    return int(lib().vtqo_f16_to_f32_bits(h))


def f32_to_f16(v: float) -> int:
    return int(lib().vtqo_f32_to_f16(v))


def fixed_tree(parts) -> np.float32:
    p = _f32(parts).copy()
    return np.float32(lib().vtqo_fixed_tree(_ptr(p), p.size))


def canonical_dot(x, w, n=None) -> np.float32:
    x, w = _f32(x), _f32(w)
    n = x.size if n is None else n
    return np.float32(lib().vtqo_canonical_dot(_ptr(x), _ptr(w), n))


def canonical_chunk(x, w) -> np.float32:
    x, w = _f32(x), _f32(w)
    return np.float32(lib().vtqo_canonical_chunk(_ptr(x), _ptr(w), x.size))


def canonical_combine(sums) -> np.float32:
    s = _f32(sums).copy()
    return np.float32(lib().vtqo_canonical_combine(_ptr(s), s.size))


def canonical_dot_regime2(x, w, n=None) -> np.float32:
    x, w = _f32(x), _f32(w)
    n = x.size if n is None else n
    return np.float32(lib().vtqo_canonical_dot_regime2(_ptr(x), _ptr(w), n))


_DEQ = {"q4_0": (32, 18), "q5_0": (32, 22), "q8_0": (32, 34), "q4_k": (256, 144), "q6_k": (256, 210)}


def dequantize(kind: str, w) -> np.ndarray:
    w = _u8(w)
    numel, nbytes = _DEQ[kind]
    out = np.zeros(max(1, (w.size // nbytes) * numel), dtype=np.float32)
    msg = ctypes.c_char_p()
    rc = getattr(lib(), f"vtqo_dequantize_{kind}")(_ptr(w), w.size, _ptr(out), ctypes.byref(msg))
    _check(rc, msg)
    return out[: (w.size // nbytes) * numel]


def quantize(kind: str, x) -> np.ndarray:
    x = _f32(x)
    numel, nbytes = _DEQ[kind]
    out = np.zeros(max(1, (x.size // numel) * nbytes), dtype=np.uint8)
    msg = ctypes.c_char_p()
    rc = getattr(lib(), f"vtqo_quantize_{kind}")(_ptr(x), x.size, _ptr(out), ctypes.byref(msg))
    _check(rc, msg)
    return out[: (x.size // numel) * nbytes]


class Q8Block(ctypes.Structure):
    """src/ops/quant.rs:738-743"""

    _fields_ = [("d", ctypes.c_float), ("qs", ctypes.c_int8 * 256), ("bsums", ctypes.c_int32 * 8)]


def quantize_block_q8(x) -> Q8Block:
    x = _f32(x)
    assert x.size <= 256
    b = Q8Block()
    lib().vtqo_quantize_block_q8(_ptr(x), x.size, ctypes.byref(b))
    return b


def dot_q4k_q8_block(w, xq: Q8Block, n=256) -> np.float32:
    w = _u8(w)
    return np.float32(lib().vtqo_dot_q4k_q8_block(_ptr(w), ctypes.byref(xq), n))


def dot_q6k_q8_block(w, xq: Q8Block, n=256) -> np.float32:
    w = _u8(w)
    return np.float32(lib().vtqo_dot_q6k_q8_block(_ptr(w), ctypes.byref(xq), n))


def _rowdot(name, x, w, n):
    x, w = _f32(x), _u8(w)
    out = ctypes.c_float()
    msg = ctypes.c_char_p()
    rc = getattr(lib(), name)(_ptr(x), _ptr(w), w.size, n, ctypes.byref(out), ctypes.byref(msg))
    _check(rc, msg)
    return np.float32(out.value)


def integer_dot_q4k(x, w, n):
    return _rowdot("vtqo_integer_dot_q4k", x, w, n)


def canonical_dot_q4k_fused(x, w, n):
    return _rowdot("vtqo_canonical_dot_q4k_fused", x, w, n)


def canonical_dot_q6k_fused(x, w, n):
    return _rowdot("vtqo_canonical_dot_q6k_fused", x, w, n)


def _linear(name, x, w, batch, in_feat, out_feat, threads):
    x, w = _f32(x), _u8(w)
    y = np.zeros(max(1, batch * out_feat), dtype=np.float32)
    msg = ctypes.c_char_p()
    rc = getattr(lib(), name)(_ptr(x), _ptr(w), w.size, _ptr(y), batch, in_feat, out_feat, threads,
                              ctypes.byref(msg))
    _check(rc, msg)
    return y[: batch * out_feat]


def linear_q4_k_integer(x, w, batch, in_feat, out_feat, threads=1):
    return _linear("vtqo_linear_q4_k_integer", x, w, batch, in_feat, out_feat, threads)


def linear_q6_k_integer(x, w, batch, in_feat, out_feat, threads=1):
    return _linear("vtqo_linear_q6_k_integer", x, w, batch, in_feat, out_feat, threads)


def linear_q4_k_fused(x, w, batch, in_feat, out_feat, threads=1):
    return _linear("vtqo_linear_q4_k_fused", x, w, batch, in_feat, out_feat, threads)


def linear_q6_k_fused(x, w, batch, in_feat, out_feat, threads=1):
    return _linear("vtqo_linear_q6_k_fused", x, w, batch, in_feat, out_feat, threads)


def _linear_cpu(name, x, w, batch, in_feat, out_feat, x_len=None, y_len=None):
    x, w = _f32(x), _u8(w)
    y_len = batch * out_feat if y_len is None else y_len
    y = np.zeros(max(1, y_len), dtype=np.float32)
    msg = ctypes.c_char_p()
    rc = getattr(lib(), name)(_ptr(x), x.size if x_len is None else x_len, _ptr(w), w.size, _ptr(y), y_len,
                              batch, in_feat, out_feat, ctypes.byref(msg))
    _check(rc, msg)
    return y[:y_len]


def linear_q4_k_cpu(x, w, batch, in_feat, out_feat):
    return _linear_cpu("vtqo_linear_q4_k_cpu", x, w, batch, in_feat, out_feat)


def linear_q6_k_cpu(x, w, batch, in_feat, out_feat):
    return _linear_cpu("vtqo_linear_q6_k_cpu", x, w, batch, in_feat, out_feat)


def linear_q4_0_cpu(x, w, batch, in_feat, out_feat, x_len=None, y_len=None):
    return _linear_cpu("vtqo_linear_q4_0_cpu", x, w, batch, in_feat, out_feat, x_len, y_len)


def linear_dispatch(ggml_type, regime, x, w, batch, in_feat, out_feat, threads=1):
    x, w = _f32(x), _u8(w)
    y = np.zeros(max(1, batch * out_feat), dtype=np.float32)
    msg = ctypes.c_char_p()
    rc = lib().vtqo_linear_dispatch(int(ggml_type), int(regime), _ptr(x), x.size, _ptr(w), w.size, _ptr(y),
                                    batch * out_feat, batch, in_feat, out_feat, threads, ctypes.byref(msg))
    _check(rc, msg)
    return y[: batch * out_feat]


def matmul_f32(a, b, m, k, n):
    a, b = _f32(a), _f32(b)
    out = np.zeros(max(1, m * n), dtype=np.float32)
    lib().vtqo_matmul_f32(_ptr(a), _ptr(b), _ptr(out), m, k, n)
    return out[: m * n]


def lcg_pair(n: int):
    """The reference's test-vector stream (src/ops/quant.rs:1856-1865): a then b from one LCG."""
    s = 0x1234
    mask = (1 << 64) - 1
    vals = np.empty(2 * n, dtype=np.float32)
    for i in range(2 * n):
        s = (s * 6364136223846793005 + 1) & mask
        vals[i] = np.float32(np.float32(s >> 33) / np.float32(2147483648.0)) * np.float32(2.0) - np.float32(1.0)
    return vals[:n].copy(), vals[n:].copy()


def _lcg_states(n: int, seed: int) -> np.ndarray:
    """States s_1..s_n of s = s*6364136223846793005 + 1 (mod 2^64), vectorised by jumping K steps."""
    a, mask, K = 6364136223846793005, (1 << 64) - 1, 1024
    first = np.empty(min(n, K), dtype=np.uint64)
    s = seed
    for i in range(first.size):
        s = (s * a + 1) & mask
        first[i] = s
    if n <= K:
        return first
    # s_{i+K} = A*s_i + C with A = a^K, C = sum_{t<K} a^t (mod 2^64)
    A, C = 1, 0
    for _ in range(K):
        A, C = (A * a) & mask, (C * a + 1) & mask
    out = np.empty(((n + K - 1) // K) * K, dtype=np.uint64)
    out[:K] = first
    with np.errstate(over="ignore"):
        Au, Cu = np.uint64(A), np.uint64(C)
        for j in range(1, out.size // K):
            out[j * K:(j + 1) * K] = out[(j - 1) * K:j * K] * Au + Cu
    return out[:n]


def lcg_bytes(n: int, seed: int) -> np.ndarray:
    """Byte stream of the reference's tests: s = s*6364136223846793005 + 1; byte = s >> 40
    (src/ops/quant.rs:2018-2022)."""
    return ((_lcg_states(n, seed) >> np.uint64(40)) & np.uint64(0xFF)).astype(np.uint8)


def ramp_x(n: int) -> np.ndarray:
    """Activations of the reference's tests: ((i*7919) % 1000) / 500 - 1 (src/ops/quant.rs:2023-2025)."""
    i = np.arange(n, dtype=np.int64)
    return (((i * 7919) % 1000).astype(np.float32) / np.float32(500.0)) - np.float32(1.0)


# ---------------------------------------------------------------- end-to-end


def expf(v: float) -> np.float32:
    return np.float32(lib().vtqo_expf(v))


def powf(x: float, y: float) -> np.float32:
    return np.float32(lib().vtqo_powf(x, y))


def sinf(v: float) -> np.float32:
    return np.float32(lib().vtqo_sinf(v))


def cosf(v: float) -> np.float32:
    return np.float32(lib().vtqo_cosf(v))


def rms_norm(x, w, eps) -> np.ndarray:
    """rms_norm_slice (src/ops/rms_norm.rs:60-110) of one row."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    out = np.empty_like(x)
    lib().vtqo_rms_norm(_ptr(x), _ptr(w), x.size, eps, _ptr(out))
    return out


def softmax(x) -> np.ndarray:
    """softmax_inplace (src/model/forward_quantized.rs:925-941), on a copy."""
    v = np.array(x, dtype=np.float32)
    lib().vtqo_softmax(_ptr(v), v.size)
    return v


def argmax(v) -> int:
    """argmax_last_dim (src/ops/argmax.rs:21-68) of one row."""
    v = np.ascontiguousarray(v, dtype=np.float32)
    return int(lib().vtqo_argmax(_ptr(v), v.size))


def blake3(data) -> str:
    d = _u8(data)
    out = (ctypes.c_uint8 * 32)()
    lib().vtqo_blake3_hash(_ptr(d) if d.size else None, d.size, out)
    return bytes(out).hex()


def transcendental_hash():
    """(input count, hex) of tests/transcendental_determinism.rs's sweep."""
    out = (ctypes.c_uint8 * 32)()
    n = lib().vtqo_transcendental_hash(out)
    return int(n), bytes(out).hex()


def _fields(items):
    names = (ctypes.c_char_p * max(1, len(items)))(*[k.encode() for k, _ in items])
    bufs = [bytes(v) for _, v in items]
    datas = (ctypes.c_char_p * max(1, len(items)))(*bufs)
    lens = (ctypes.c_size_t * max(1, len(items)))(*[len(b) for b in bufs])
    return names, datas, lens, bufs


def gguf_parse(blob, level=0):
    """GgufFile::parse (level 0) or parse + Config / QuantizedWeights (level
    1): (status, message); status 0 is Ok, else the include/vtq.h code of the
    reference's Error variant."""
    b = _u8(blob)
    msg = ctypes.c_char_p()
    rc = lib().vtqo_gguf_parse(_ptr(b) if b.size else None, b.size, level, ctypes.byref(msg))
    return rc, (msg.value.decode() if msg.value else "")


def digest_v1(inputs, outputs) -> str:
    """Frozen vitnify-receipt v1 digest of [(name, bytes)] inputs and outputs."""
    ni, di, li, keep_i = _fields(inputs)
    no, do, lo, keep_o = _fields(outputs)
    out = (ctypes.c_uint8 * 32)()
    lib().vtqo_digest_v1_full(len(inputs), ni, di, li, len(outputs), no, do, lo, 0, None, 0, None, out)
    return bytes(out).hex()


def digest_v2(inputs, outputs) -> str:
    """vitnify-receipt v2 digest of [(name, bytes)] inputs and outputs."""
    ni, di, li, keep_i = _fields(inputs)
    no, do, lo, keep_o = _fields(outputs)
    out = (ctypes.c_uint8 * 32)()
    lib().vtqo_digest_v2(len(inputs), ni, di, li, len(outputs), no, do, lo, out)
    return bytes(out).hex()


RECORD_OPS = 1
RECORD_ACTIVATIONS = 2
NO_LAYER = 0xFFFFFFFF


class OpRecord(ctypes.Structure):
    """OpRecord (src/cert/builder.rs): op_index, layer, op_name, input/params/output hashes."""
    _fields_ = [("op_index", ctypes.c_uint32), ("layer", ctypes.c_uint32), ("op_name", ctypes.c_char * 16),
                ("input_hash", ctypes.c_uint8 * 32), ("params_hash", ctypes.c_uint8 * 32),
                ("output_hash", ctypes.c_uint8 * 32)]

    def key(self):
        return (self.op_index, self.layer, self.op_name, bytes(self.input_hash), bytes(self.params_hash),
                bytes(self.output_hash))


class ActRecord(ctypes.Structure):
    """ActivationRecord (src/cert/builder.rs): act_index, token_index, layer, checkpoint, tensor hash."""
    _fields_ = [("act_index", ctypes.c_uint32), ("token_index", ctypes.c_uint32), ("layer", ctypes.c_uint32),
                ("checkpoint", ctypes.c_char * 16), ("tensor_hash", ctypes.c_uint8 * 32)]

    def key(self):
        return (self.act_index, self.token_index, self.layer, self.checkpoint, bytes(self.tensor_hash))


class Model:
    """GGUF model for inference::run_quantized (the blob must stay alive).
    After run(), digest_v1 holds the frozen v1 digest of the same cert."""

    def __init__(self, blob):
        self.digest_v1 = None
        self.blob = _u8(blob)
        self.handle = ctypes.c_void_p()
        msg = ctypes.c_char_p()
        rc = lib().vtqo_model_load(_ptr(self.blob), self.blob.size, ctypes.byref(self.handle), ctypes.byref(msg))
        _check(rc, msg)
        dims = np.zeros(7, dtype=np.int32)
        lib().vtqo_model_dims(self.handle, _ptr(dims))
        self.dim, self.hidden, self.layers, self.heads, self.kv_heads, self.vocab, self.seq_len = map(int, dims)

    def run(self, prompt, n_new, weights_hash: bytes, regime=0, model_id="vitni-receipt", threads=1,
            want_logits=True):
        prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
        wh = np.frombuffer(bytes(weights_hash), dtype=np.uint8).copy()
        tokens = np.zeros(max(1, n_new), dtype=np.uint32)
        logits = np.zeros((prompt.size + n_new) * self.vocab, dtype=np.float32) if want_logits else None
        digest = (ctypes.c_uint8 * 32)()
        digest_v1 = (ctypes.c_uint8 * 32)()
        msg = ctypes.c_char_p()
        rc = lib().vtqo_run_quantized(self.handle, regime, model_id.encode(), _ptr(wh), _ptr(prompt), prompt.size,
                                      n_new, threads, _ptr(logits), _ptr(tokens), digest, digest_v1,
                                      ctypes.byref(msg))
        _check(rc, msg)
        self.digest_v1 = bytes(digest_v1).hex()  # compute_digest_v1 of the same cert
        if logits is not None:
            logits = logits.reshape(prompt.size + n_new, self.vocab)
        return tokens[:n_new], bytes(digest).hex(), logits

    def run_recorded(self, prompt, n_new, weights_hash: bytes, flags=RECORD_OPS | RECORD_ACTIVATIONS, regime=0,
                     model_id="vitni-receipt", threads=1):
        """run_quantized with per-op / activation recorders on every step:
        (tokens, digest hex, [OpRecord], [ActRecord])."""
        prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
        wh = np.frombuffer(bytes(weights_hash), dtype=np.uint8).copy()
        tokens = np.zeros(max(1, n_new), dtype=np.uint32)
        steps = prompt.size + n_new
        ops = (OpRecord * max(1, steps * (9 * self.layers + 2)))()
        acts = (ActRecord * max(1, steps * (2 * self.layers + 3)))()
        n_ops, n_acts = ctypes.c_size_t(), ctypes.c_size_t()
        digest = (ctypes.c_uint8 * 32)()
        msg = ctypes.c_char_p()
        rc = lib().vtqo_run_quantized_recorded(self.handle, regime, model_id.encode(), _ptr(wh), _ptr(prompt),
                                               prompt.size, n_new, threads, flags, _ptr(tokens), ops, len(ops),
                                               acts, len(acts), ctypes.byref(n_ops), ctypes.byref(n_acts), digest,
                                               ctypes.byref(msg))
        _check(rc, msg)
        return tokens[:n_new], bytes(digest).hex(), list(ops[:n_ops.value]), list(acts[:n_acts.value])

    def __del__(self):
        if getattr(self, "handle", None):
            lib().vtqo_model_free(self.handle)
            self.handle = None
