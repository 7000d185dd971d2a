"""Seeded synthetic workloads of the benchmark configurations.

Wraps libvtq_synth.so (generator specified in synth/vtq_synth.h).  The same
bytes are produced on every machine with this image, so tests and the
benchmark feed the GPU path and the CPU oracle identical inputs.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import numpy as np

from . import BLOCK, F32, LIB_DIR, Q4_0, Q4_K, Q5_0, Q6_K, Q8_0

SEED_BASE = 0x5654_5100_0000_0000
X_SEED_OFFSET = 0x80
SCALE_SIGMA = 0.01  # d, dmin = f16(|N(0, 0.01)|)

_synth = None


class LlamaCfg(ctypes.Structure):
    """vtqs_llama (synth/vtq_synth.h)"""

    _fields_ = [("dim", ctypes.c_uint32), ("hidden", ctypes.c_uint32), ("layers", ctypes.c_uint32),
                ("heads", ctypes.c_uint32), ("kv_heads", ctypes.c_uint32), ("vocab", ctypes.c_uint32),
                ("ctx", ctypes.c_uint32), ("rope_theta", ctypes.c_float), ("rms_eps", ctypes.c_float),
                ("arch", ctypes.c_uint32), ("tied", ctypes.c_uint32), ("qkv_bias", ctypes.c_uint32),
                ("alignment", ctypes.c_uint32), ("short_rows", ctypes.c_uint32)]


def lib() -> ctypes.CDLL:
    global _synth
    if _synth is None:
        path = os.path.join(LIB_DIR, "libvtq_synth.so")
        if not os.path.exists(path):
            raise ImportError(f"{path} is missing (run __graft_entry__.build())")
        s = ctypes.CDLL(path)
        u64, vp, sz, f = ctypes.c_uint64, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_float
        for name in ("vtqs_q4_k", "vtqs_q6_k", "vtqs_q8_0", "vtqs_q5_0", "vtqs_q4_0"):
            getattr(s, name).argtypes = [u64, vp, sz, sz, f]
            getattr(s, name).restype = None
        s.vtqs_normal_f32.argtypes = [u64, vp, sz, f]
        s.vtqs_normal_f32.restype = None
        s.vtqs_bytes.argtypes = [u64, vp, sz]
        s.vtqs_bytes.restype = None
        s.vtqs_f32_to_f16_rne.argtypes = [f]
        s.vtqs_f32_to_f16_rne.restype = ctypes.c_uint16
        s.vtqs_tokens.argtypes = [u64, vp, sz, ctypes.c_uint32]
        s.vtqs_tokens.restype = None
        s.vtqs_llama_gguf.argtypes = [ctypes.POINTER(LlamaCfg), u64, vp]
        s.vtqs_llama_gguf.restype = sz
        _synth = s
    return _synth


def weights(ggml_type: int, rows: int, in_feat: int, seed: int, sigma: float = SCALE_SIGMA) -> np.ndarray:
    """GGUF blocks of W[rows, in_feat] (uint8), generator of vtq_synth.h."""
    s = lib()
    if ggml_type == F32:
        w = np.empty(rows * in_feat, dtype=np.float32)
        s.vtqs_normal_f32(seed, w.ctypes.data, w.size, sigma)
        return w.view(np.uint8)
    numel, nbytes = BLOCK[ggml_type]
    assert in_feat % numel == 0
    w = np.empty(rows * (in_feat // numel) * nbytes, dtype=np.uint8)
    fn = {Q4_K: s.vtqs_q4_k, Q6_K: s.vtqs_q6_k, Q8_0: s.vtqs_q8_0, Q5_0: s.vtqs_q5_0, Q4_0: s.vtqs_q4_0}[ggml_type]
    fn(seed, w.ctypes.data, rows, in_feat, sigma)
    return w


def activations(n: int, seed: int, sigma: float = 1.0) -> np.ndarray:
    x = np.empty(n, dtype=np.float32)
    lib().vtqs_normal_f32(seed, x.ctypes.data, n, sigma)
    return x


def random_bytes(n: int, seed: int) -> np.ndarray:
    w = np.empty(n, dtype=np.uint8)
    lib().vtqs_bytes(seed, w.ctypes.data, n)
    return w


@dataclass(frozen=True)
class Config:
    """One BASELINE.json configuration of the linear layer."""

    index: int
    name: str
    ggml_type: int
    out_feat: int
    in_feat: int
    batch: int

    @property
    def w_seed(self) -> int:
        return SEED_BASE + self.index

    @property
    def x_seed(self) -> int:
        return SEED_BASE + self.index + X_SEED_OFFSET

    def make(self, rows: int | None = None, batch: int | None = None):
        """(x, w) for the first `rows` output rows (default all) and `batch` rows of x."""
        rows = self.out_feat if rows is None else rows
        batch = self.batch if batch is None else batch
        w = weights(self.ggml_type, rows, self.in_feat, self.w_seed)
        x = activations(batch * self.in_feat, self.x_seed)
        return x, w

    def weight_bytes(self) -> int:
        numel, nbytes = BLOCK[self.ggml_type]
        return self.out_feat * (self.in_feat // numel) * nbytes

    def algorithmic_bytes(self) -> int:
        """Packed weights + fp32 activations in + fp32 outputs out."""
        return self.weight_bytes() + 4 * self.batch * (self.in_feat + self.out_feat)


CONFIGS = {
    "q8_0_4096x4096": Config(0, "q8_0_4096x4096", Q8_0, 4096, 4096, 1),
    "q4k_11008x4096": Config(1, "q4k_11008x4096", Q4_K, 11008, 4096, 1),
    "q4k_4096x11008": Config(2, "q4k_4096x11008", Q4_K, 4096, 11008, 1),
    "q6k_32000x4096": Config(3, "q6k_32000x4096", Q6_K, 32000, 4096, 1),
    "q4k_gemm_14336x4096_m512": Config(4, "q4k_gemm_14336x4096_m512", Q4_K, 14336, 4096, 512),
}


# ---------------------------------------------------------------- config 5

# random-init Llama 1.1B, Q4_K attention/FFN and
# token_embd, Q6_K output head, F32 norms; 128 random prompt ids, 64 new tokens
LLAMA_1B1 = dict(dim=2048, hidden=5632, layers=22, heads=32, kv_heads=4, vocab=32000, ctx=1024,
                 rope_theta=10000.0, rms_eps=1e-5)
E2E_INDEX = 4
E2E_PROMPT = 128
E2E_NEW = 64


def llama_gguf(cfg: dict, seed: int, arch: str = "llama", tied: bool = False, qkv_bias: bool = False,
               alignment: int = 32, short_rows: int = 0) -> np.ndarray:
    """GGUF v3 blob of a random-init Llama (or Qwen2-layout) model
    (synth/vtq_synth.h): arch "qwen2" names the qwen2.* keys (NeoX RoPE),
    tied drops output.weight (the head is token_embd), qkv_bias adds the
    attention biases, alignment sets general.alignment, short_rows drops
    rows from blk.0.attn_k.weight."""
    c = LlamaCfg(**cfg, arch={"llama": 0, "qwen2": 1}[arch], tied=int(tied), qkv_bias=int(qkv_bias),
                 alignment=alignment, short_rows=short_rows)
    n = lib().vtqs_llama_gguf(ctypes.byref(c), seed, None)
    out = np.empty(n, dtype=np.uint8)
    lib().vtqs_llama_gguf(ctypes.byref(c), seed, out.ctypes.data)
    return out


def tokens(seed: int, n: int, vocab: int) -> np.ndarray:
    out = np.empty(n, dtype=np.uint32)
    lib().vtqs_tokens(seed, out.ctypes.data, n, vocab)
    return out


def e2e_inputs(cfg: dict = None, prompt_len: int = E2E_PROMPT, **variant):
    """(gguf blob, prompt ids) of the end-to-end configuration; `variant`
    passes llama_gguf's options (arch, tied, qkv_bias, alignment, short_rows)."""
    cfg = LLAMA_1B1 if cfg is None else cfg
    blob = llama_gguf(cfg, SEED_BASE + E2E_INDEX, **variant)
    prompt = tokens(SEED_BASE + E2E_INDEX + X_SEED_OFFSET, prompt_len, cfg["vocab"])
    return blob, prompt
