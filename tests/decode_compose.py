"""Decode steps of degenerate models, composed from independently pinned parts.

A decode step (src/model/forward_quantized.rs:380-660) is a composition of
parts that the oracle pins one by one: embedding_row (a dequantize, pinned by
the reference's known-answer blocks), rms_norm_slice, linear_dispatch, the
libm expf of SiLU, and argmax.  The composition itself (which tensor feeds
which, the residual wiring, the GQA head map h / kv_mul, the KV-cache
indexing, RoPE placement, the token loop of run_quantized,
src/model/inference.rs:312-327) has no reference vector.  For the models
below the step reduces to those parts exactly, so a run of the oracle or of
the GPU runtime can be checked against them without trusting either one's
own step:

* zero_out: every attn_output and ffn_down weight is zero, so the residual
  stream stays the embedding row (up to the sign of exact zeros, which the
  head's activation quantization cannot see) and each step's logits are
  head(rms_norm(embedding_row(token), output_norm)).  This pins the token
  loop: which token feeds step t, which logits row is recorded, and that the
  token picked after the last prompt position is fed but not returned.
* step0: at position 0 the softmax has one score, exp(0) = 1 and 1 / 1 = 1,
  so each head's attention output is 0.0 + 1.0 * v of its KV head; RoPE at
  position 0 only touches q and k.  Step 0's logits are then a chain of
  norms, linears, the SwiGLU and residual adds (any model).
* zero_q: every attn_q weight (and bias) is zero, so q is +0.0 after RoPE,
  every score is +0.0, each softmax weight is exactly 1 / (pos + 1) and a
  head's output is the serial f32 sum over the cached positions of that
  weight times v of its KV head: it pins the cache indexing and h / kv_mul
  at every position.

Test infrastructure: it imports the oracle, never the product.
"""
import numpy as np

import gguf_edit as G
import oracle as O

F = np.float32
Q4_K, Q6_K, F32_T = 12, 14, 0


class Weights:
    """Tensors of a synthetic Llama / Qwen2 GGUF blob (the layout of
    synth/vtq_synth.c) and the model's dimensions."""

    def __init__(self, blob, cfg, threads=8):
        self.raw = np.frombuffer(bytes(blob), np.uint8)
        self.table = G.tensor_table(blob)
        self.cfg = cfg
        self.dim, self.hidden, self.layers = cfg["dim"], cfg["hidden"], cfg["layers"]
        self.heads, self.kv_heads, self.vocab = cfg["heads"], cfg["kv_heads"], cfg["vocab"]
        self.hs = self.dim // self.heads
        self.kv_dim = self.kv_heads * self.hs
        self.kv_mul = self.heads // self.kv_heads
        self.eps = F(cfg["rms_eps"])
        self.threads = threads

    def has(self, name):
        return name in self.table

    def bytes(self, name):
        _, _, off, size = self.table[name]
        return self.raw[off:off + size]

    def f32(self, name):
        return self.bytes(name).view(F)

    def linear(self, name, x, in_f, out_f):
        t = self.table[name][1]
        return O.linear_dispatch(t, 0, x, self.bytes(name), 1, in_f, out_f, self.threads)

    def embedding_row(self, tok):
        # embedding_row Q4_K (src/model/forward_quantized.rs:818-923): dequantize one row
        rb = self.dim // 256 * 144
        return O.dequantize("q4_k", self.bytes("token_embd.weight")[tok * rb:(tok + 1) * rb])

    def head(self, x):
        xf = O.rms_norm(x, self.f32("output_norm.weight"), self.eps)
        name = "output.weight" if self.has("output.weight") else "token_embd.weight"  # tied head
        return self.linear(name, xf, self.dim, self.vocab)

    def add_bias(self, v, name):
        return v + self.f32(name) if self.has(name) else v

    def ffn(self, l, x):
        n = O.rms_norm(x, self.f32(f"blk.{l}.ffn_norm.weight"), self.eps)
        g = self.linear(f"blk.{l}.ffn_gate.weight", n, self.dim, self.hidden)
        u = self.linear(f"blk.{l}.ffn_up.weight", n, self.dim, self.hidden)
        e = np.array([O.expf(-gi) for gi in g], F)
        inner = (g / (F(1.0) + e)) * u  # silu(g) * u, each op rounded in f32
        return x + self.linear(f"blk.{l}.ffn_down.weight", inner, self.hidden, self.dim)

    def v_rows(self, l, x):
        xb = O.rms_norm(x, self.f32(f"blk.{l}.attn_norm.weight"), self.eps)
        v = self.linear(f"blk.{l}.attn_v.weight", xb, self.dim, self.kv_dim)
        return self.add_bias(v, f"blk.{l}.attn_v.bias")

    def attn_out(self, l, heads_out, x):
        return x + self.linear(f"blk.{l}.attn_output.weight", heads_out, self.dim, self.dim)


def token_loop(prompt, n_new, logits_of):
    """run_quantized's loop (src/model/inference.rs:312-327): step t feeds
    prompt[t] inside the prompt, else the argmax of step t - 1; tokens are
    the argmaxes of steps prompt_len .. prompt_len + n_new - 1."""
    cur, rows, out = int(prompt[0]), [], []
    total = len(prompt) + n_new
    for pos in range(total):
        lg = logits_of(pos, cur)
        rows.append(lg)
        picked = O.argmax(lg)
        nxt = int(prompt[pos + 1]) if pos + 1 < len(prompt) else picked
        if pos >= len(prompt):
            out.append(nxt)
        cur = nxt
    return np.array(out, np.uint32), np.stack(rows)


def zero_out_model(blob, layers):
    names = [f"blk.{l}.attn_output.weight" for l in range(layers)] + \
            [f"blk.{l}.ffn_down.weight" for l in range(layers)]
    return G.zero_tensors(blob, names)


def zero_out_run(w, prompt, n_new):
    """(tokens, logits per step) of a zero_out model."""
    return token_loop(prompt, n_new, lambda pos, tok: w.head(w.embedding_row(tok)))


def step0_logits(w, tok):
    """Step 0 of any model: each head's attention output is 0.0 + 1.0 * v."""
    x = w.embedding_row(tok)
    for l in range(w.layers):
        v = w.v_rows(l, x)
        heads_out = np.concatenate([F(0.0) + F(1.0) * v[(h // w.kv_mul) * w.hs:(h // w.kv_mul + 1) * w.hs]
                                    for h in range(w.heads)]).astype(F)
        x = w.attn_out(l, heads_out, x)
        x = w.ffn(l, x)
    return w.head(x)


def zero_q_model(blob, layers):
    names = [f"blk.{l}.attn_q.weight" for l in range(layers)]
    table = G.tensor_table(blob)
    names += [f"blk.{l}.attn_q.bias" for l in range(layers) if f"blk.{l}.attn_q.bias" in table]
    return G.zero_tensors(blob, names)


def zero_q_run(w, prompt, n_new):
    """(tokens, logits per step) of a zero_q model: at position p every
    softmax weight is fl(1 / (p + 1)) and a head's output is the serial sum,
    from 0.0 in position order, of weight * v of its KV head."""
    cache = [[] for _ in range(w.layers)]  # v rows per layer, in position order

    def logits_of(pos, tok):
        x = w.embedding_row(tok)
        a = F(1.0) * (F(1.0) / F(pos + 1))  # exp(0) = 1 each; inv = 1 / sum; weight = 1 * inv
        for l in range(w.layers):
            cache[l].append(w.v_rows(l, x))
            heads_out = np.zeros(w.dim, F)
            for h in range(w.heads):
                kv = (h // w.kv_mul) * w.hs
                acc = np.zeros(w.hs, F)
                for t in range(pos + 1):
                    acc = acc + a * cache[l][t][kv:kv + w.hs]
                heads_out[h * w.hs:(h + 1) * w.hs] = acc
            x = w.attn_out(l, heads_out, x)
            x = w.ffn(l, x)
        return w.head(x)

    return token_loop(prompt, n_new, logits_of)


# ------------------------------------------------------- adversarial rows

def _q4k_block(d_bits, dmin_bits, sc, m, qs):
    """One Q4_K block from f16 d / dmin bits, 8 six-bit scales and mins and
    256 four-bit codes (the packing get_scale_min_k4 reads,
    src/ops/quant.rs:267-276)."""
    s = np.zeros(12, np.uint8)
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (m[j] & 63) | ((m[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((m[j + 4] & 15) << 4)
    q = np.asarray(qs, np.uint8).reshape(4, 2, 32)  # element 64h + 32hi + l
    packed = (q[:, 0, :] | (q[:, 1, :] << 4)).reshape(128)
    return np.concatenate([np.frombuffer(np.uint16(d_bits).tobytes(), np.uint8),
                           np.frombuffer(np.uint16(dmin_bits).tobytes(), np.uint8), s, packed]).astype(np.uint8)


def adversarial_row(kind, dim, rng):
    """Q4_K bytes of one embedding row of the given kind: 'halves' (x = q/2,
    squares with ties), 'short' (a 2^-6 grid), 'huge' (|x| up to 6.2e7),
    'outliers' (one block 10^4 times the rest), 'nan', 'inf', 'zero'."""
    nb = dim // 256
    blocks = []
    for b in range(nb):
        qs = rng.integers(0, 16, 256)
        sc, m, d, dmin = [1] * 8, [0] * 8, 0x3800, 0  # d = 0.5
        if kind == "short":
            sc, d = list(rng.integers(1, 4, 8)), 0x2400  # d = 2^-6
        elif kind == "huge":
            sc, d = [63] * 8, 0x7BFF  # d = 65504
        elif kind == "outliers":
            sc, m, d, dmin = list(rng.integers(1, 64, 8)), list(rng.integers(0, 64, 8)), 0x1E66, 0x1A66
            if b == nb // 2:
                d = 0x5A00  # 192: four orders of magnitude above the rest
        elif kind == "nan" and b == nb - 1:
            d = 0x7E00
        elif kind == "inf" and b == 0:
            d, qs = 0x7C00, np.maximum(qs, 1)
        elif kind == "zero":
            d, qs = 0, np.zeros(256, np.int64)
        blocks.append(_q4k_block(d, dmin, sc, m, qs))
    return np.concatenate(blocks)


ADVERSARIAL_KINDS = ["halves", "short", "huge", "outliers", "nan", "inf", "zero"]


def with_embedding_rows(blob, dim, rows):
    """The blob with token_embd rows replaced: rows = {token: Q4_K bytes}."""
    b = bytearray(bytes(blob))
    _, t, off, size = G.tensor_table(b)["token_embd.weight"]
    assert t == Q4_K
    rb = dim // 256 * 144
    for tok, data in rows.items():
        assert data.size == rb and (tok + 1) * rb <= size
        b[off + tok * rb:off + (tok + 1) * rb] = data.tobytes()
    return bytes(b)


def bits_equal_nan(got, want):
    """Finite outputs bit for bit, the same NaN positions (IEEE leaves NaN
    payloads unspecified), infinities exactly."""
    got, want = np.asarray(got, F).reshape(-1), np.asarray(want, F).reshape(-1)
    nan_g, nan_w = np.isnan(got), np.isnan(want)
    return bool(np.array_equal(nan_g, nan_w) and
                np.array_equal(got[~nan_w].view(np.uint32), want[~nan_w].view(np.uint32)))
