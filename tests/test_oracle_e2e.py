"""Pins of the oracle's end-to-end pieces (CPU only).

* libm: the reference's PINNED_TRANSCENDENTAL BLAKE3 over expf / sqrtf /
  cosf / sinf / powf(1e4, .) / powf(1e6, .) / sigmoid on 489,509 inputs,
  large-argument cos/sin included (tests/transcendental_determinism.rs:14-63).
* BLAKE3: the published empty-input vector, and the multi-chunk stream of the
  transcendental sweep (13.7 MB) through the pin above.
* receipt: the reference's v2 digest pin (src/cert/builder.rs:719-741).
* forward-step helpers: the reference's known answers for rms_norm
  (src/ops/rms_norm.rs:117-160) and argmax (src/ops/argmax.rs:74-125), and
  closed forms of softmax.
* GGUF: the synthetic model parses to the configured shape.
"""
import numpy as np
import pytest

import oracle
from vtq import synth

SMALL = dict(dim=256, hidden=512, layers=2, heads=4, kv_heads=2, vocab=1000, ctx=64, rope_theta=10000.0,
             rms_eps=1e-5)


def test_transcendental_hash_pinned():
    n, h = oracle.transcendental_hash()
    assert n == 489509
    assert h == "0ae93cd6394c934bfb94a5803a0528193ba0c2330002162a0094062c294bc3d0"


def test_blake3_empty_vector():
    assert oracle.blake3(b"") == "af1349b9f5f9a1a6a0404dea36dcc9499bcb25c9adc112b7cc9a93cae41f3262"


def test_blake3_streaming_boundaries():
    # one-shot vs the same bytes split at chunk and block edges must agree,
    # and every length around the 1024-byte chunk size hashes distinctly
    data = (np.arange(5000) % 251).astype(np.uint8)
    seen = set()
    for n in (0, 1, 63, 64, 65, 1023, 1024, 1025, 2048, 2049, 3072, 4096, 4097, 5000):
        seen.add(oracle.blake3(data[:n]))
    assert len(seen) == 14


def test_digest_v2_pinned():
    d = oracle.digest_v2([("model_id", b"tinyllama"), ("prompt_tokens", bytes([1, 0, 0, 0]))],
                         [("output_tokens", bytes([9, 0, 0, 0]))])
    assert d == "6d5f534cf69c441ba2832c6e63747a7989ccb5de9a2cc9dc528e5b8e0359cf1e"


def test_digest_binds_order_and_lengths():
    a = oracle.digest_v2([("ab", b"c")], [])
    b = oracle.digest_v2([("a", b"bc")], [])
    c = oracle.digest_v2([], [("ab", b"c")])
    assert len({a, b, c}) == 3


def test_libm_closed_forms():
    # values every float libm must get exactly
    assert oracle.expf(0.0) == 1.0
    assert oracle.cosf(0.0) == 1.0 and oracle.sinf(0.0) == 0.0
    assert oracle.powf(10000.0, 0.0) == 1.0 and oracle.powf(2.0, 10.0) == 1024.0
    assert oracle.powf(10000.0, 0.5) == 100.0
    assert np.isinf(oracle.expf(89.0)) and oracle.expf(-104.0) == 0.0


def test_synthetic_gguf_parses_to_config():
    blob, prompt = synth.e2e_inputs(SMALL, 8)
    m = oracle.Model(blob)
    assert (m.dim, m.hidden, m.layers, m.heads, m.kv_heads, m.vocab, m.seq_len) == (256, 512, 2, 4, 2, 1000, 64)
    assert prompt.max() < 1000


def test_run_quantized_deterministic_and_threads_invariant():
    blob, prompt = synth.e2e_inputs(SMALL, 8)
    wh = bytes.fromhex(oracle.blake3(blob))
    m = oracle.Model(blob)
    t1, d1, l1 = m.run(prompt, 8, wh, regime=0, threads=1)
    t2, d2, l2 = m.run(prompt, 8, wh, regime=0, threads=4)
    assert d1 == d2 and np.array_equal(l1.view(np.uint32), l2.view(np.uint32))
    assert np.isfinite(l1).all()


def test_run_quantized_errors():
    blob, prompt = synth.e2e_inputs(SMALL, 8)
    m = oracle.Model(blob)
    with pytest.raises(oracle.OracleError, match="exceeds seq_len"):
        m.run(prompt, 64, b"\0" * 32)
    with pytest.raises(oracle.OracleError, match="bad magic"):
        oracle.Model(np.frombuffer(b"GGML" + b"\0" * 60, dtype=np.uint8))


def test_rms_norm_reference_known_answers():
    # rms_norm_identity_scale, rms_norm_weighted: exact; rms_norm_known: the
    # reference's 1e-4 tolerance, and the bits of x * (1/sqrt(12.5)) * 1
    assert np.array_equal(oracle.rms_norm(np.ones(4), np.ones(4), 0.0), np.ones(4, dtype=np.float32))
    assert np.array_equal(oracle.rms_norm([1.0, 1.0], [2.0, 3.0], 0.0), np.array([2.0, 3.0], dtype=np.float32))
    y = oracle.rms_norm([3.0, 4.0], [1.0, 1.0], 0.0)
    assert abs(y[0] - 0.8485281) < 1e-4 and abs(y[1] - 1.1313708) < 1e-4
    scale = np.float32(1.0) / np.sqrt(np.float32(12.5))  # sum 25 and mean 12.5 are exact
    assert y.tobytes() == (np.array([3.0, 4.0], dtype=np.float32) * scale).tobytes()
    # the sum of squares is serial: 1 + 2^-24 + 2^-24 rounds each add back to 1
    x = np.array([1.0, 2.0 ** -12, 2.0 ** -12], dtype=np.float32)
    serial = oracle.rms_norm(x, np.ones(3), 0.0)
    scale = np.float32(1.0) / np.sqrt(np.float32(1.0) / np.float32(3.0))
    assert serial.tobytes() == (x * scale).tobytes()


def test_argmax_reference_known_answers():
    assert oracle.argmax([0.1, 0.5, 0.3, 0.8, 0.2]) == 3          # argmax_simple
    assert oracle.argmax([0.1, 0.5, 0.3, 0.5, 0.2]) == 1          # argmax_tie_picks_first
    assert oracle.argmax([0.1, 0.5, 0.3]) == 1 and oracle.argmax([0.9, 0.2, 0.4]) == 0  # argmax_per_row
    nan = float("nan")
    assert oracle.argmax([nan, 5.0, 7.0]) == 0                      # nothing is > NaN at index 0
    assert oracle.argmax([1.0, nan, 7.0, 7.0]) == 2                 # later NaNs never win
    assert oracle.argmax([-0.0, 0.0]) == 0                          # +0 > -0 is false


def test_softmax_closed_forms():
    for n in (1, 2, 4, 64, 256):
        assert np.array_equal(oracle.softmax(np.full(n, 3.5)), np.full(n, 1.0 / n, dtype=np.float32))
    y = oracle.softmax([0.0, float(np.log(3.0))])
    assert abs(float(y.sum()) - 1.0) < 1e-6 and y[1] > y[0]
    # the max is subtracted first: huge equal inputs do not overflow
    assert np.array_equal(oracle.softmax([1e30, 1e30]), np.array([0.5, 0.5], dtype=np.float32))


def test_per_op_and_activation_receipts():
    # perop_records_expected_count_and_matches_baseline_logits and
    # perop_records_are_deterministic_across_runs (forward_quantized.rs:1235-1420):
    # 9 ops per layer + 2 per step, the recorder only observes, and the same
    # run gives the same records and digest
    blob, prompt = synth.e2e_inputs(SMALL, 5)
    wh = bytes.fromhex(oracle.blake3(blob))
    m = oracle.Model(blob)
    tokens, digest, _ = m.run(prompt, 3, wh, want_logits=False)
    t1, d1, ops, acts = m.run_recorded(prompt, 3, wh)
    steps, L = 8, SMALL["layers"]
    assert np.array_equal(t1, tokens)
    assert len(ops) == steps * (9 * L + 2) and len(acts) == steps * (2 * L + 3)
    assert [o.op_index for o in ops] == list(range(len(ops)))
    assert ops[0].op_name == b"rms_norm" and ops[1].op_name == b"linear_q4_0" and ops[0].layer == 0
    assert ops[9 * L].layer == oracle.NO_LAYER and ops[9 * L + 1].op_name == b"linear_q4_0"
    assert [a.checkpoint for a in acts[:2 * L + 3]] == [b"post_embed"] + [b"post_attn", b"post_ffn"] * L + \
        [b"pre_lm_head", b"post_lm_head"]
    assert acts[2 * L + 3].token_index == 1
    # op inputs chain to the previous op's output where the reference feeds them
    assert bytes(ops[1].input_hash) == bytes(ops[0].output_hash) == bytes(ops[2].input_hash)
    # the records are bound into the digest; without recorders it is run_quantized's
    assert d1 != digest
    t2, d2, ops2, acts2 = m.run_recorded(prompt, 3, wh)
    assert d2 == d1 and [o.key() for o in ops2] == [o.key() for o in ops]
    _, d_ops, ops_only, acts_none = m.run_recorded(prompt, 3, wh, flags=oracle.RECORD_OPS)
    assert acts_none == [] and len(ops_only) == len(ops) and d_ops not in (d1, digest)
    _, d0, _, _ = m.run_recorded(prompt, 3, wh, flags=0)
    assert d0 == digest


def _leb128(v):
    out = bytearray()
    while True:
        b = v & 0x7F
        v >>= 7
        out.append(b | (0x80 if v else 0))
        if not v:
            return bytes(out)


def _frame(domain, regime, inputs, outputs):
    """write_sections (src/cert/builder.rs:491-519) with the v1 or v2 domain,
    framed here in Python, independently of the oracle's C framing."""
    b = bytearray(domain)
    if regime is not None:
        b += _leb128(len(regime)) + regime
    for fields in (inputs, outputs):
        b += _leb128(len(fields))
        for k, v in fields:
            b += _leb128(len(k)) + k.encode() + _leb128(len(v)) + v
    b += b"\0\0\0"  # no ops, activations, interventions
    return bytes(b)


def test_digest_v1_is_the_frozen_framing():
    """compute_digest_v1 (builder.rs:476-487): the v2 sections under the v1
    domain with no regime.  The Python framing is pinned first by
    reproducing the reference's v2 constant; under the v1 domain it must
    then equal the oracle's v1, and v1 must differ from v2 (builder.rs:738-740)."""
    ins = [("model_id", b"tinyllama"), ("prompt_tokens", bytes([1, 0, 0, 0]))]
    outs = [("output_tokens", bytes([9, 0, 0, 0]))]
    v2 = oracle.blake3(_frame(b"vitnify-receipt v2\0", b"vitni-regime-1", ins, outs))
    assert v2 == "6d5f534cf69c441ba2832c6e63747a7989ccb5de9a2cc9dc528e5b8e0359cf1e"
    v1 = oracle.blake3(_frame(b"vitnify-receipt v1\0", None, ins, outs))
    assert oracle.digest_v1(ins, outs) == v1 != v2


def test_run_quantized_v1_digest():
    blob, prompt = synth.e2e_inputs(SMALL, 5)
    wh = bytes.fromhex(oracle.blake3(blob))
    m = oracle.Model(blob)
    toks, d2, _ = m.run(prompt, 4, wh, regime=0, want_logits=False)
    arch = (f"llama2c:dim=256,hidden=512,layers=2,heads=4,kv_heads=2,vocab=1000,seq=64,shared=false").encode()
    ins = [("model_id", b"vitni-receipt"), ("weights_hash", wh), ("arch_hash", bytes.fromhex(oracle.blake3(arch))),
           ("prompt_tokens", prompt.astype("<u4").tobytes()), ("n_new_tokens", (4).to_bytes(4, "little"))]
    ob = toks.astype("<u4").tobytes()
    outs = [("output_tokens", ob), ("output_tokens_hash", bytes.fromhex(oracle.blake3(ob)))]
    assert d2 == oracle.blake3(_frame(b"vitnify-receipt v2\0", b"vitni-regime-1", ins, outs))
    assert m.digest_v1 == oracle.blake3(_frame(b"vitnify-receipt v1\0", None, ins, outs)) != d2


def test_model_variants_load():
    """The Qwen2 layout (qwen2.* keys: NeoX RoPE), the tied head (no
    output.weight) and attention biases parse as QuantizedWeights does, and
    each changes the computation."""
    cfg = dict(SMALL, vocab=256)
    runs = {}
    for name, kw in [("llama", {}), ("qwen2", dict(arch="qwen2")), ("tied", dict(tied=True)),
                     ("bias", dict(qkv_bias=True)), ("align8", dict(alignment=8))]:
        blob, prompt = synth.e2e_inputs(cfg, 6, **kw)
        m = oracle.Model(blob)
        assert (m.dim, m.vocab) == (256, 256)
        t, d, lg = m.run(prompt, 4, b"\0" * 32, regime=0)
        assert np.isfinite(lg).all()
        runs[name] = lg
    # alignment only moves bytes; every other variant changes the logits
    assert np.array_equal(runs["align8"].view(np.uint32), runs["llama"].view(np.uint32))
    for name in ("qwen2", "tied", "bias"):
        assert not np.array_equal(runs[name], runs["llama"]), name


def test_run_errors_follow_the_reference_order():
    import gguf_edit

    cfg = dict(SMALL, vocab=256)
    # a K projection 4 rows short: linear_dispatch's shape check, per regime's function
    blob, prompt = synth.e2e_inputs(cfg, 4, short_rows=4)
    m = oracle.Model(blob)
    with pytest.raises(oracle.OracleError) as e:
        m.run(prompt, 2, b"\0" * 32, regime=0)
    assert (e.value.code, e.value.message) == (1, "linear_q4_k_integer: weight shape mismatch")
    with pytest.raises(oracle.OracleError) as e:
        m.run(prompt, 2, b"\0" * 32, regime=1)
    assert (e.value.code, e.value.message) == (1, "linear_q4_k_fused: weight shape mismatch")
    # a norm weight of the wrong length: rms_norm_slice's ShapeMismatch
    blob, prompt = synth.e2e_inputs(cfg, 4)
    bad = gguf_edit.set_tensor_dims(blob, "blk.1.ffn_norm.weight", [252])
    with pytest.raises(oracle.OracleError) as e:
        oracle.Model(bad).run(prompt, 2, b"\0" * 32)
    assert (e.value.code, e.value.message) == (8, "expected weight length == last dim of x, got weight mismatch")
    # a prompt token past the embedding table
    m = oracle.Model(blob)
    with pytest.raises(oracle.OracleError) as e:
        m.run(np.array([3, 256], dtype=np.uint32), 2, b"\0" * 32)
    assert (e.value.code, e.value.message) == (1, "embedding_row Q4_K: row past end of table")
    with pytest.raises(oracle.OracleError) as e:
        m.run(np.zeros(0, dtype=np.uint32), 2, b"\0" * 32)
    assert (e.value.code, e.value.message) == (9, "prompt_tokens must not be empty")
