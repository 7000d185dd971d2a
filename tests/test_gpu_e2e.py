"""End-to-end decode on the GPU runtime vs the CPU oracle (config 5).

libvtq_runtime (every linear on the GPU through libvtq) must reproduce the
oracle's restatement of inference::run_quantized (src/model/inference.rs:
274-345) bit for bit: the logits of every decode step, the generated tokens
and the vitnify-receipt v2 digest, in both Q4_K regimes, with the prompt
taken in one batched pass (the runtime's default) and step by step.
"""
import numpy as np
import pytest

import oracle
from vtq import runtime, synth

pytestmark = pytest.mark.gpu

SMALL = dict(dim=256, hidden=512, layers=2, heads=4, kv_heads=2, vocab=1000, ctx=64, rope_theta=10000.0,
             rms_eps=1e-5)
MEDIUM = dict(dim=512, hidden=1536, layers=4, heads=8, kv_heads=2, vocab=4096, ctx=160, rope_theta=10000.0,
              rms_eps=1e-5)
# dim 2560: the fused RMSNorm's serial chain over two passes, the second
# partial; head_dim 128 and positions past 256: attention's general path;
# hidden 4352: two-window rows for W2
WIDE = dict(dim=2560, hidden=4352, layers=1, heads=20, kv_heads=4, vocab=512, ctx=300, rope_theta=10000.0,
            rms_eps=1e-5)
# dim 1024 and 4096: the smallest and largest rows the fused RMSNorm's binade
# walk takes (a 640-term serial head, and a 2560-term one with the walk's full
# 1536 terms after it)
WALK_LO = dict(dim=1024, hidden=768, layers=1, heads=16, kv_heads=4, vocab=512, ctx=40, rope_theta=10000.0,
               rms_eps=1e-5)
WALK_HI = dict(dim=4096, hidden=1024, layers=1, heads=32, kv_heads=8, vocab=512, ctx=40, rope_theta=10000.0,
               rms_eps=1e-5)


def compare(cfg, prompt_len, n_new, regimes=(0, 1), threads=8, **variant):
    blob, prompt = synth.e2e_inputs(cfg, prompt_len, **variant)
    wh_o = bytes.fromhex(oracle.blake3(blob))
    wh_p = runtime.blake3(blob)
    assert wh_o == wh_p
    om = oracle.Model(blob)
    gm = runtime.Model(blob)
    try:
        for regime in regimes:
            t_o, d_o, l_o = om.run(prompt, n_new, wh_o, regime=regime, threads=threads)
            for stepwise in (False, True):
                mode = f"regime {regime}, {'stepwise' if stepwise else 'batched'} prompt"
                t_g, d_g, l_g = gm.run(prompt, n_new, wh_p, regime=regime, stepwise=stepwise)
                assert l_g.shape == l_o.shape
                bad = np.nonzero((l_g.view(np.uint32) != l_o.view(np.uint32)).any(axis=1))[0]
                assert bad.size == 0, f"{mode}: logits differ first at step {bad[0]}"
                assert np.array_equal(t_g, t_o), f"{mode}: tokens {t_g} vs {t_o}"
                assert d_g == d_o, f"{mode}: digest {d_g} vs {d_o}"
                # compute_digest_v1 of the same cert (vitni-receipt's model_digest_v1)
                assert gm.digest_v1 == om.digest_v1 != d_o
                # without the logits history the batched pass computes only
                # the last prompt position's logits
                t_n, d_n, _ = gm.run(prompt, n_new, wh_p, regime=regime, stepwise=stepwise, want_logits=False)
                assert np.array_equal(t_n, t_o) and d_n == d_o, f"{mode}, no logits history"
    finally:
        gm.close()
    return d_o


def test_e2e_small_both_regimes():
    compare(SMALL, 8, 8)


def test_e2e_batched_prompt_lengths():
    # prompts of 2 (the smallest batched pass), 31 / 32 / 33 rows (the
    # linears switch from the batched GEMV to the prefill GEMM at 32) and a
    # prompt with no new tokens (the pass ends at the last prompt step)
    for p, n in ((2, 3), (31, 2), (32, 2), (33, 2), (40, 0)):
        compare(MEDIUM, p, n, regimes=(0,))
    compare(SMALL, 33, 4, regimes=(1,))


def test_e2e_medium_odd_lengths():
    # kv heads < heads (GQA), prompt of 1, long generation
    compare(MEDIUM, 1, 40, regimes=(0,))
    compare(MEDIUM, 13, 29, regimes=(1,))


def test_e2e_wide_long_context():
    compare(WIDE, 250, 12, regimes=(0,), threads=16)


# A context too long for the attention kernel's LDS (30000 scores beside the
# cached-v tiles): every head keeps its scores in a row of HBM.  Positions
# past 256 also take the tiled path of the weighted sum.
LONG_CTX = dict(dim=256, hidden=512, layers=2, heads=4, kv_heads=2, vocab=1000, ctx=30000, rope_theta=10000.0,
                rms_eps=1e-5)


def test_e2e_context_beyond_lds_scores():
    compare(LONG_CTX, 280, 10, regimes=(0,), threads=16)


# Head dims other than 64 and 128 take both attention kernels' generic
# instantiations.  32 with eight query heads per KV head: the prompt pass's
# workgroups of 8 waves use 256-row tiles of the cache, which a 300-position
# prompt crosses.  256 with two query heads per KV head (qwen2: NeoX pairs
# and biases): 2-wave workgroups and 8-row tiles.
HD32 = dict(dim=256, hidden=512, layers=2, heads=8, kv_heads=1, vocab=1000, ctx=320, rope_theta=10000.0,
            rms_eps=1e-5)
HD256 = dict(dim=512, hidden=512, layers=2, heads=2, kv_heads=1, vocab=1000, ctx=48, rope_theta=10000.0,
             rms_eps=1e-5)


def test_e2e_generic_head_dims():
    compare(HD32, 300, 6, regimes=(0,), threads=16)
    compare(HD256, 30, 8, regimes=(0,), arch="qwen2", qkv_bias=True)


def test_e2e_walk_row_bounds():
    compare(WALK_LO, 5, 9, regimes=(0,))
    compare(WALK_HI, 5, 9, regimes=(0,), threads=16)


def test_e2e_qwen2_neox_bias_tied_head():
    """The paths a Llama file does not take (forward_quantized.rs:389-445,
    :617-627): qwen2.* metadata (NeoX split-half RoPE, rope base 1e6, eps
    1e-6), q/k/v biases, the tied head (token_embd as the lm_head), and
    general.alignment 8 (tensors off 16 bytes in the file)."""
    cfg = dict(SMALL, rope_theta=1e6, rms_eps=1e-6)
    compare(cfg, 6, 10, arch="qwen2", qkv_bias=True, tied=True, alignment=8)
    compare(MEDIUM, 5, 12, regimes=(0,), arch="qwen2", qkv_bias=True)
    compare(MEDIUM, 3, 9, regimes=(1,), tied=True, qkv_bias=True, alignment=4)


def _errors(m, prompt, n_new, regime=0):
    try:
        m.run(prompt, n_new, b"\0" * 32, regime=regime)
    except Exception as e:  # noqa: BLE001 - both sides' exception types carry code and message
        return (e.code, e.message)
    return None


def test_e2e_errors_mirror_reference():
    import gguf_edit

    cfg = dict(SMALL, vocab=256)
    blob, prompt = synth.e2e_inputs(cfg, 4)
    short, _ = synth.e2e_inputs(cfg, 4, short_rows=4)
    bad_norm = gguf_edit.set_tensor_dims(blob, "blk.1.ffn_norm.weight", [252])
    cases = [
        (blob, prompt, cfg["ctx"], 0, (9, "prompt + n_new_tokens exceeds seq_len")),
        (blob, np.zeros(0, dtype=np.uint32), 4, 0, (9, "prompt_tokens must not be empty")),
        (blob, np.array([3, 256], dtype=np.uint32), 2, 0, (1, "embedding_row Q4_K: row past end of table")),
        # a K projection 4 rows short: refused on the host before any launch
        (short, prompt, 2, 0, (1, "linear_q4_k_integer: weight shape mismatch")),
        (short, prompt, 2, 1, (1, "linear_q4_k_fused: weight shape mismatch")),
        (bad_norm, prompt, 2, 0, (8, "expected weight length == last dim of x, got weight mismatch")),
    ]
    for b, p, n, regime, want in cases:
        gm = runtime.Model(b)
        try:
            assert _errors(gm, p, n, regime) == want
            assert _errors(oracle.Model(b), p, n, regime) == want
            # the model still runs after a refused call
            if b is blob:
                gm.run(prompt, 2, b"\0" * 32)
        finally:
            gm.close()
    with pytest.raises(Exception, match="bad magic"):
        runtime.Model(np.frombuffer(b"GGML" + b"\0" * 60, dtype=np.uint8))
    gm = runtime.Model(blob)
    try:
        import vtq

        for bad in (-1, 2):
            assert runtime.lib().vtqrt_set_prompt_mode(gm.handle, bad) == vtq.E_INVALID_ARGUMENT
        gm.run(prompt, 2, b"\0" * 32)  # the mode in force is unchanged
    finally:
        gm.close()


def test_e2e_config5_full_bit_exact():
    # Llama 1.1B shape, 128 prompt ids, 64 new tokens,
    # integer (std-parallel) regime; logits compared at all 192 steps
    compare(synth.LLAMA_1B1, synth.E2E_PROMPT, synth.E2E_NEW, regimes=(0,), threads=16)


def compare_recorded(cfg, prompt_len, n_new, flags, regime=0):
    blob, prompt = synth.e2e_inputs(cfg, prompt_len)
    wh = bytes.fromhex(oracle.blake3(blob))
    om = oracle.Model(blob)
    gm = runtime.Model(blob)
    try:
        t_o, d_o, ops_o, acts_o = om.run_recorded(prompt, n_new, wh, flags=flags, regime=regime, threads=16)
        t_g, d_g, ops_g, acts_g = gm.run_recorded(prompt, n_new, wh, flags=flags, regime=regime)
    finally:
        gm.close()
    assert len(ops_g) == len(ops_o) and len(acts_g) == len(acts_o)
    for a, b in zip(ops_g, ops_o):
        assert a.key() == b.key(), f"op {b.op_index} ({b.op_name.decode()}, layer {b.layer}) differs"
    for a, b in zip(acts_g, acts_o):
        assert a.key() == b.key(), f"activation {b.act_index} ({b.checkpoint.decode()}, token {b.token_index}) differs"
    assert np.array_equal(t_g, t_o) and d_g == d_o
    return d_o


def test_e2e_per_op_and_activation_receipts():
    compare_recorded(SMALL, 5, 4, runtime.RECORD_OPS | runtime.RECORD_ACTIVATIONS)
    compare_recorded(MEDIUM, 3, 6, runtime.RECORD_OPS, regime=1)
    compare_recorded(MEDIUM, 2, 3, runtime.RECORD_ACTIVATIONS)


def test_e2e_config5_receipts_bit_exact():
    # config 5 with both recorders: 192 steps x 200 op records and 47 checkpoints
    d = compare_recorded(synth.LLAMA_1B1, synth.E2E_PROMPT, synth.E2E_NEW,
                         runtime.RECORD_OPS | runtime.RECORD_ACTIVATIONS)
    assert len(d) == 64
