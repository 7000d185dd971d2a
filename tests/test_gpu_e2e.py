"""End-to-end decode on the GPU runtime vs the CPU oracle (config 5).

libvtq_runtime (every linear on the GPU through libvtq) must reproduce the
oracle's restatement of inference::run_quantized (src/model/inference.rs:
274-345) bit for bit: the logits of every decode step, the generated tokens
and the vitnify-receipt v2 digest, in both Q4_K regimes.
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


def compare(cfg, prompt_len, n_new, regimes=(0, 1), threads=8):
    blob, prompt = synth.e2e_inputs(cfg, prompt_len)
    wh_o = bytes.fromhex(oracle.blake3(blob))
    wh_p = runtime.blake3(blob)
    assert wh_o == wh_p
    om = oracle.Model(blob)
    gm = runtime.Model(blob)
    try:
        for regime in regimes:
            t_o, d_o, l_o = om.run(prompt, n_new, wh_o, regime=regime, threads=threads)
            t_g, d_g, l_g = gm.run(prompt, n_new, wh_p, regime=regime)
            assert l_g.shape == l_o.shape
            bad = np.nonzero((l_g.view(np.uint32) != l_o.view(np.uint32)).any(axis=1))[0]
            assert bad.size == 0, f"regime {regime}: logits differ first at step {bad[0]}"
            assert np.array_equal(t_g, t_o), f"regime {regime}: tokens {t_g} vs {t_o}"
            assert d_g == d_o, f"regime {regime}: digest {d_g} vs {d_o}"
    finally:
        gm.close()
    return d_o


def test_e2e_small_both_regimes():
    compare(SMALL, 8, 8)


def test_e2e_medium_odd_lengths():
    # kv heads < heads (GQA), prompt of 1, long generation
    compare(MEDIUM, 1, 40, regimes=(0,))
    compare(MEDIUM, 13, 29, regimes=(1,))


def test_e2e_wide_long_context():
    compare(WIDE, 250, 12, regimes=(0,), threads=16)


def test_e2e_errors_mirror_reference():
    blob, prompt = synth.e2e_inputs(SMALL, 4)
    gm = runtime.Model(blob)
    try:
        with pytest.raises(Exception, match="exceeds seq_len"):
            gm.run(prompt, SMALL["ctx"], b"\0" * 32)
        with pytest.raises(Exception, match="must not be empty"):
            gm.run(np.zeros(0, dtype=np.uint32), 4, b"\0" * 32)
    finally:
        gm.close()
    with pytest.raises(Exception, match="bad magic"):
        runtime.Model(np.frombuffer(b"GGML" + b"\0" * 60, dtype=np.uint8))


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
