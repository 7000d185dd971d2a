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
