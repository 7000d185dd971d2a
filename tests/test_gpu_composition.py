"""The GPU decode step's composition, pinned on degenerate models.

The same reductions as tests/test_decode_composition.py (which holds the
oracle to them), now against libvtq_runtime on the GPU: the expected logits
and tokens are composed on the CPU from independently pinned parts
(tests/decode_compose.py), not taken from the oracle's run.  The
zero-output-projection model and the first step are also checked at the
1.1B config-5 shape (22 layers, GQA 32/4, dim 2048, FFN 5632, Q6_K head),
where the fused decode kernels run their production paths.
"""
import numpy as np
import pytest

import decode_compose as C
from test_decode_composition import IDS, NORM_DIMS, VARIANTS, WH, adversarial_model, bits
from vtq import runtime, synth

pytestmark = pytest.mark.gpu

THREADS = 16


def run_gpu(blob, prompt, n_new):
    m = runtime.Model(blob)
    try:
        toks, _, logits = m.run(prompt, n_new, WH)
    finally:
        m.close()
    return toks, logits


@pytest.mark.parametrize("cfg,variant", VARIANTS, ids=IDS)
def test_gpu_zero_output_projections(cfg, variant):
    blob, prompt = synth.e2e_inputs(cfg, 6, **variant)
    blob = C.zero_out_model(blob, cfg["layers"])
    print(f"[gpu] composition zero_out {cfg['dim']}x{cfg['layers']} {variant}", flush=True)
    toks, logits = run_gpu(blob, prompt, 5)
    want_toks, want_logits = C.zero_out_run(C.Weights(blob, cfg, THREADS), prompt, 5)
    assert np.array_equal(bits(logits), bits(want_logits))
    assert np.array_equal(toks, want_toks)


@pytest.mark.parametrize("cfg,variant", VARIANTS, ids=IDS)
def test_gpu_first_step(cfg, variant):
    blob, prompt = synth.e2e_inputs(cfg, 3, **variant)
    print(f"[gpu] composition step0 {cfg['dim']}x{cfg['layers']} {variant}", flush=True)
    _, logits = run_gpu(blob, prompt, 1)
    want = C.step0_logits(C.Weights(blob, cfg, THREADS), int(prompt[0]))
    assert np.array_equal(bits(logits[0]), bits(want))


@pytest.mark.parametrize("cfg,variant", VARIANTS[:3], ids=IDS[:3])
def test_gpu_zero_query_weights(cfg, variant):
    blob, prompt = synth.e2e_inputs(cfg, 5, **variant)
    blob = C.zero_q_model(blob, cfg["layers"])
    print(f"[gpu] composition zero_q {cfg['dim']}x{cfg['layers']} {variant}", flush=True)
    toks, logits = run_gpu(blob, prompt, 4)
    want_toks, want_logits = C.zero_q_run(C.Weights(blob, cfg, THREADS), prompt, 4)
    assert np.array_equal(bits(logits), bits(want_logits))
    assert np.array_equal(toks, want_toks)


def test_gpu_config5_shape_zero_output_projections():
    # config 5's model and token counts (128 prompt ids, 64 new tokens) with
    # every attn_output and ffn_down weight zero: every step's logits are
    # head(rms_norm(embedding_row(token))), the token loop at full length
    cfg = synth.LLAMA_1B1
    blob, prompt = synth.e2e_inputs()
    blob = C.zero_out_model(blob, cfg["layers"])
    print("[gpu] composition zero_out config-5 shape", flush=True)
    toks, logits = run_gpu(blob, prompt, synth.E2E_NEW)
    want_toks, want_logits = C.zero_out_run(C.Weights(blob, cfg, THREADS), prompt, synth.E2E_NEW)
    assert np.array_equal(bits(logits), bits(want_logits))
    assert np.array_equal(toks, want_toks)


def test_gpu_config5_shape_first_step():
    cfg = synth.LLAMA_1B1
    blob, prompt = synth.e2e_inputs(cfg, 2)
    print("[gpu] composition step0 config-5 shape", flush=True)
    _, logits = run_gpu(blob, prompt, 1)
    want = C.step0_logits(C.Weights(blob, cfg, THREADS), int(prompt[0]))
    assert np.array_equal(bits(logits[0]), bits(want))


@pytest.mark.parametrize("zero_wo", [False, True], ids=["full", "zero-wo"])
@pytest.mark.parametrize("cfg", NORM_DIMS, ids=[f"dim{c['dim']}" for c in NORM_DIMS])
def test_gpu_first_step_on_adversarial_rows(cfg, zero_wo):
    # the fused normalising GEMVs on rows of ties, short mantissas, huge
    # values, outliers, NaN, Inf and zeros: the QKV GEMV's norm prologue sees
    # the embedding row, and with attn_output zero so does the W1/W3 SwiGLU
    # kernel's; dims 1024-4096 take the binade walk, 2560 its longer head
    blob = adversarial_model(cfg, zero_wo)
    w = C.Weights(blob, cfg, THREADS)
    m = runtime.Model(blob)
    try:
        for tok in range(1, 1 + len(C.ADVERSARIAL_KINDS)):
            kind = C.ADVERSARIAL_KINDS[tok - 1]
            print(f"[gpu] adversarial norm row {kind} dim {cfg['dim']} zero_wo={zero_wo}", flush=True)
            _, _, logits = m.run(np.array([tok, 0], np.uint32), 1, WH)
            assert C.bits_equal_nan(logits[0], C.step0_logits(w, tok)), kind
    finally:
        m.close()
