"""The decode step's composition, pinned on degenerate models (oracle, CPU).

tests/decode_compose.py reduces run_quantized on three kinds of model to
parts the oracle pins one by one (see its docstring).  Here the oracle's own
run_quantized (oracle/vtq_oracle_e2e.c) must agree with those reductions
bit for bit: logits at every step and the returned tokens.  The GPU runtime
is held to the same reductions in tests/test_gpu_composition.py.
"""
import numpy as np
import pytest

import decode_compose as C
import gguf_edit as G
import oracle as O
from vtq import synth

SMALL = dict(dim=256, hidden=512, layers=2, heads=4, kv_heads=2, vocab=1000, ctx=32, rope_theta=10000.0,
             rms_eps=1e-5)
GQA4 = dict(dim=512, hidden=768, layers=2, heads=8, kv_heads=2, vocab=700, ctx=32, rope_theta=500000.0,
            rms_eps=1e-6)
VARIANTS = [(SMALL, {}), (GQA4, {}), (SMALL, {"arch": "qwen2", "qkv_bias": True}), (GQA4, {"tied": True})]
IDS = ["llama", "llama-gqa4", "qwen2-bias", "llama-gqa4-tied"]
WH = bytes(32)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def run_oracle(blob, prompt, n_new):
    toks, _, logits = O.Model(blob).run(prompt, n_new, WH, threads=8)
    return toks, logits


@pytest.mark.parametrize("cfg,variant", VARIANTS, ids=IDS)
def test_zero_output_projections_reduce_to_embedding_head(cfg, variant):
    blob, prompt = synth.e2e_inputs(cfg, 6, **variant)
    blob = C.zero_out_model(blob, cfg["layers"])
    toks, logits = run_oracle(blob, prompt, 5)
    want_toks, want_logits = C.zero_out_run(C.Weights(blob, cfg), prompt, 5)
    assert np.array_equal(bits(logits), bits(want_logits))
    assert np.array_equal(toks, want_toks)


@pytest.mark.parametrize("cfg,variant", VARIANTS, ids=IDS)
def test_first_step_reduces_to_value_passthrough(cfg, variant):
    blob, prompt = synth.e2e_inputs(cfg, 3, **variant)
    _, logits = run_oracle(blob, prompt, 1)
    want = C.step0_logits(C.Weights(blob, cfg), int(prompt[0]))
    assert np.array_equal(bits(logits[0]), bits(want))


@pytest.mark.parametrize("cfg,variant", VARIANTS[:3], ids=IDS[:3])
def test_zero_query_weights_reduce_to_uniform_attention(cfg, variant):
    blob, prompt = synth.e2e_inputs(cfg, 5, **variant)
    blob = C.zero_q_model(blob, cfg["layers"])
    toks, logits = run_oracle(blob, prompt, 4)
    want_toks, want_logits = C.zero_q_run(C.Weights(blob, cfg), prompt, 4)
    assert np.array_equal(bits(logits), bits(want_logits))
    assert np.array_equal(toks, want_toks)


def test_reductions_are_not_vacuous():
    # the reductions must distinguish: a model whose token loop fed the
    # picked token back one step late, or whose attention ignored the cache,
    # would produce other logits (checked on the composition itself)
    blob, prompt = synth.e2e_inputs(SMALL, 5)
    w = C.Weights(C.zero_q_model(blob, SMALL["layers"]), SMALL)
    _, lg = C.zero_q_run(w, prompt, 2)
    assert not np.array_equal(bits(lg[1]), bits(C.step0_logits(w, int(prompt[1]))))
    wz = C.Weights(C.zero_out_model(blob, SMALL["layers"]), SMALL)
    toks, lz = C.zero_out_run(wz, prompt, 3)
    assert len(set(map(int, toks))) > 1 or not np.array_equal(bits(lz[-1]), bits(lz[-2]))


NORM_DIMS = [dict(dim=d, hidden=768, layers=1, heads=d // 64, kv_heads=d // 256, vocab=300, ctx=8,
                  rope_theta=10000.0, rms_eps=1e-5) for d in (1024, 2048, 2560, 4096)]


def adversarial_model(cfg, zero_wo):
    blob, _ = synth.e2e_inputs(cfg, 2)
    rng = np.random.default_rng(cfg["dim"])
    rows = {1 + i: C.adversarial_row(k, cfg["dim"], rng) for i, k in enumerate(C.ADVERSARIAL_KINDS)}
    blob = C.with_embedding_rows(blob, cfg["dim"], rows)
    if zero_wo:  # the FFN's norm then sees the embedding row itself
        blob = G.zero_tensors(blob, [f"blk.{l}.attn_output.weight" for l in range(cfg["layers"])])
    return blob


@pytest.mark.parametrize("zero_wo", [False, True], ids=["full", "zero-wo"])
@pytest.mark.parametrize("cfg", NORM_DIMS, ids=[f"dim{c['dim']}" for c in NORM_DIMS])
def test_first_step_on_adversarial_rows(cfg, zero_wo):
    # the first step's norms on rows of ties, short mantissas, huge values,
    # outliers, NaN, Inf and zeros (embedding rows of crafted Q4_K blocks)
    blob = adversarial_model(cfg, zero_wo)
    w = C.Weights(blob, cfg)
    for tok in range(1, 1 + len(C.ADVERSARIAL_KINDS)):
        _, logits = run_oracle(blob, np.array([tok, 0], np.uint32), 1)
        assert C.bits_equal_nan(logits[0], C.step0_logits(w, tok)), C.ADVERSARIAL_KINDS[tok - 1]
