"""Seeded random model shapes through the runtime vs the CPU oracle.

Each case draws a small Llama- or Qwen2-shaped model (head dims 32, 64 and
128, KV groups of 1 to 8 heads, one or two layers, hidden and vocab sizes
off the powers of two), a prompt of 2-200 ids and a few new tokens, and
compares the logits of every position, the tokens and both receipt digests
with the oracle's run_quantized restatement (src/model/inference.rs:274-345),
with the prompt batched and stepped.  The shapes reach the prefill GEMM's
split-K, per-wave and LDS-operand forms, the prompt pass's attention with
every workgroup size and several row tiles, and the residual adds folded
into the norms.
"""
import numpy as np
import pytest

import oracle
from vtq import runtime, synth

pytestmark = pytest.mark.gpu


def cases(n=30, seed=20261202):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        hd = int(rng.choice([32, 64, 128]))
        heads = int(rng.choice([h for h in (2, 4, 6, 8, 12, 16, 24, 32) if (h * hd) % 256 == 0 and h * hd <= 2048]))
        kv = int(rng.choice([k for k in range(1, heads + 1) if heads % k == 0 and heads // k <= 8]))
        dim = heads * hd
        P = int(rng.integers(2, 201)) if dim <= 1024 else int(rng.integers(2, 64))
        n_new = int(rng.integers(2, 9))
        cfg = dict(dim=dim, hidden=int(rng.choice([256, 512, 768, 1280, 1536])), layers=int(rng.integers(1, 3)),
                   heads=heads, kv_heads=kv, vocab=int(rng.integers(300, 3001)),
                   ctx=P + n_new + int(rng.integers(0, 40)), rope_theta=float(rng.choice([10000.0, 1e6])),
                   rms_eps=float(rng.choice([1e-5, 1e-6])))
        qwen = bool(rng.integers(0, 2))
        variant = dict(arch="qwen2" if qwen else "llama", qkv_bias=qwen and bool(rng.integers(0, 2)),
                       tied=bool(rng.integers(0, 2)))
        out.append((cfg, P, n_new, variant, int(rng.integers(1, 1 << 30))))
    return out


@pytest.mark.parametrize("cfg,P,n_new,variant,seed", cases())
def test_e2e_random_shapes(cfg, P, n_new, variant, seed):
    print(f"[gpu] e2e sweep {cfg} P={P} new={n_new} {variant} seed={seed}", flush=True)
    blob = synth.llama_gguf(cfg, seed, **variant)
    prompt = synth.tokens(seed + 1, P, cfg["vocab"])
    wh_o = bytes.fromhex(oracle.blake3(blob))
    wh_p = runtime.blake3(blob)
    assert wh_o == wh_p
    om = oracle.Model(blob)
    gm = runtime.Model(blob)
    try:
        t_o, d_o, l_o = om.run(prompt, n_new, wh_o, regime=0, threads=16)
        for stepwise in (False, True):
            mode = "stepwise" if stepwise else "batched"
            t_g, d_g, l_g = gm.run(prompt, n_new, wh_p, regime=0, stepwise=stepwise)
            assert l_g.shape == l_o.shape
            bad = np.nonzero((l_g.view(np.uint32) != l_o.view(np.uint32)).any(axis=1))[0]
            assert bad.size == 0, f"{mode}: logits differ first at position {bad[0]}"
            assert np.array_equal(t_g, t_o), f"{mode}: tokens {t_g} vs {t_o}"
            assert d_g == d_o, f"{mode}: digest"
            assert gm.digest_v1 == om.digest_v1
    finally:
        gm.close()
