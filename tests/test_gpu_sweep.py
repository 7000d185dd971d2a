"""GPU parity over a seeded sweep of shapes (every dtype and regime).

The fixed-shape tests pin each kernel at the configurations it was built
for; this sweep draws shapes around every switch point the dispatch and the
kernels have: k-quant rows of one, two and three 16-block windows and the
windows kernel beyond them, rows of at most 8 super-blocks paired in a wave
step, batches either side of the prefill GEMM's 32-token threshold and of its
32-token tiles, row counts either side of the reference's PAR_MIN_ROWS = 512,
and canonical-dot lengths that are not multiples of the 8-lane chunking.
Every case is compared bit for bit with the oracle (tests/test_gpu_parity.py's
rule for non-finite outputs).
"""
import numpy as np
import pytest

import oracle as O
import vtq
from vtq import synth

from test_gpu_parity import THREADS, assert_bits_equal

pytestmark = pytest.mark.gpu

KQ_IN = [256 * k for k in (1, 2, 7, 8, 9, 15, 16, 17, 31, 32, 33, 43, 47, 48, 49, 64, 127, 128)]
CANON_IN = [32, 64, 224, 256, 288, 992, 1024, 4064, 4096, 4128, 8192, 8224, 16416]
F32_IN = [1, 5, 8, 13, 255, 256, 1000, 4097, 8191, 8200]
BATCH = [1, 2, 5, 31, 32, 33, 47, 64, 70]
OUT = [1, 2, 3, 17, 255, 256, 511, 512, 513, 700]
MAX_MACS = 24_000_000  # keeps the oracle leg of each case well under a second


# the switch points themselves, then a seeded draw around them
EDGES = [
    (vtq.Q4_K, 0, 32, 256, 33), (vtq.Q4_K, 0, 33, 2048, 64), (vtq.Q4_K, 0, 31, 4096, 65),
    (vtq.Q4_K, 0, 64, 11008, 17), (vtq.Q4_K, 0, 40, 12288, 3), (vtq.Q4_K, 0, 1, 12544, 40),
    (vtq.Q4_K, 0, 1, 2048, 511), (vtq.Q4_K, 0, 1, 2048, 513), (vtq.Q4_K, 1, 1, 4096, 512),
    (vtq.Q6_K, 0, 1, 8192, 5), (vtq.Q6_K, 0, 1, 8448, 5), (vtq.Q6_K, 0, 33, 2048, 9),
    (vtq.Q8_0, 0, 1, 8224, 9), (vtq.Q5_0, 0, 3, 16416, 4), (vtq.Q4_0, 0, 2, 32, 513),
]


def cases(n=192, seed=20261202):
    rng = np.random.default_rng(seed)
    out = [c + (1000 + i,) for i, c in enumerate(EDGES)]
    n += len(out)
    kinds = [(vtq.Q4_K, 0), (vtq.Q4_K, 1), (vtq.Q6_K, 0), (vtq.Q8_0, 0), (vtq.Q5_0, 0), (vtq.Q4_0, 0), (vtq.F32, 0)]
    while len(out) < n:
        t, regime = kinds[len(out) % len(kinds)]
        ins = KQ_IN if t in (vtq.Q4_K, vtq.Q6_K) else F32_IN if t == vtq.F32 else CANON_IN
        in_f = int(rng.choice(ins))
        batch = int(rng.choice(BATCH))
        out_f = int(rng.choice(OUT))
        if batch * in_f * out_f > MAX_MACS:
            continue
        out.append((t, regime, batch, in_f, out_f, int(rng.integers(1, 1 << 30))))
    return out


@pytest.mark.parametrize("t,regime,batch,in_f,out_f,seed", cases())
def test_sweep_bit_exact(ctx, t, regime, batch, in_f, out_f, seed):
    w = synth.weights(t, out_f, in_f, seed, sigma=1.0) if t == vtq.F32 else synth.weights(t, out_f, in_f, seed)
    x = synth.activations(batch * in_f, seed + 1)
    y = np.full(batch * out_f, np.nan, np.float32)
    print(f"[gpu] sweep type={vtq.TYPE_NAMES[t]} regime={regime} batch={batch} in={in_f} out={out_f} seed={seed}",
          flush=True)
    try:
        ctx.linear(t, regime, x, w, y, batch, in_f, out_f)
    finally:
        ctx.release_weights()
    want = O.linear_dispatch(t, regime, x, w, batch, in_f, out_f, THREADS)
    assert_bits_equal(y, want, f"{vtq.TYPE_NAMES[t]} regime {regime} {batch}x{in_f}->{out_f}")
