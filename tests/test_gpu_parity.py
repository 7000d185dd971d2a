"""GPU parity: libvtq (HIP, gfx950) against the pinned CPU oracle, bit for bit.

Every call goes through the C ABI of include/vtq.h.  Small shapes are
compared with the oracle run in-process; the full BASELINE configurations
are compared with the oracle (threaded) and with the committed golden
hashes of tests/golden/golden.json.  Non-finite outputs only need to agree
on being NaN/Inf: IEEE-754 leaves NaN payloads unspecified and the
reference excludes them from its own bit comparisons
(src/ops/quant.rs:2032-2044).
"""
import hashlib
import json
import os

import numpy as np
import pytest

import oracle as O
import vtq
from vtq import synth

pytestmark = pytest.mark.gpu

F = np.float32
GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "golden.json")))
THREADS = min(os.cpu_count() or 1, 16)


def assert_bits_equal(got, want, what=""):
    got = np.asarray(got, F).reshape(-1)
    want = np.asarray(want, F).reshape(-1)
    assert got.shape == want.shape, what
    fin = np.isfinite(want)
    bad = np.nonzero(got[fin].view(np.uint32) != want[fin].view(np.uint32))[0]
    assert bad.size == 0, (
        f"{what}: {bad.size} of {fin.sum()} finite outputs differ; first at {np.nonzero(fin)[0][bad[0]]}: "
        f"gpu {got[fin][bad[0]]!r} ({got[fin].view(np.uint32)[bad[0]]:08x}) vs "
        f"oracle {want[fin][bad[0]]!r} ({want[fin].view(np.uint32)[bad[0]]:08x})")
    assert np.array_equal(np.isnan(got[~fin]), np.isnan(want[~fin])), what
    assert np.array_equal(got[~fin & ~np.isnan(want)], want[~fin & ~np.isnan(want)]), what


def run_gpu(ctx, ggml_type, regime, x, w, batch, in_f, out_f):
    y = np.full(batch * out_f, np.nan, F)
    print(f"[gpu] type={vtq.TYPE_NAMES.get(ggml_type, ggml_type)} regime={regime} batch={batch} "
          f"in={in_f} out={out_f}", flush=True)
    try:
        ctx.linear(ggml_type, regime, x, w, y, batch, in_f, out_f)
    finally:
        # weights are cached by address; test arrays are freed and reused
        ctx.release_weights()
    return y


def pinned_q4k(rows, in_f, seed):
    w = O.lcg_bytes(rows * (in_f // 256) * 144, seed).reshape(-1, 144)
    w[:, 0:2] = np.frombuffer(np.uint16(0x2E66).tobytes(), np.uint8)
    w[:, 2:4] = np.frombuffer(np.uint16(0x2666).tobytes(), np.uint8)
    return w.reshape(-1)


def pinned_q6k(rows, in_f, seed):
    w = O.lcg_bytes(rows * (in_f // 256) * 210, seed).reshape(-1, 210)
    w[:, 208:210] = np.frombuffer(np.uint16(0x2E66).tobytes(), np.uint8)
    return w.reshape(-1)


def check(ctx, ggml_type, regime, x, w, batch, in_f, out_f):
    got = run_gpu(ctx, ggml_type, regime, x, w, batch, in_f, out_f)
    want = O.linear_dispatch(ggml_type, regime, x, w, batch, in_f, out_f, THREADS)
    assert_bits_equal(got, want, f"type {ggml_type} regime {regime} {batch}x{in_f}->{out_f}")
    return got


# ------------------------------------------------------------ k-quant integer

# rows of at most 8 super-blocks (in_feat <= 2048) go two to a wave step: odd row
# counts leave the last pair half empty; batch > 1 runs one grid slice per row
KQ_SHAPES = [(1, 256, 1), (1, 256, 3), (1, 512, 7), (1, 4096, 64), (1, 11008, 17), (3, 4096, 300),
             (1, 2048, 2048), (1, 2048, 256), (1, 5632, 2048), (2, 4096 * 4 + 256, 33), (1, 32768, 9),
             (2, 2048, 7), (3, 1792, 4099)]


@pytest.mark.parametrize("batch,in_f,out_f", KQ_SHAPES)
def test_q4k_integer_synthetic(ctx, batch, in_f, out_f):
    w = synth.weights(vtq.Q4_K, out_f, in_f, seed=in_f * 7 + out_f)
    x = synth.activations(batch * in_f, seed=in_f + batch)
    check(ctx, vtq.Q4_K, 0, x, w, batch, in_f, out_f)


@pytest.mark.parametrize("batch,in_f,out_f", KQ_SHAPES)
def test_q6k_integer_synthetic(ctx, batch, in_f, out_f):
    w = synth.weights(vtq.Q6_K, out_f, in_f, seed=in_f * 11 + out_f)
    x = synth.activations(batch * in_f, seed=in_f + 3 * batch)
    check(ctx, vtq.Q6_K, 0, x, w, batch, in_f, out_f)


# batch >= 32 takes the i8-MFMA prefill GEMM (split-K at these grid sizes)
GEMM_SHAPES = [(32, 256, 32), (33, 512, 1), (64, 4096, 100), (130, 2048, 70), (128, 5632, 64),
               (256, 11008, 40), (40, 256 * 127, 8), (300, 4096, 33)]


@pytest.mark.parametrize("batch,in_f,out_f", GEMM_SHAPES)
def test_q4k_prefill_gemm(ctx, batch, in_f, out_f):
    w = synth.weights(vtq.Q4_K, out_f, in_f, seed=in_f * 31 + out_f)
    x = synth.activations(batch * in_f, seed=in_f * 37 + batch)
    check(ctx, vtq.Q4_K, 0, x, w, batch, in_f, out_f)


# small grids take the split-K GEMM (one 32-row x 32-token tile per
# workgroup, the row's super-blocks cut into fixed_tree subtrees): every row
# length 1..16 (each tree shape of its counter), token counts either side of
# the 32-token tiles, row counts either side of the 32-row tiles
SHORT_ROW_SHAPES = [(32, 256, 129), (64, 512, 1), (33, 768, 129), (65, 1024, 300), (96, 1280, 128), (97, 1536, 513),
             (127, 1792, 31), (128, 2048, 130), (34, 2304, 64), (200, 2560, 257), (70, 2816, 77),
             (160, 3072, 96), (129, 3328, 33), (95, 3584, 200), (63, 3840, 127), (192, 4096, 255)]
# rows of at most 16 super-blocks over more than 1024 tiles take the per-wave
# GEMM with two 32-token tiles per wave: an odd tile count (the last wave's
# second tile repeats the last one), ragged rows, row lengths 1, 3, 4, 11, 16
PW2_SHAPES = [(272, 768, 13312), (300, 256, 13313), (512, 1024, 13000), (257, 16 * 256, 4200),
              (200, 11 * 256, 6000)]
# rows longer than 16 super-blocks where the LDS-operand GEMM launches at
# least 256 workgroups (one per 32 rows x 128 tokens)
LDS_SHAPES = [(129, 17 * 256, 4096), (130, 33 * 256, 4096), (257, 20 * 256, 3000), (160, 70 * 256, 8192)]


# split-K rows longer than 16 super-blocks: each piece size C = 1, 2, 4, 8,
# 16, trees smaller than a piece (R = 17, 33, 65, 97), a row length of one
# whole tree (R = 64), the prompt pass's W2 shape (R = 22, 2048 rows, 128
# tokens)
SK_SHAPES = [(37, 12 * 256, 70), (33, 22 * 256, 2048), (32, 40 * 256, 100), (64, 100 * 256, 33),
             (40, 127 * 256, 40), (95, 17 * 256, 96), (34, 33 * 256, 130), (65, 65 * 256, 64),
             (41, 97 * 256, 31), (100, 64 * 256, 64), (128, 22 * 256, 2048), (130, 43 * 256, 1000)]


def _gemm_form(R, N, M):
    """The form q4k_gemm.hip's gemm_form picks (used to spread the random
    cases below over all three; the check itself is bit-exactness)."""
    if N * R * 144 >= 1 << 31:
        return "lds"
    if R <= 16:
        return "sk" if (N + 31) // 32 * ((M + 31) // 32) <= 1024 else "pw2"
    return "sk" if (N + 31) // 32 * ((M + 127) // 128) < 256 else "lds"


def random_gemm_cases(per_form=7, seed=7):
    rng = np.random.default_rng(seed)
    got = {"sk": [], "pw2": [], "lds": []}
    while any(len(v) < per_form for v in got.values()):
        R = int(rng.choice([1, 2, 3, 5, 8, 11, 16, 17, 22, 33, 43, 64, 100, 127]))
        M, N = int(rng.integers(32, 641)), int(rng.integers(1, 16385))
        if M * R * 256 * N > 3e9:
            continue
        f = _gemm_form(R, N, M)
        if len(got[f]) < per_form:
            got[f].append(pytest.param(M, R * 256, N, id=f"{f}-{M}x{R * 256}x{N}"))
    return [c for v in got.values() for c in v]


# seeded random shapes, seven per GEMM form, up to 3 G multiply-adds each
@pytest.mark.parametrize("batch,in_f,out_f", random_gemm_cases())
def test_q4k_prefill_gemm_random_forms(ctx, batch, in_f, out_f):
    w = synth.weights(vtq.Q4_K, out_f, in_f, seed=in_f * 5 + out_f)
    x = synth.activations(batch * in_f, seed=in_f * 41 + batch)
    check(ctx, vtq.Q4_K, 0, x, w, batch, in_f, out_f)


@pytest.mark.parametrize("batch,in_f,out_f", SK_SHAPES)
def test_q4k_prefill_gemm_split_k_shapes(ctx, batch, in_f, out_f):
    w = synth.weights(vtq.Q4_K, out_f, in_f, seed=in_f * 7 + out_f)
    x = synth.activations(batch * in_f, seed=in_f * 23 + batch)
    check(ctx, vtq.Q4_K, 0, x, w, batch, in_f, out_f)


@pytest.mark.parametrize("batch,in_f,out_f", LDS_SHAPES)
def test_q4k_prefill_gemm_lds_operand_shapes(ctx, batch, in_f, out_f):
    w = synth.weights(vtq.Q4_K, out_f, in_f, seed=in_f * 3 + out_f)
    x = synth.activations(batch * in_f, seed=in_f * 29 + batch)
    check(ctx, vtq.Q4_K, 0, x, w, batch, in_f, out_f)


@pytest.mark.parametrize("batch,in_f,out_f", PW2_SHAPES)
def test_q4k_prefill_gemm_two_tiles_per_wave(ctx, batch, in_f, out_f):
    w = synth.weights(vtq.Q4_K, out_f, in_f, seed=in_f * 11 + out_f)
    x = synth.activations(batch * in_f, seed=in_f * 19 + batch)
    check(ctx, vtq.Q4_K, 0, x, w, batch, in_f, out_f)


@pytest.mark.parametrize("batch,in_f,out_f", SHORT_ROW_SHAPES)
def test_q4k_prefill_gemm_short_row_lengths(ctx, batch, in_f, out_f):
    w = synth.weights(vtq.Q4_K, out_f, in_f, seed=in_f * 13 + out_f)
    x = synth.activations(batch * in_f, seed=in_f * 17 + batch)
    check(ctx, vtq.Q4_K, 0, x, w, batch, in_f, out_f)


def q4k_blocks(rows, in_f, d_bits, dmin_bits, scale_byte, seed):
    """Q4_K blocks with fixed f16 d / dmin and all twelve scale bytes equal
    (0xFF: every sub-block scale and min is 63; 0x00: all 0), random codes."""
    w = O.lcg_bytes(rows * (in_f // 256) * 144, seed).reshape(-1, 144)
    w[:, 0:2] = np.frombuffer(np.uint16(d_bits).tobytes(), np.uint8)
    w[:, 2:4] = np.frombuffer(np.uint16(dmin_bits).tobytes(), np.uint8)
    w[:, 4:16] = scale_byte
    return w.reshape(-1)


def test_q4k_prefill_gemm_min_term_extremes(ctx):
    # the per-wave GEMM forms the min term sum_j m_j * bsum_j on an f16 MFMA:
    # m = 63 with |bsum| = 4064 (every code +-127) gives the largest |accm|
    # (2,048,256), and alternating signs per sub-block give partial sums of
    # both signs
    batch, in_f, out_f = 64, 4096, 64
    x = np.ones((batch, in_f), F)
    x[1::2] = -1.0
    x[2::4] *= np.repeat(np.array([1, -1] * (in_f // 64), F), 32)
    x[3::4] = synth.activations(in_f * (batch // 4), seed=11).reshape(batch // 4, in_f)
    w = q4k_blocks(out_f, in_f, 0x2E66, 0x2666, 0xFF, 0xAB)
    check(ctx, vtq.Q4_K, 0, x.reshape(-1), w, batch, in_f, out_f)


def test_q4k_prefill_gemm_zero_min_sign(ctx):
    # m = 0 against negative bsums makes every min-term product -0.0; the
    # reference's f32(accm = 0) is +0.0, so the sum must come out +0.0.  With
    # sc = 0, d < 0 and dmin > 0 every part is (-0.0) - (+0.0) = -0.0 and the
    # outputs are -0.0; a -0.0 min term would turn them into +0.0.
    batch, in_f, out_f = 64, 2048, 40
    x = -np.abs(synth.activations(batch * in_f, seed=21))
    w = q4k_blocks(out_f, in_f, 0xBC00, 0x3C00, 0x00, 0xCD)  # d = -1.0, dmin = +1.0
    got = check(ctx, vtq.Q4_K, 0, x, w, batch, in_f, out_f)
    assert np.all(got.view(np.uint32) == np.uint32(0x80000000))


# the GEMM walks the batch in launches of 8192 tokens (bounded workspace): one
# token, and one whole 32-token tile, past the first launch
@pytest.mark.parametrize("batch,in_f,out_f", [(8193, 256, 40), (8224, 512, 9)])
def test_q4k_prefill_gemm_batch_chunks(ctx, batch, in_f, out_f):
    x = synth.activations(batch * in_f, seed=batch)
    check(ctx, vtq.Q4_K, 0, x, synth.weights(vtq.Q4_K, out_f, in_f, seed=in_f + out_f), batch, in_f, out_f)


def test_q4k_prefill_gemm_edge_activations(ctx):
    batch, in_f, out_f = 48, 1024, 40
    x = synth.activations(batch * in_f, seed=5).reshape(batch, in_f)
    x[0] = 0.0                     # an all-zero token
    x[1] = -0.0
    x[2, :256] = np.nan
    x[3, 7] = np.inf
    x[4] = (x[4] * F(1e-42)).astype(F)
    x[5] = (x[5] * F(3e37)).astype(F)
    x[6, :64] = np.arange(64, dtype=F) + F(0.5)
    w = synth.weights(vtq.Q4_K, out_f, in_f, seed=77)
    check(ctx, vtq.Q4_K, 0, x.reshape(-1), w, batch, in_f, out_f)
    check(ctx, vtq.Q4_K, 0, x.reshape(-1), pinned_q4k(out_f, in_f, 0xC0FFEE), batch, in_f, out_f)


@pytest.mark.parametrize("in_f,out_f", [(256, 3), (1024, 7), (4096, 31), (14336, 5)])
def test_kquant_random_bytes(ctx, in_f, out_f):
    # the reference's LCG byte blocks with pinned finite scales, ramp activations
    x = O.ramp_x(in_f)
    check(ctx, vtq.Q4_K, 0, x, pinned_q4k(out_f, in_f, 0xC0FFEE), 1, in_f, out_f)
    check(ctx, vtq.Q6_K, 0, x, pinned_q6k(out_f, in_f, 0xBEEF), 1, in_f, out_f)


def test_kquant_unrestricted_bytes(ctx):
    # arbitrary bytes: f16 scales may be Inf/NaN/subnormal; finite outputs must match
    in_f, out_f = 2048, 64
    x = synth.activations(in_f, seed=99)
    check(ctx, vtq.Q4_K, 0, x, synth.random_bytes(out_f * 8 * 144, 5), 1, in_f, out_f)
    check(ctx, vtq.Q6_K, 0, x, synth.random_bytes(out_f * 8 * 210, 6), 1, in_f, out_f)


def test_q4k_prefill_gemm_unrestricted_bytes(ctx):
    # the GEMM's scale decode and f16 conversion on arbitrary block bytes
    batch, in_f, out_f = 40, 2048, 72
    x = synth.activations(batch * in_f, seed=98)
    check(ctx, vtq.Q4_K, 0, x, synth.random_bytes(out_f * 8 * 144, 7), batch, in_f, out_f)


def test_activation_edge_cases(ctx):
    # zero blocks, NaN, +-Inf, subnormals, huge values, exact ties, -0.0
    in_f, out_f = 8 * 256, 40
    x = synth.activations(in_f, seed=3)
    x[0:256] = 0.0
    x[256:512] = -0.0
    x[512] = np.nan
    x[800] = np.inf
    x[1024:1280] = (x[1024:1280] * F(1e-42)).astype(F)  # subnormal block
    x[1280:1536] = (x[1280:1536] * F(3e37)).astype(F)
    x[1536] = 127.0
    x[1537] = F(0.5) - F(2.0 ** -25)
    x[1538:1600] = np.arange(62, dtype=F) + F(0.5)
    for t in (vtq.Q4_K, vtq.Q6_K):
        w = synth.weights(t, out_f, in_f, seed=t)
        check(ctx, t, 0, x, w, 1, in_f, out_f)


# ------------------------------------------------------------- canonical dot

CANON_SHAPES = [(1, 32, 1), (1, 64, 5), (1, 4096, 33), (2, 4096, 100), (1, 8192, 9), (1, 8192 + 32, 9),
                (1, 14336, 17), (1, 11008, 40), (1, 65536, 3), (3, 2048, 70)]


@pytest.mark.parametrize("ggml_type", [vtq.Q8_0, vtq.Q5_0, vtq.Q4_0])
@pytest.mark.parametrize("batch,in_f,out_f", CANON_SHAPES)
def test_canonical_block_formats(ctx, ggml_type, batch, in_f, out_f):
    w = synth.weights(ggml_type, out_f, in_f, seed=in_f * 13 + out_f + ggml_type)
    x = synth.activations(batch * in_f, seed=in_f * 5 + batch)
    check(ctx, ggml_type, 0, x, w, batch, in_f, out_f)


# Q8_0 rows of 256..4096 inputs take the LDS-resident kernel, one template
# instance per 256-element window count; 13 rows leave the second workgroup
# five of its eight rows, batch 2 runs a second grid slice
@pytest.mark.parametrize("nwin", range(1, 17))
@pytest.mark.parametrize("batch,out_f", [(1, 13), (2, 8)])
def test_q8_0_every_window_count(ctx, nwin, batch, out_f):
    in_f = 256 * nwin
    x = synth.activations(batch * in_f, seed=1000 + nwin)
    check(ctx, vtq.Q8_0, 0, x, synth.weights(vtq.Q8_0, out_f, in_f, seed=2000 + nwin), batch, in_f, out_f)


@pytest.mark.parametrize("nwin", [1, 5, 16])
def test_q8_0_arbitrary_bytes(ctx, nwin):
    # any bytes: block scales may be Inf, NaN or subnormal f16 values
    in_f, out_f = 256 * nwin, 11
    w = O.lcg_bytes(out_f * (in_f // 32) * 34, 0xA5A5 + nwin)
    check(ctx, vtq.Q8_0, 0, synth.activations(in_f, seed=3000 + nwin), w, 1, in_f, out_f)


@pytest.mark.parametrize("batch,in_f,out_f", CANON_SHAPES[:8] + [(1, 13, 4), (1, 4100, 7), (2, 8195, 5)])
def test_canonical_f32(ctx, batch, in_f, out_f):
    w = synth.weights(vtq.F32, out_f, in_f, seed=in_f * 17 + out_f, sigma=1.0)
    x = synth.activations(batch * in_f, seed=in_f * 19 + batch)
    check(ctx, vtq.F32, 0, x, w, batch, in_f, out_f)


@pytest.mark.parametrize("batch,in_f,out_f", [(1, 256, 3), (1, 4096, 50), (1, 8192, 3), (1, 14336, 9),
                                              (2, 11008, 20), (1, 65536, 2)])
def test_q4k_float_fused_regime(ctx, batch, in_f, out_f):
    w = synth.weights(vtq.Q4_K, out_f, in_f, seed=in_f * 23 + out_f)
    x = synth.activations(batch * in_f, seed=in_f * 29 + batch)
    check(ctx, vtq.Q4_K, 1, x, w, batch, in_f, out_f)


def test_canonical_reference_vectors(ctx):
    # F32 arm on the reference's LCG pair: must land on the pinned bits.
    for n, want in ((4096, 0x40CE39E1), (14336, 0xC1A3BF11)):
        a, b = O.lcg_pair(n)
        y = run_gpu(ctx, vtq.F32, 0, a, b.view(np.uint8), 1, n, 1)
        assert int(y.view(np.uint32)[0]) == want


# -------------------------------------------------------- full configurations


@pytest.mark.parametrize("name", ["q8_0_4096x4096", "q4k_11008x4096", "q4k_4096x11008", "q6k_32000x4096",
                                  "q4k_gemm_14336x4096_m512"])
def test_full_config_bit_exact(ctx, name):
    cfg = synth.CONFIGS[name]
    g = GOLDEN["configs"][name]
    x, w = cfg.make()
    assert hashlib.sha256(w.tobytes()).hexdigest() == g["w_sha256"], "generator drift (weights)"
    assert hashlib.sha256(x.tobytes()).hexdigest() == g["x_sha256"], "generator drift (activations)"
    got = run_gpu(ctx, cfg.ggml_type, 0, x, w, cfg.batch, cfg.in_feat, cfg.out_feat)
    want = O.linear_dispatch(cfg.ggml_type, 0, x, w, cfg.batch, cfg.in_feat, cfg.out_feat, THREADS)
    assert_bits_equal(got, want, name)
    assert hashlib.sha256(got.tobytes()).hexdigest() == g["y_sha256"]


def test_determinism_repeat_calls(ctx):
    cfg = synth.CONFIGS["q4k_4096x11008"]
    x, w = cfg.make()
    a = run_gpu(ctx, cfg.ggml_type, 0, x, w, 1, cfg.in_feat, cfg.out_feat)
    for _ in range(3):
        b = run_gpu(ctx, cfg.ggml_type, 0, x, w, 1, cfg.in_feat, cfg.out_feat)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


# ------------------------------------------------------- edges and errors


def test_empty_and_degenerate_shapes(ctx):
    y = np.full(3, np.nan, F)
    ctx.linear(vtq.Q4_K, 0, np.zeros(0, F), np.zeros(0, np.uint8), y, 1, 0, 3)
    assert y.tolist() == [0.0, 0.0, 0.0] and not np.signbit(y).any()
    y = np.full(4, 7.0, F)
    ctx.linear(vtq.Q6_K, 0, np.zeros(0, F), np.zeros(4 * 210, np.uint8), y, 0, 256, 4)
    assert y.tolist() == [7.0] * 4  # batch 0 writes nothing
    # the weight-shape check does not depend on batch (src/ops/quant.rs:1071-1074)
    with pytest.raises(vtq.Internal, match="linear_q6_k_integer: weight shape mismatch"):
        ctx.linear(vtq.Q6_K, 0, np.zeros(0, F), np.zeros(0, np.uint8), y, 0, 256, 4)
    ctx.linear(vtq.Q8_0, 0, np.zeros(64, F), np.zeros(0, np.uint8), np.zeros(1, F), 1, 64, 0)


def test_errors_mirror_reference(ctx):
    y = np.zeros(4, F)
    with pytest.raises(vtq.Internal, match="linear_q4_k_integer: in_feat not a multiple of 256"):
        ctx.linear_q4_k_integer(np.zeros(100, F), np.zeros(144, np.uint8), y, 1, 100, 1)
    with pytest.raises(vtq.Internal, match="linear_q4_k_integer: weight shape mismatch"):
        ctx.linear_q4_k_integer(np.zeros(256, F), np.zeros(143, np.uint8), y, 1, 256, 1)
    with pytest.raises(vtq.Internal, match="linear_q6_k_integer_parallel: weight shape"):
        ctx.linear(vtq.Q6_K, 0, np.zeros(256, F), np.zeros(100, np.uint8), np.zeros(600, F), 1, 256, 600)
    with pytest.raises(vtq.NotImplementedDtype, match="weight dtype not"):
        ctx.linear(vtq.F16, 0, np.zeros(32, F), np.zeros(64, np.uint8), y, 1, 32, 1)
    with pytest.raises(vtq.Internal, match="linear_q4_0: x size mismatch"):
        ctx.linear_q4_0(np.zeros(31, F), np.zeros(18, np.uint8), np.zeros(1, F), 1, 32, 1)
    with pytest.raises(vtq.Internal, match="x shorter"):
        ctx.linear_q4_k_integer(np.zeros(255, F), np.zeros(144, np.uint8), y, 1, 256, 1)
    # the context stays usable after errors
    test_q4k_integer_synthetic(ctx, 1, 256, 3)


# Rows longer than the kernels hold (k-quant: 32768 inputs, the canonical dot:
# 65536) run as aligned segments whose sums fixed_tree combines: one to five
# segments, a last segment of one block or one chunk, batch rows gathered or
# strided, and the GEMM batch size (>= 32) on rows too long for the GEMM.
LONG_KQ = [(1, 49152, 5), (2, 32768 + 256, 7), (3, 65536 + 2048, 4), (1, 131072 + 4096, 3), (40, 40960, 3)]
LONG_CANON = [(vtq.Q8_0, 0, 1, 65536 + 32, 3), (vtq.Q8_0, 0, 2, 2 * 65536 + 8192 + 32, 5),
              (vtq.Q5_0, 0, 1, 73728, 3), (vtq.Q4_0, 0, 2, 73728, 2), (vtq.F32, 0, 1, 65536 + 7, 3),
              (vtq.F32, 0, 2, 131073, 2), (vtq.Q4_K, 1, 1, 65536 + 256, 3), (vtq.Q4_K, 1, 2, 98304, 2)]


@pytest.mark.parametrize("batch,in_f,out_f", LONG_KQ)
@pytest.mark.parametrize("ggml_type", [vtq.Q4_K, vtq.Q6_K])
def test_kquant_long_rows_segmented(ctx, ggml_type, batch, in_f, out_f):
    w = synth.weights(ggml_type, out_f, in_f, seed=in_f + 5 * out_f + ggml_type)
    x = synth.activations(batch * in_f, seed=in_f * 3 + batch)
    check(ctx, ggml_type, 0, x, w, batch, in_f, out_f)


@pytest.mark.parametrize("ggml_type,regime,batch,in_f,out_f", LONG_CANON)
def test_canonical_long_rows_segmented(ctx, ggml_type, regime, batch, in_f, out_f):
    w = synth.weights(ggml_type, out_f, in_f, seed=in_f + 7 * out_f + ggml_type)
    x = synth.activations(batch * in_f, seed=in_f * 5 + batch)
    check(ctx, ggml_type, regime, x, w, batch, in_f, out_f)


def test_weight_cache_rekeys_on_length_and_release(ctx):
    in_f, out_f = 512, 8
    w = synth.weights(vtq.Q4_K, out_f, in_f, seed=1)
    x = synth.activations(in_f, seed=2)
    y = np.zeros(out_f, F)
    ctx.linear(vtq.Q4_K, 0, x, w, y, 1, in_f, out_f)
    a = y.copy()
    w[:] = synth.weights(vtq.Q4_K, out_f, in_f, seed=3)
    ctx.linear(vtq.Q4_K, 0, x, w, y, 1, in_f, out_f)
    assert np.array_equal(y.view(np.uint32), a.view(np.uint32)), "same key: cached bytes must be reused"
    ctx.release_weights(w)
    ctx.linear(vtq.Q4_K, 0, x, w, y, 1, in_f, out_f)
    assert_bits_equal(y, O.linear_dispatch(vtq.Q4_K, 0, x, w, 1, in_f, out_f), "after release")
    ctx.linear(vtq.Q4_K, 0, x, w[: w.size // 2], y[: out_f // 2], 1, in_f, out_f // 2)  # new length: new key
    ctx.release_weights()


def test_device_pointer_entry_matches_host(ctx):
    import torch

    cfg = synth.CONFIGS["q4k_11008x4096"]
    x, w = cfg.make(rows=1000)
    dx = torch.from_numpy(x).cuda()
    dw = torch.from_numpy(w).cuda()
    dy = torch.full((1000,), float("nan"), device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    ctx.linear_device(vtq.Q4_K, 0, dx.data_ptr(), dw.data_ptr(), w.size, dy.data_ptr(), 1, cfg.in_feat, 1000, stream)
    torch.cuda.synchronize()
    want = O.linear_dispatch(vtq.Q4_K, 0, x, w, 1, cfg.in_feat, 1000, THREADS)
    assert_bits_equal(dy.cpu().numpy(), want, "device entry")
