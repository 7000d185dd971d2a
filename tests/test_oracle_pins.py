"""Pins of the CPU oracle against the reference's own constants and tests.

The oracle (oracle/vtq_oracle.c) restates src/ops/quant.rs in C.  The Rust
reference cannot be built here (no Rust toolchain), so each check below is
either one of the reference's own tests with its published constant, or a
property that mathematics fixes (closed forms, exhaustive enumeration,
brute force with exact integers), chosen so that a plausible transcription
mistake -- a dropped term, a wrong index, a transposed operand, a different
tree shape -- fails at least one of them.
"""
import numpy as np
import pytest

import oracle as O

F = np.float32


def bits(v) -> int:
    return int(np.asarray(v, dtype=np.float32).view(np.uint32))


# ------------------------------------------------------------------ pinned constants


def test_canonical_dot_reference_bits_pinned():
    # src/ops/quant.rs:1571, :1992-2005
    a, b = O.lcg_pair(4096)
    assert bits(O.canonical_dot(a, b)) == 0x40CE39E1


def test_canonical_dot_discriminating_reference_pinned():
    # src/ops/quant.rs:1974-1990 and :1943-1963
    a, b = O.lcg_pair(14336)
    v = O.canonical_dot(a, b)
    assert bits(v) == 0xC1A3BF11
    r2 = O.canonical_dot_regime2(a, b)
    assert bits(r2) != bits(v) and abs(float(r2) - float(v)) < 1e-2
    a, b = O.lcg_pair(4096)
    assert bits(O.canonical_dot_regime2(a, b)) == bits(O.canonical_dot(a, b))


def test_matmul_reduction_hash_pinned():
    # src/ops/matmul.rs:135, :158-196: FNV-1a over the f32 bits of 4x64 @ 64x4
    m, k, n = 4, 64, 4
    a, b = O.lcg_pair(256)  # one stream: a = first m*k draws, b = next k*n draws
    out = O.matmul_f32(a, b, m, k, n)
    h = 0xCBF29CE484222325
    for byte in out.astype(np.float32).tobytes():
        h ^= byte
        h = (h * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    assert h == 0x8A428433686D13AF


def test_matmul_known_answers():
    # src/ops/matmul.rs:198-240
    eye = O.matmul_f32(np.array([1, 2, 3, 4], F), np.array([1, 0, 0, 1], F), 2, 2, 2)
    assert eye.tolist() == [1.0, 2.0, 3.0, 4.0]
    c = O.matmul_f32(np.arange(1, 7, dtype=F), np.arange(7, 13, dtype=F), 2, 3, 2)
    assert c.tolist() == [58.0, 64.0, 139.0, 154.0]


# ------------------------------------------------------- canonical dot structure


def spec_canonical(a, b):
    """Literal transcription of the v2 spec (src/ops/quant.rs:1904-1918), numpy float32 scalars."""
    n = a.size
    sums = []
    for s in range(0, n, 8192):
        lanes = [F(0.0)] * 8
        for i in range(s, min(s + 8192, n)):
            lanes[(i - s) % 8] = F(lanes[(i - s) % 8] + F(a[i] * b[i]))
        sums.append(literal_tree(np.array(lanes, F)))
    return literal_tree(np.array(sums, F)) if sums else F(0.0)


def literal_tree(p):
    """fixed_tree by whole-level halving (src/ops/quant.rs:461-476), vectorised."""
    p = np.array(p, dtype=F)
    if p.size == 0:
        return F(0.0)
    while p.size > 1:
        even, odd = p[0::2], p[1::2]
        nxt = even.copy()
        nxt[: odd.size] = even[: odd.size] + odd
        p = nxt
    return p[0]


def stride_tree(p):
    """Stride form used by the GPU kernels: at stride s, slot i (multiple of 2s) += slot i+s."""
    p = np.array(p, dtype=F)
    n = p.size
    if n == 0:
        return F(0.0)
    s = 1
    while s < n:
        idx = np.arange(0, n - s, 2 * s)
        p[idx] = p[idx] + p[idx + s]
        s *= 2
    return p[0]


def window_tree(p, w):
    """fixed_tree over aligned windows of w (a power of two), each reduced by fixed_tree."""
    p = np.array(p, dtype=F)
    if p.size == 0:
        return F(0.0)
    return literal_tree(np.array([literal_tree(p[i:i + w]) for i in range(0, p.size, w)], F))


def binary_fold(p):
    """Streaming form: balanced sums over the binary digits of n, folded right to left."""
    p = np.array(p, dtype=F)
    n = p.size
    if n == 0:
        return F(0.0)
    blocks, start = [], 0
    for e in reversed(range(n.bit_length())):
        if n >> e & 1:
            blocks.append(literal_tree(p[start:start + (1 << e)]))
            start += 1 << e
    acc = blocks[-1]
    for blk in reversed(blocks[:-1]):
        acc = F(blk + acc)
    return acc


def test_fixed_tree_forms_agree_exhaustively():
    rng = np.random.default_rng(1234)
    for n in range(0, 1100):
        # wide dynamic range so that any different pairing changes the rounding
        p = (rng.standard_normal(n) * np.exp2(rng.integers(-20, 20, n))).astype(F)
        want = bits(O.fixed_tree(p))
        assert bits(literal_tree(p)) == want, n
        assert bits(stride_tree(p)) == want, n
        assert bits(window_tree(p, 16)) == want, n
        assert bits(window_tree(p, 8)) == want, n
        assert bits(binary_fold(p)) == want, n
    for n in (2048, 3000, 4095, 4096):
        p = (rng.standard_normal(n) * np.exp2(rng.integers(-20, 20, n))).astype(F)
        want = bits(O.fixed_tree(p))
        assert bits(literal_tree(p)) == want and bits(stride_tree(p)) == want


def test_negative_zero_is_tree_identity():
    # The GPU trees pad unused slots with -0.0: x + (-0.0) == x bit for bit, also for x = +-0.0.
    for x in (F(0.0), F(-0.0), F(1.5), F(-3e-41), F(np.inf)):
        assert bits(F(x + F(-0.0))) == bits(x)


@pytest.mark.parametrize("n", [1, 7, 8, 9, 63, 64, 65, 4096, 8193])
def test_canonical_matches_spec_transcription(n):
    # src/ops/quant.rs:1899-1929
    a, b = O.lcg_pair(n)
    assert bits(spec_canonical(a, b)) == bits(O.canonical_dot(a, b))


def test_canonical_chunk_completion_order():
    # src/ops/quant.rs:1870-1893
    n = 8192 * 5 + 137
    a, b = O.lcg_pair(n)
    sums = np.zeros((n + 8191) // 8192, F)
    for c in reversed(range(sums.size)):
        s, e = c * 8192, min(c * 8192 + 8192, n)
        sums[c] = O.canonical_chunk(a[s:e], b[s:e])
    assert bits(O.canonical_combine(sums)) == bits(O.canonical_dot(a, b))


def test_canonical_empty_is_zero():
    assert bits(O.canonical_dot(np.zeros(0, F), np.zeros(0, F))) == 0


# ------------------------------------------------------------------------- f16


def test_f16_decode_exhaustive():
    codes = np.arange(65536, dtype=np.uint32)
    ref = codes.astype(np.uint16).view(np.float16).astype(np.float32)
    got = np.array([O.f16_to_f32_bits(int(c)) for c in codes], dtype=np.uint32).view(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    # NaN: payload shifted, not quieted (src/ops/quant.rs:59-61)
    c = codes[nan]
    want = ((c >> 15) << 31) | 0x7F800000 | ((c & 0x3FF) << 13)
    assert np.array_equal(got[nan].view(np.uint32), want.astype(np.uint32))


def test_f16_known_constants():
    # src/ops/quant.rs:1677-1692
    for v, h in ((1.0, 0x3C00), (-2.0, 0xC000), (0.5, 0x3800), (0.0, 0x0000)):
        assert O.f32_to_f16(v) == h
        assert float(O.f16_to_f32(h)) == v


# ------------------------------------------------------------- decoders (KATs)


def blk_q4k(d=1.0, dmin=0.0):
    b = np.zeros(144, np.uint8)
    b[0:2] = np.frombuffer(np.uint16(O.f32_to_f16(d)).tobytes(), np.uint8)
    b[2:4] = np.frombuffer(np.uint16(O.f32_to_f16(dmin)).tobytes(), np.uint8)
    return b


def test_q4_k_dequant_uniform_scale_one():
    # src/ops/quant.rs:1704-1749
    b = blk_q4k(1.0, 0.0)
    b[4:8] = 1
    b[16:144] = 0x10
    out = O.dequantize("q4_k", b)
    assert out.size == 256
    assert (out[0:32] == 0).all() and (out[32:64] == 1).all()
    assert (out[64:96] == 0).all() and (out[96:128] == 1).all() and (out[128:] == 0).all()


def test_q4_k_dequant_negative_min():
    # src/ops/quant.rs:1751-1767
    b = blk_q4k(1.0, 2.0)
    b[8] = 3
    out = O.dequantize("q4_k", b)
    assert np.all(np.abs(out[:32] - (-6.0)) < 1e-5)


def test_q4_k_scale_min_unpack_closed_form():
    # get_scale_min_k4 (src/ops/quant.rs:267-276) for every (sub-block, value) pair:
    # with d = 1, qs = 1 and dmin = 0, sub-block j decodes to sc_j exactly;
    # with qs = 0 and dmin = -1 it decodes to +m_j.
    rng = np.random.default_rng(7)
    for _ in range(64):
        sc = rng.integers(0, 64, 8)
        m = rng.integers(0, 64, 8)
        k = np.zeros(12, np.uint8)
        for j in range(4):
            k[j] = sc[j] | ((sc[j + 4] >> 4) << 6)
            k[j + 4] = m[j] | ((m[j + 4] >> 4) << 6)
            k[j + 8] = (sc[j + 4] & 15) | ((m[j + 4] & 15) << 4)
        b = blk_q4k(1.0, 0.0)
        b[4:16] = k
        b[16:] = 0x11
        out = O.dequantize("q4_k", b)
        assert np.array_equal(out.reshape(8, 32)[:, 0], sc.astype(F))
        b = blk_q4k(1.0, -1.0)
        b[4:16] = k
        out = O.dequantize("q4_k", b)
        assert np.array_equal(out.reshape(8, 32)[:, 0], m.astype(F))


def test_q6_k_dequant_known_answers():
    # src/ops/quant.rs:1769-1813
    b = np.zeros(210, np.uint8)
    b[192:208] = 1
    b[208:210] = np.frombuffer(np.uint16(0x3C00).tobytes(), np.uint8)
    assert np.all(np.abs(O.dequantize("q6_k", b) + 32.0) < 1e-5)
    b[128] = 0b11_10_01_00
    out = O.dequantize("q6_k", b)
    assert (out[0], out[32], out[64], out[96]) == (-32.0, -16.0, 0.0, 16.0)


def test_q4_0_and_q5_0_element_order():
    # Q4_0 keeps the reference's (2k, 2k+1) nibble order (src/ops/quant.rs:102-108);
    # Q5_0 uses (j, j+16) with the 5th bit from qh (:176-183).
    b = np.zeros(18, np.uint8)
    b[0:2] = np.frombuffer(np.uint16(0x3C00).tobytes(), np.uint8)
    b[2:] = np.arange(16, dtype=np.uint8) | (np.uint8(15) << 4)
    out = O.dequantize("q4_0", b)
    assert out[0::2].tolist() == [float(k - 8) for k in range(16)] and (out[1::2] == 7).all()
    b = np.zeros(22, np.uint8)
    b[0:2] = np.frombuffer(np.uint16(0x3C00).tobytes(), np.uint8)
    qh = (1 << 3) | (1 << 20)
    b[2:6] = np.frombuffer(np.uint32(qh).tobytes(), np.uint8)
    b[6:] = 0x21
    out = O.dequantize("q5_0", b)
    want = np.full(32, 0.0, F)
    want[:16] = 1 - 16
    want[16:] = 2 - 16
    want[3] += 16
    want[20] += 16
    assert np.array_equal(out, want)


def test_q8_0_round_trip_and_decode():
    # src/ops/quant.rs:1608-1633 (encoder), decode d*q exact
    i = np.arange(1024, dtype=F) * F(0.0271)
    data = (np.sin(i) * F(0.5) - np.cos(i * F(1.7)) * F(0.3)).astype(F)
    dq = O.dequantize("q8_0", O.quantize("q8_0", data))
    assert np.mean(np.abs(data - dq)) / np.max(np.abs(data)) < 0.005
    q = O.quantize("q8_0", data).reshape(-1, 34)
    d = q[:, 0:2].copy().view(np.uint16).reshape(-1)
    codes = q[:, 2:].view(np.int8).astype(np.float64)
    exact = np.array([float(O.f16_to_f32(int(h))) for h in d])[:, None] * codes
    assert np.array_equal(dq.reshape(-1, 32).astype(np.float64), exact)


def test_linear_q4_0_matches_dequant_then_matmul():
    # src/ops/quant.rs:1635-1675
    in_f, out_f, batch = 64, 8, 2
    w = (np.sin(np.arange(out_f * in_f, dtype=F) * F(0.013)) * F(0.7)).astype(F)
    wq = O.quantize("q4_0", w)
    wd = O.dequantize("q4_0", wq).reshape(out_f, in_f).astype(np.float64)
    x = (np.cos(np.arange(batch * in_f, dtype=F) * F(0.071)) * F(0.5)).astype(F)
    y = O.linear_q4_0_cpu(x, wq, batch, in_f, out_f)
    ref = x.reshape(batch, in_f).astype(np.float64) @ wd.T
    assert np.max(np.abs(y - ref.reshape(-1))) < 1e-5


# ------------------------------------------------------------ fused == dequant


@pytest.mark.parametrize("in_f,out_f", [(256, 3), (512, 5), (1024, 7), (4096, 2), (8192, 2), (14336, 2)])
def test_fused_q4k_bit_identical_to_dequant_then_dot(in_f, out_f):
    # src/ops/quant.rs:2012-2055
    w = O.lcg_bytes(out_f * (in_f // 256) * 144, 0xC0FFEE)
    x = O.ramp_x(in_f)
    ref = O.linear_q4_k_cpu(x, w, 1, in_f, out_f)
    fused = O.linear_q4_k_fused(x, w, 1, in_f, out_f)
    fin = np.isfinite(ref)
    assert np.array_equal(ref[fin].view(np.uint32), fused[fin].view(np.uint32))


@pytest.mark.parametrize("in_f,out_f", [(256, 3), (1024, 5), (4096, 2), (8192, 2)])
def test_fused_q6k_bit_identical_to_dequant_then_dot(in_f, out_f):
    # src/ops/quant.rs:2097-2128
    w = O.lcg_bytes(out_f * (in_f // 256) * 210, 0xBEEF).reshape(-1, 210)
    w[:, 208:210] = np.frombuffer(np.uint16(0x2E66).tobytes(), np.uint8)
    w = w.reshape(-1)
    x = O.ramp_x(in_f)
    ref = O.linear_q6_k_cpu(x, w, 1, in_f, out_f)
    fused = O.linear_q6_k_fused(x, w, 1, in_f, out_f)
    assert np.array_equal(ref.view(np.uint32), fused.view(np.uint32))


def _pinned_q4k_rows(n_rows, in_f, seed):
    w = O.lcg_bytes(n_rows * (in_f // 256) * 144, seed).reshape(-1, 144)
    w[:, 0:2] = np.frombuffer(np.uint16(0x2E66).tobytes(), np.uint8)
    w[:, 2:4] = np.frombuffer(np.uint16(0x2666).tobytes(), np.uint8)
    return w.reshape(-1)


def test_parallel_matches_serial_every_thread_count():
    # src/ops/quant.rs:2057-2095 (fused), extended to the integer kernels
    in_f, out_f = 4096, 1024
    w = _pinned_q4k_rows(out_f, in_f, 0xC0FFEE)
    x = O.ramp_x(in_f)
    serial_f = O.linear_q4_k_fused(x, w, 1, in_f, out_f)
    serial_i = O.linear_q4_k_integer(x, w, 1, in_f, out_f)
    w6 = O.lcg_bytes(out_f * 16 * 210, 0xBEEF).reshape(-1, 210)
    w6[:, 208:210] = np.frombuffer(np.uint16(0x2E66).tobytes(), np.uint8)
    w6 = w6.reshape(-1)
    serial_6 = O.linear_q6_k_integer(x, w6, 1, in_f, out_f)
    for t in (1, 2, 3, 4, 7, 8, 16, 33):
        assert np.array_equal(O.linear_q4_k_fused(x, w, 1, in_f, out_f, t).view(np.uint32), serial_f.view(np.uint32))
        assert np.array_equal(O.linear_q4_k_integer(x, w, 1, in_f, out_f, t).view(np.uint32), serial_i.view(np.uint32))
        assert np.array_equal(O.linear_q6_k_integer(x, w6, 1, in_f, out_f, t).view(np.uint32), serial_6.view(np.uint32))


# ------------------------------------------------------------ integer k-quants


def test_quantize_block_q8_known_answers():
    # src/ops/quant.rs:750-771: d = amax/127, round half away from zero on the
    # rounded sum t = s + 0.5 (not roundf), NaN ignored by amax and mapped to 0.
    x = np.zeros(256, F)
    x[0] = 127.0  # d = 1, inv = 1: s == x exactly
    x[1] = F(0.5) - F(2.0 ** -25)  # 0.49999997: t rounds to 1.0, so q = 1
    x[2] = -x[1]
    x[3], x[4], x[5] = 1.5, 2.5, -2.5
    x[6] = np.nan
    x[7] = 126.6
    x[40] = -0.0
    q = O.quantize_block_q8(x)
    assert bits(q.d) == bits(F(1.0))
    qs = np.array(q.qs, dtype=np.int32)
    assert qs[:8].tolist() == [127, 1, -1, 2, 3, -3, 0, 127]
    assert list(q.bsums) == [int(qs[32 * j:32 * j + 32].sum()) for j in range(8)]
    # all zero block
    z = O.quantize_block_q8(np.zeros(256, F))
    assert bits(z.d) == 0 and not any(z.qs)
    # an infinite input: d = inf, inv = 0, every code 0 (inf*0 = NaN -> 0)
    xi = np.ones(256, F)
    xi[5] = np.inf
    qi = O.quantize_block_q8(xi)
    assert np.isinf(qi.d) and not any(qi.qs)


def test_quantize_block_q8_random_properties():
    rng = np.random.default_rng(5)
    for _ in range(200):
        x = (rng.standard_normal(256) * np.exp2(rng.integers(-30, 30))).astype(F)
        q = O.quantize_block_q8(x)
        qs = np.array(q.qs, dtype=np.int32)
        amax = np.max(np.abs(x))
        assert bits(q.d) == bits(F(amax) / F(127.0))
        assert np.abs(qs).max() <= 127 and qs[np.argmax(np.abs(x))] in (127, -127)
        # within half a step of x/d (double arithmetic)
        assert np.all(np.abs(qs - x.astype(np.float64) / float(q.d)) <= 0.5 + 1e-4)


def _q4k_block_reversed(w, q):
    """dot_q4k_q8_block with every integer sum taken back to front (src/ops/quant.rs:2135-2182)."""
    d = O.f16_to_f32(int(w[0]) | int(w[1]) << 8)
    dmin = O.f16_to_f32(int(w[2]) | int(w[3]) << 8)
    s = w[4:16].astype(np.int32)
    qs = w[16:].astype(np.int32)
    xq = np.array(q.qs, np.int32)
    acc = accm = 0
    for h in reversed(range(4)):
        sc, mn = [], []
        for j in (2 * h, 2 * h + 1):
            if j < 4:
                sc.append(s[j] & 63)
                mn.append(s[j + 4] & 63)
            else:
                sc.append((s[j + 4] & 15) | ((s[j - 4] >> 6) << 4))
                mn.append((s[j + 4] >> 4) | ((s[j] >> 6) << 4))
        s_lo = sum(int(qs[32 * h + l] & 15) * int(xq[64 * h + l]) for l in reversed(range(32)))
        s_hi = sum(int(qs[32 * h + l] >> 4) * int(xq[64 * h + 32 + l]) for l in reversed(range(32)))
        acc += int(sc[0]) * s_lo + int(sc[1]) * s_hi
        accm += int(mn[0]) * q.bsums[2 * h] + int(mn[1]) * q.bsums[2 * h + 1]
    return F(F(F(d) * F(q.d)) * F(acc)) - F(F(F(dmin) * F(q.d)) * F(accm))


def test_integer_q4k_block_dot_is_order_independent():
    w = O.lcg_bytes(144, 0xABCDEF)
    w[0:2] = np.frombuffer(np.uint16(0x2E66).tobytes(), np.uint8)
    w[2:4] = np.frombuffer(np.uint16(0x2666).tobytes(), np.uint8)
    q = O.quantize_block_q8(O.ramp_x(256))
    assert bits(O.dot_q4k_q8_block(w, q)) == bits(_q4k_block_reversed(w, q))


def _roundtrip(x):
    out = np.zeros_like(x)
    for b in range(x.size // 256):
        q = O.quantize_block_q8(x[b * 256:(b + 1) * 256])
        out[b * 256:(b + 1) * 256] = F(q.d) * np.array(q.qs, dtype=F)
    return out


@pytest.mark.parametrize("n", [256, 1024, 4096, 14336])
def test_integer_q4k_agrees_with_float_on_same_activations(n):
    # src/ops/quant.rs:2191-2245
    w = _pinned_q4k_rows(1, n, 0x13579)
    x = O.ramp_x(n)
    f = O.canonical_dot_q4k_fused(_roundtrip(x), w, n)
    i = O.integer_dot_q4k(x, w, n)
    assert abs(float(f) - float(i)) / max(abs(float(f)), 1.0) < 1e-4


def test_integer_q4k_single_superblock_bit_exact_vs_float():
    # src/ops/quant.rs:2226-2244: one super-block is entirely integer, so the
    # integer path lands on exactly the float-fused bits of the pinned chain.
    w = _pinned_q4k_rows(1, 256, 0x13579)
    x = O.ramp_x(256)
    assert bits(O.canonical_dot_q4k_fused(_roundtrip(x), w, 256)) == bits(O.integer_dot_q4k(x, w, 256))


def test_linear_q4k_integer_is_tree_of_block_dots():
    # linear_q4_k_integer (src/ops/quant.rs:936-980) == fixed_tree of per-block
    # dot_q4k_q8_block over quantize_block_q8 of each 256-slice.
    in_f, out_f = 11008, 3
    w = _pinned_q4k_rows(out_f, in_f, 0x2468).reshape(out_f, -1)
    x = O.ramp_x(in_f)
    y = O.linear_q4_k_integer(x, w.reshape(-1), 1, in_f, out_f)
    for o in range(out_f):
        parts = [O.dot_q4k_q8_block(w[o, s * 144:(s + 1) * 144], O.quantize_block_q8(x[s * 256:(s + 1) * 256]))
                 for s in range(in_f // 256)]
        assert bits(y[o]) == bits(literal_tree(np.array(parts, F)))


def test_q6k_integer_block_brute_force():
    # No published bit pin exists for Q6_K.  Exact brute force: integer codes
    # taken from the pinned float decoder (d = 1, scales = 1 gives code - 32
    # exactly), scale of element e is byte 192 + e//16, acc summed in int64,
    # then (d*dx)*f32(acc) with one float32 rounding per operation.
    rng = np.random.default_rng(11)
    for trial in range(300):
        w = rng.integers(0, 256, 210).astype(np.uint8)
        w[208:210] = np.frombuffer(np.uint16(O.f32_to_f16(float(rng.uniform(1e-3, 0.1)))).tobytes(), np.uint8)
        probe = w.copy()
        probe[192:208] = 1
        probe[208:210] = np.frombuffer(np.uint16(0x3C00).tobytes(), np.uint8)
        codes = O.dequantize("q6_k", probe).astype(np.int64)  # code - 32
        sc = w[192:208].view(np.int8).astype(np.int64)
        x = (rng.standard_normal(256) * (trial % 7 + 1)).astype(F)
        q = O.quantize_block_q8(x)
        xq = np.array(q.qs, dtype=np.int64)
        acc = int(np.sum(sc[np.arange(256) // 16] * codes * xq))
        d = O.f16_to_f32(int(w[208]) | int(w[209]) << 8)
        want = F(F(F(d) * F(q.d)) * F(acc))
        assert bits(O.dot_q6k_q8_block(w, q)) == bits(want), trial


def test_q4k_integer_block_brute_force():
    # Exact brute force of dot_q4k_q8_block with codes from the pinned float
    # decoder: d = 1, dmin = 0 and a probe scale byte layout gives each code.
    rng = np.random.default_rng(12)
    for trial in range(300):
        w = rng.integers(0, 256, 144).astype(np.uint8)
        w[0:2] = np.frombuffer(np.uint16(O.f32_to_f16(float(rng.uniform(1e-3, 0.1)))).tobytes(), np.uint8)
        w[2:4] = np.frombuffer(np.uint16(O.f32_to_f16(float(rng.uniform(1e-3, 0.1)))).tobytes(), np.uint8)
        probe = w.copy()
        probe[0:4] = np.frombuffer(np.array([0x3C00, 0], np.uint16).tobytes(), np.uint8)
        probe[4:16] = [1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1]  # every sub-block scale 1, min 0
        codes = O.dequantize("q4_k", probe).astype(np.int64)  # nibble of element e
        sc = O.dequantize("q4_k", _with(w, qs=0x11, d=1.0, dmin=0.0)).reshape(8, 32)[:, 0].astype(np.int64)
        mn = O.dequantize("q4_k", _with(w, qs=0x00, d=0.0, dmin=-1.0)).reshape(8, 32)[:, 0].astype(np.int64)
        x = (rng.standard_normal(256) * (trial % 5 + 1)).astype(F)
        q = O.quantize_block_q8(x)
        xq = np.array(q.qs, dtype=np.int64)
        acc = int(np.sum(sc[np.arange(256) // 32] * codes * xq))
        accm = int(np.sum(mn * xq.reshape(8, 32).sum(axis=1)))
        d = O.f16_to_f32(int(w[0]) | int(w[1]) << 8)
        dmin = O.f16_to_f32(int(w[2]) | int(w[3]) << 8)
        want = F(F(F(d) * F(q.d)) * F(acc)) - F(F(F(dmin) * F(q.d)) * F(accm))
        assert bits(O.dot_q4k_q8_block(w, q)) == bits(want), trial


def _with(w, qs, d, dmin):
    b = w.copy()
    b[0:2] = np.frombuffer(np.uint16(O.f32_to_f16(d)).tobytes(), np.uint8)
    b[2:4] = np.frombuffer(np.uint16(O.f32_to_f16(dmin)).tobytes(), np.uint8)
    b[16:] = qs
    return b


@pytest.mark.parametrize("n", [256, 1024, 4096])
def test_integer_q6k_agrees_with_float_on_same_activations(n):
    # src/ops/quant.rs:2292-2327
    w = O.lcg_bytes((n // 256) * 210, 0x2468).reshape(-1, 210)
    w[:, 208:210] = np.frombuffer(np.uint16(0x2E66).tobytes(), np.uint8)
    w = w.reshape(-1)
    x = O.ramp_x(n)
    yf = O.linear_q6_k_fused(_roundtrip(x), w, 1, n, 1)
    yi = O.linear_q6_k_integer(x, w, 1, n, 1)
    assert abs(float(yf[0]) - float(yi[0])) / max(abs(float(yf[0])), 1.0) < 1e-4


# ------------------------------------------------------------- error behaviour


def test_error_messages_mirror_reference():
    x = np.zeros(100, F)
    with pytest.raises(O.OracleError, match="linear_q4_k_integer: in_feat not a multiple of 256"):
        O.linear_q4_k_integer(x, np.zeros(144, np.uint8), 1, 100, 1)
    with pytest.raises(O.OracleError, match="linear_q4_k_integer: weight shape mismatch"):
        O.linear_q4_k_integer(np.zeros(256, F), np.zeros(143, np.uint8), 1, 256, 1)
    with pytest.raises(O.OracleError, match="linear_q6_k_integer_parallel: weight shape"):
        O.linear_q6_k_integer(np.zeros(256, F), np.zeros(209, np.uint8), 1, 256, 1, threads=4)
    with pytest.raises(O.OracleError, match="weight dtype not"):
        O.linear_dispatch(1, 0, np.zeros(32, F), np.zeros(64, np.uint8), 1, 32, 1)
    with pytest.raises(O.OracleError, match="linear_q4_0: x size mismatch"):
        O.linear_q4_0_cpu(np.zeros(31, F), np.zeros(18, np.uint8), 1, 32, 1)
    with pytest.raises(O.OracleError, match="Q8_0: in_feat must be a multiple of 32"):
        O.linear_dispatch(8, 0, np.zeros(33, F), np.zeros(34, np.uint8), 1, 33, 1)


def test_empty_shapes():
    assert O.linear_q4_k_integer(np.zeros(0, F), np.zeros(0, np.uint8), 1, 0, 3).tolist() == [0.0, 0.0, 0.0]
    assert O.linear_q6_k_integer(np.zeros(256, F), np.zeros(0, np.uint8), 1, 256, 0).size == 0
    assert O.linear_dispatch(8, 0, np.zeros(0, F), np.zeros(4 * 68, np.uint8), 0, 64, 4).size == 0
    # the blob check does not depend on batch (src/model/forward_quantized.rs:756-758)
    with pytest.raises(O.OracleError, match="weight blob too small"):
        O.linear_dispatch(8, 0, np.zeros(0, F), np.zeros(0, np.uint8), 0, 64, 4)
