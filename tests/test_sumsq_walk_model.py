"""The sum-of-squares binade walk (vtq_sumsq.h) on the CPU, fuzzed.

tests/native/sumsq_walk_model.c restates sumsq_walk_helper and sumsq_walk
statement for statement (64 lanes as loops, ballots as bit masks, the DPP
scans in their order).  Every row's result must equal rms_norm_slice's
serial chain (src/ops/rms_norm.rs:96-100) bit for bit, and the rows below
must reach every branch of the walk: crossings and ties, moving one and
several binades at once, leaving the window, the stop limit, capped helper
totals, and the helpers' fallback for non-finite or tiny sums (the check of
the head's sum against the window is defensive and unreachable, see below).
The walk tables start each row filled with a stale byte pattern, as LDS
holds whatever the last row left.  The empty second ballot (guarded in the
kernel) must never occur.
"""
import ctypes
import os
import shutil
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
F = np.float32
FLAGS = {"helper_fb": 1, "start_fb": 2, "no_event": 4, "cross": 8, "tie": 16, "next_bin": 32, "jump_bin": 64,
         "left_window": 128, "stop_limit": 256, "capped": 512, "guard": 1024}


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    cc = shutil.which("gcc")
    if not cc:
        pytest.skip("gcc not available")
    so = str(tmp_path_factory.mktemp("walk") / "libwalk.so")
    subprocess.run([cc, "-O2", "-std=c11", "-ffp-contract=off", "-fno-fast-math", "-shared", "-fPIC", "-o", so,
                    os.path.join(ROOT, "tests", "native", "sumsq_walk_model.c"), "-lm"], check=True)
    lib = ctypes.CDLL(so)
    fp, i, ip = ctypes.POINTER(ctypes.c_float), ctypes.c_int, ctypes.POINTER(ctypes.c_int)
    lib.walk_sumsq.argtypes = [fp, i, i, ip]
    lib.walk_sumsq.restype = ctypes.c_float
    lib.serial_sumsq.argtypes = [fp, i]
    lib.serial_sumsq.restype = ctypes.c_float
    lib.walk_head.argtypes = [i]
    lib.walk_head.restype = i
    return lib


def run(lib, x, stale=0xA5):
    x = np.ascontiguousarray(x, F)
    fl = ctypes.c_int()
    p = x.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
    got = np.float32(lib.walk_sumsq(p, x.size, stale, ctypes.byref(fl)))
    want = np.float32(lib.serial_sumsq(p, x.size))
    return got, want, fl.value


def rows(n, count, seed):
    """Seeded rows of every kind, cycling through the kinds."""
    rng = np.random.default_rng(seed)
    lib_h = 640 if n - 1536 < 640 else n - 1536
    for r in range(count):
        kind = r % 12
        if kind == 0:  # Gaussian, the decode step's case
            x = rng.standard_normal(n)
        elif kind == 1:  # short mantissas: values on a 2^-6 grid, ties everywhere
            x = rng.integers(-64, 65, n) / 64.0
        elif kind == 2:  # one large term after the head lifts the sum 1-4 binades at once
            x = rng.standard_normal(n)
            x[rng.integers(lib_h, n)] = np.sqrt(n) * 2.0 ** rng.uniform(0.5, 2.5)
        elif kind == 3:  # eight large squares in one helper lane: totals above the cap
            x = rng.standard_normal(n) * 1e-3
            j = lib_h + 8 * rng.integers(0, (n - lib_h) // 8)
            x[j:j + 8] = rng.uniform(1.0, 4.0, 8)
        elif kind == 4:  # a steadily growing row: many crossings, the stop limit
            x = rng.standard_normal(n) * np.exp(np.linspace(0, rng.uniform(4, 12), n))
        elif kind == 5:  # short mantissas with a large term: ties on and around crossings
            x = rng.integers(-8, 9, n) / 8.0
            x[rng.integers(lib_h, n)] = rng.integers(16, 96) / 2.0
        elif kind == 6:  # tiny and subnormal squares, zeros
            x = rng.standard_normal(n) * 10.0 ** rng.uniform(-30, -19)
            x[rng.random(n) < 0.3] = 0.0
        elif kind == 7:  # non-finite and overflowing squares
            x = rng.standard_normal(n)
            x[rng.integers(0, n)] = [np.inf, -np.inf, np.nan, 3e19][r % 4]
        elif kind == 8:  # a zero head, then values: the head's sum is outside every window
            x = rng.standard_normal(n)
            x[:lib_h] = 0.0
        elif kind == 9:  # outliers in the head, a quiet tail
            x = rng.standard_normal(n) * 1e-2
            x[rng.integers(0, lib_h, 4)] = rng.uniform(5, 50, 4)
        elif kind == 11:  # squares on a 1/16 grid, so the running sum lands exactly on powers of two,
            # then terms with bits below the unit, so a missed crossing would round them wrong
            x = rng.choice(np.array([-1.0, -0.5, -0.25, 0.25, 0.5, 1.0]), n)
            t = rng.integers(lib_h, n)
            x[t:] += rng.standard_normal(n - t) * 1e-3
        else:  # a tie at almost every term: x = k * 2^-12, k odd, so each square's lowest set
            # bit is 2^-24, half a unit of the binade [1, 2) the sum stays in: the stop limit
            kmax = int(np.sqrt(1.9 * 3 * 2.0 ** 24 / n))
            x = (2 * rng.integers(0, kmax // 2, n) + 1) * 2.0 ** -12
        yield kind, x.astype(F)


def crossing_rows(n):
    """Rows whose running sum crosses a power of two P on a term p that
    rounds past P by more than one unit u of the old binade: grid terms
    (squares 2^-8 in the head, 2^-6 after it) bring the sum to P - r
    exactly, then p with p - r in (u, 1.5u) (the sum rounds to P + 2u in the
    new binade, while u-grid rounding would give P + u and then P), then
    small grid terms that keep the sum below 2P.  A walk that missed the
    crossing would round the crossing term twice and end 2u low."""
    out = []
    H = 640 if n - 1536 < 640 else n - 1536
    for frac in (1.1, 1.25, 1.45):
        x = np.full(n, 1.0 / 8, F)
        x[:H] = 1.0 / 16
        head = F(H / 256.0)
        P = F(2.0 ** (np.floor(np.log2(head)) + 1))
        t = H + int(np.ceil((P - head) * 64)) - 1  # before term t the sum is P - r, 0 < r <= 2^-6
        S = F(head + (t - H) / 64.0)
        r = P - S
        u = F(2.0 ** (np.floor(np.log2(S)) - 23))
        if t + 2 >= n or not (0 < r <= 1.0 / 64):
            continue
        xt = F(np.sqrt(float(r + frac * u)))
        for _ in range(64):  # nudge x until its rounded square lands in the interval
            pt = xt * xt
            if pt - r <= u:
                xt = np.nextafter(xt, F(1.0))
            elif pt - r >= F(1.5) * u:
                xt = np.nextafter(xt, F(0.0))
            else:
                break
        if u < (xt * xt) - r < F(1.5) * u:
            x[t] = xt
            x[t + 1:] = 1.0 / 64  # squares 2^-12: exact adds that keep the sum below 2P
            out.append(x)
    return out


@pytest.mark.parametrize("n", [1024, 2048, 2560, 4096])
def test_walk_crossing_that_rounds_past_a_unit(model, n):
    xs = crossing_rows(n)
    assert xs, "no row constructed"
    for x in xs:
        got, want, fl = run(model, x)
        assert fl & FLAGS["cross"]
        assert got.view(np.uint32) == want.view(np.uint32), f"walk {got!r} vs serial {want!r} (flags {fl:#x})"


@pytest.mark.parametrize("n", [1024, 2048, 2560, 4096])
def test_walk_equals_serial_chain(model, n):
    seen = 0
    for r, (kind, x) in enumerate(rows(n, 6000, 1000 + n)):
        got, want, fl = run(model, x, stale=(0xA5, 0x00, 0xFF)[r % 3])
        seen |= fl
        assert fl & FLAGS["guard"] == 0, f"row {r} kind {kind}: the second ballot came back empty"
        if np.isnan(want):
            assert np.isnan(got), f"row {r} kind {kind}"
        else:
            assert got.view(np.uint32) == want.view(np.uint32), (
                f"n {n} row {r} kind {kind}: walk {got!r} vs serial {want!r} (flags {fl:#x})")
    # start_fb is defensive: every summation order of non-negative terms is
    # within n * 2^-24 relative of the serial head sum, inside the window's
    # 2^-12 margin, so the head's sum always lies in the window
    missing = [k for k, b in FLAGS.items() if k not in ("guard", "start_fb") and not seen & b]
    assert not missing, f"n {n}: branches never reached: {missing}"


def test_planted_mistake_is_caught(model):
    # the serial chain is the checker: a sum formed pairwise differs on the
    # decode step's kind of row, so agreement above is not vacuous
    x = np.random.default_rng(3).standard_normal(2048).astype(F)
    got, want, _ = run(model, x)
    pairwise = np.float32(np.sum(x.astype(F) * x.astype(F), dtype=F))
    assert got.view(np.uint32) == want.view(np.uint32)
    assert pairwise.view(np.uint32) != want.view(np.uint32)
