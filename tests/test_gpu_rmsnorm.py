"""rms_norm_slice on the GPU (vtqrt_rms_norm_device) vs the CPU oracle.

The sum of squares is the reference's serial fp32 chain (src/ops/rms_norm.rs:
60-110), which the GPU runs as a register chain with readlane hand-offs
between 32-value segments, or, for 1024-4096 values (a multiple of 64), as a
serial head followed by an exact walk over per-binade integer prefix sums
(the sizes around 1024, 2048 and 4096 take both forms).  The inputs cover round-to-even ties (short
mantissas, small half-integers), subnormal squares, a sum that overflows to
inf, NaN, zero runs, binade changes late in the chain, and sizes around the
segment and 2048-value pass boundaries.  Outputs must match bit for bit (NaN
positions where the sum is NaN).
"""
import numpy as np
import pytest
import torch

import oracle
from vtq import runtime

pytestmark = pytest.mark.gpu

# up to 32768, the entry point's limit; past 16384 the products take more
# than 64 KiB of LDS (the kernel's raised dynamic-LDS limit)
SIZES = [1, 7, 256, 575, 576, 1000, 1024, 1040, 1088, 2048, 2049, 2112, 2560, 3072, 4032, 4096, 4160, 4607, 4608,
         4609, 5000, 8192, 16384, 16385, 32768]


def make_x(kind, n, rng):
    g = rng.standard_normal(n)
    if kind == "gauss":
        x = g
    elif kind == "tiny":            # squares in the subnormal range
        x = g * 1e-22
    elif kind == "mixed_tiny":      # subnormal squares then normal ones
        x = np.where(np.arange(n) < n // 2, g * 1e-21, g * 1e-3)
    elif kind == "huge":            # sum overflows to inf
        x = g * 3e19
    elif kind == "halves":          # t/u ties are frequent
        x = rng.integers(-3, 4, n) * 0.5
    elif kind == "short":           # few mantissa bits
        x = rng.integers(0, 4096, n) * np.exp2(-rng.integers(0, 30, n).astype(np.float64))
    elif kind == "growing":         # the sum crosses many binades late
        x = g * np.exp2(np.arange(n) * (20.0 / max(n, 1)))
    elif kind == "outliers":
        x = np.where(rng.random(n) < 0.02, g * 1000.0, g)
    elif kind == "zeros_then":
        x = np.where(np.arange(n) < (3 * n) // 4, 0.0, g)
    elif kind == "ones":
        x = np.ones(n)
    elif kind == "nan":
        x = g.copy()
        x[rng.integers(0, n)] = np.nan
    elif kind == "inf":
        x = g.copy()
        x[rng.integers(0, n)] = np.inf
    else:
        raise ValueError(kind)
    return x.astype(np.float32)


KINDS = ["gauss", "tiny", "mixed_tiny", "huge", "halves", "short", "growing", "outliers", "zeros_then", "ones",
         "nan", "inf"]


def run_gpu(x, w, eps):
    dev = torch.device("cuda:0")
    dx = torch.from_numpy(x).to(dev)
    dw = torch.from_numpy(w).to(dev)
    dy = torch.full_like(dx, float("nan"))
    runtime.rms_norm_device(dx.data_ptr(), dw.data_ptr(), x.size, eps, dy.data_ptr(), None)
    torch.cuda.synchronize()
    return dy.cpu().numpy()


def same(a, b):
    nan = np.isnan(a) & np.isnan(b)
    return bool(np.all(nan | (a.view(np.uint32) == b.view(np.uint32))))


@pytest.mark.parametrize("n", SIZES)
def test_rms_norm_matches_oracle(n):
    rng = np.random.default_rng(1000 + n)
    eps = np.float32(1e-5)
    for kind in KINDS:
        for rep in range(2):
            x = make_x(kind, n, rng)
            w = (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)
            ref = oracle.rms_norm(x, w, eps)
            got = run_gpu(x, w, eps)
            assert same(got, ref), f"n={n} kind={kind} rep={rep}: first difference at {np.argmax(got != ref)}"


def test_rms_norm_many_gaussian_rows():
    # the common case at the decode step's width, many seeds
    rng = np.random.default_rng(7)
    eps = np.float32(1e-5)
    for _ in range(200):
        x = (rng.standard_normal(2048) * rng.choice([0.01, 1.0, 30.0])).astype(np.float32)
        w = rng.standard_normal(2048).astype(np.float32)
        assert same(run_gpu(x, w, eps), oracle.rms_norm(x, w, eps))


@pytest.mark.parametrize("n", [0, 32769])
def test_rms_norm_rejects_sizes_outside_the_kernel(n):
    """n = 0 and n > 32768 are refused on the host (VTQ_E_NOT_IMPLEMENTED)
    before any launch."""
    x = torch.zeros(max(n, 1), dtype=torch.float32, device="cuda:0")
    y = torch.full_like(x, 7.0)
    rc = runtime.lib().vtqrt_rms_norm_device(x.data_ptr(), x.data_ptr(), n, 1e-5, y.data_ptr(), None)
    torch.cuda.synchronize()
    assert rc == 3
    assert bool((y == 7.0).all())
