"""The device libm against the reference's transcendental pin.

RoPE, softmax, SwiGLU and RMSNorm's sqrtf run on the GPU through
vitni-tensor_amd/csrc/vtq_libm.h.  The reference pins the `libm = "0.2"`
functions with one BLAKE3 over expf, sqrtf(|x|), cosf, sinf,
powf(1e4, x/64), powf(1e6, x/64) and the sigmoid of 489,509 inputs
(tests/transcendental_determinism.rs:14-63, PINNED_TRANSCENDENTAL).  Here the
same sweep is evaluated by the device code (vtqrt_transcendentals_device) and
hashed on the host with the product's BLAKE3; the hash must be the pin.
"""
import numpy as np
import pytest
import torch

from vtq import runtime

pytestmark = pytest.mark.gpu

PINNED_TRANSCENDENTAL = "0ae93cd6394c934bfb94a5803a0528193ba0c2330002162a0094062c294bc3d0"
CORNERS = [0.0, -0.0, 1.0, -1.0, 0.5, -0.5, np.finfo(np.float32).tiny, 1e-20, 1e-10, 1e10, 1e20, 87.0, 88.0, 88.7,
           -87.0, -88.0, -104.0, np.pi, np.e]


def sweep_inputs():
    """x = -30; while x <= 30 { push x; x += 0.000123 } in f32, then the corners."""
    steps = np.full(500_000, np.float32(0.000123), dtype=np.float32)
    steps[0] = np.float32(-30.0)
    xs = np.add.accumulate(steps, dtype=np.float32)  # sequential f32 adds, as the loop
    n = int(np.argmax(~(xs <= np.float32(30.0))))
    return np.concatenate([xs[:n], np.array(CORNERS, dtype=np.float32)])


def test_device_libm_matches_transcendental_pin():
    x = sweep_inputs()
    assert x.size == 489509
    dx = torch.from_numpy(x).to("cuda:0")
    dy = torch.empty(7 * x.size, dtype=torch.float32, device="cuda:0")
    runtime.transcendentals_device(dx.data_ptr(), x.size, dy.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    y = dy.cpu().numpy()
    assert runtime.blake3(y.view(np.uint8)).hex() == PINNED_TRANSCENDENTAL
