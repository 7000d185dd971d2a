"""vtq_linear_device_noalloc against vtq_linear_device (GPU).

The allocation-free entry point keeps the prefill GEMM's workspace in a
fixed per-GPU array instead of allocating it.  Its outputs must be
bit-identical to the allocating entry point's on the same inputs, on two
calls in a row (the second smaller, so the array holds the first call's
larger contents), through the GEMM and the GEMV paths; a request whose
workspace exceeds the array is refused without a launch.  The device's free
memory is the same before and after a first GEMM call on a fresh context,
and the call captured in a HIP graph replays to the same bits."""
import ctypes

import numpy as np
import pytest
import torch

import vtq
from vtq import synth

pytestmark = pytest.mark.gpu


def _noalloc(ctx):
    f = ctx.lib.vtq_linear_device_noalloc
    vp, sz, i = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
    f.argtypes = [vp, i, i, vp, vp, sz, vp, sz, sz, sz, vp]
    f.restype = i
    return f


def _run_both(ctx, ggml_type, batch, in_feat, out_feat, seed):
    w = synth.weights(ggml_type, out_feat, in_feat, seed=seed)
    x = synth.activations(batch * in_feat, seed=seed + 1)
    dev = torch.device("cuda:0")
    dx, dw = torch.from_numpy(x).to(dev), torch.from_numpy(w).to(dev)
    ya = torch.full((batch * out_feat,), float("nan"), device=dev)
    yb = torch.full((batch * out_feat,), float("nan"), device=dev)
    s = torch.cuda.current_stream().cuda_stream
    ctx.linear_device(ggml_type, 0, dx.data_ptr(), dw.data_ptr(), w.size, ya.data_ptr(), batch, in_feat, out_feat, s)
    rc = _noalloc(ctx)(ctx.handle, ggml_type, 0, dx.data_ptr(), dw.data_ptr(), w.size, yb.data_ptr(), batch, in_feat,
                       out_feat, s)
    torch.cuda.synchronize()
    assert rc == 0, ctx.lib.vtq_last_error(ctx.handle)
    a, b = ya.cpu().numpy(), yb.cpu().numpy()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"{batch}x{in_feat}->{out_feat}: outputs differ"
    assert not np.isnan(b).any()


def test_noalloc_matches_allocating_entry_point():
    ctx = vtq.Context(0)
    try:
        # GEMM path (scratch used): the prefill shape, then a smaller one
        _run_both(ctx, vtq.Q4_K, 512, 4096, 14336, seed=11)
        _run_both(ctx, vtq.Q4_K, 40, 2048, 1000, seed=13)
        # GEMV paths (no scratch), after the scratch holds stale data
        _run_both(ctx, vtq.Q4_K, 1, 11008, 4096, seed=17)
        _run_both(ctx, vtq.Q6_K, 1, 4096, 777, seed=19)
        # rows longer than one segment: the segments' sums go through the scratch
        _run_both(ctx, vtq.Q4_K, 3, 49152, 300, seed=23)
        _run_both(ctx, vtq.Q6_K, 1, 32768 + 256, 100, seed=29)
    finally:
        ctx.close()


def test_noalloc_rejects_workspace_beyond_scratch():
    ctx = vtq.Context(0)
    try:
        # 8192 tokens x in_feat 8192: 72 MB of workspace > 32 MiB.  The
        # buffers have the full declared sizes, so even a launch would stay
        # in bounds.
        x = torch.zeros(8192 * 8192, device="cuda:0")
        w = torch.from_numpy(synth.weights(vtq.Q4_K, 1, 8192, seed=5)).to("cuda:0")
        y = torch.full((8192,), 7.0, device="cuda:0")
        rc = _noalloc(ctx)(ctx.handle, vtq.Q4_K, 0, x.data_ptr(), w.data_ptr(), w.numel(), y.data_ptr(), 8192, 8192,
                           1, None)
        torch.cuda.synchronize()
        assert rc == vtq.E_NOT_IMPLEMENTED
        assert b"32 MiB scratch" in ctx.lib.vtq_last_error(ctx.handle)
        assert bool((y == 7.0).all())
    finally:
        ctx.close()


def _inputs(ggml_type, batch, in_feat, out_feat, seed):
    dev = torch.device("cuda:0")
    w = torch.from_numpy(synth.weights(ggml_type, out_feat, in_feat, seed=seed)).to(dev)
    x = torch.from_numpy(synth.activations(batch * in_feat, seed=seed + 1)).to(dev)
    return x, w


def test_noalloc_first_call_leaves_free_memory_unchanged():
    # Kernels load their code once per process, so a first context runs both
    # paths; a fresh context then makes its first calls while the device's
    # free memory (hipMemGetInfo) is watched.  Every buffer exists beforehand.
    cases = [(vtq.Q4_K, 512, 4096, 14336, 31), (vtq.Q4_K, 1, 11008, 4096, 37)]
    bufs = []
    for t, batch, in_f, out_f, seed in cases:
        x, w = _inputs(t, batch, in_f, out_f, seed)
        bufs.append((t, batch, in_f, out_f, x, w, torch.empty(batch * out_f, device="cuda:0")))
    warm = vtq.Context(0)
    try:
        for t, batch, in_f, out_f, x, w, y in bufs:
            rc = _noalloc(warm)(warm.handle, t, 0, x.data_ptr(), w.data_ptr(), w.numel(), y.data_ptr(), batch, in_f,
                                out_f, torch.cuda.current_stream().cuda_stream)
            assert rc == 0, warm.lib.vtq_last_error(warm.handle)
        torch.cuda.synchronize()
    finally:
        warm.close()
    ctx = vtq.Context(0)
    try:
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info(0)[0]
        for t, batch, in_f, out_f, x, w, y in bufs:
            rc = _noalloc(ctx)(ctx.handle, t, 0, x.data_ptr(), w.data_ptr(), w.numel(), y.data_ptr(), batch, in_f,
                               out_f, torch.cuda.current_stream().cuda_stream)
            assert rc == 0, ctx.lib.vtq_last_error(ctx.handle)
        torch.cuda.synchronize()
        free1 = torch.cuda.mem_get_info(0)[0]
        assert free1 == free0, f"free device memory changed by {free0 - free1} bytes"
    finally:
        ctx.close()


@pytest.mark.parametrize("ggml_type,batch,in_feat,out_feat", [(vtq.Q4_K, 64, 4096, 1000), (vtq.Q4_K, 96, 5632, 300),
                                                              (vtq.Q4_K, 1, 11008, 4096), (vtq.Q6_K, 1, 4096, 777)])
def test_noalloc_under_graph_capture(ggml_type, batch, in_feat, out_feat):
    # the GEMM paths (per-wave kernel at in_feat 4096, LDS-operand kernel at
    # 5632) and two GEMV paths, captured once and replayed three times; before
    # each replay the output is overwritten eagerly and unrelated work runs
    ctx = vtq.Context(0)
    try:
        x, w = _inputs(ggml_type, batch, in_feat, out_feat, 41 + in_feat)
        want = torch.full((batch * out_feat,), float("nan"), device="cuda:0")
        ctx.linear_device(ggml_type, 0, x.data_ptr(), w.data_ptr(), w.numel(), want.data_ptr(), batch, in_feat,
                          out_feat, torch.cuda.current_stream().cuda_stream)
        y = torch.full((batch * out_feat,), float("nan"), device="cuda:0")
        f = _noalloc(ctx)
        # one eager call first: launch attributes are set outside the capture
        assert f(ctx.handle, ggml_type, 0, x.data_ptr(), w.data_ptr(), w.numel(), y.data_ptr(), batch, in_feat,
                 out_feat, torch.cuda.current_stream().cuda_stream) == 0
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            rc = f(ctx.handle, ggml_type, 0, x.data_ptr(), w.data_ptr(), w.numel(), y.data_ptr(), batch, in_feat,
                   out_feat, torch.cuda.current_stream().cuda_stream)
        assert rc == 0, ctx.lib.vtq_last_error(ctx.handle)
        ref = want.cpu().numpy().view(np.uint32)
        for k in range(3):
            y.fill_(float("nan"))
            junk = torch.randn(1 << 20, device="cuda:0").sum()  # unrelated eager work between replays
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            got = y.cpu().numpy().view(np.uint32)
            assert np.array_equal(got, ref), f"replay {k}: {int((got != ref).sum())} outputs differ"
            del junk
        del g
    finally:
        ctx.close()
