"""Benchmark of the quantized linear hot path on one MI355X.

Default workload: one step = the Q4_K decode GEMV
pair of a Llama-7B FFN, 11008x4096 then 4096x11008, batch 1, exact-integer
regime, through libvtq's device-pointer entry point with inputs resident in
HBM.  Weights rotate over enough copies (> 512 MB) that every launch reads
them from HBM, not from the 256 MB MALL.

Prints ONE JSON line (rank 0).  `value` is whole-step throughput in GB/s of
algorithmic bytes (packed weights + fp32 x in + fp32 y out) over exactly
--steps steps replayed from a HIP graph.  `roofline` describes the dominant
kernel of the step (the slower of the pair, 4096x11008): its launch time is
the median over >= 50 graph replays of back-to-back launches, bracketed by
HIP events on the launch stream.  `cpu_baseline` is the pinned C
restatement of the reference path (oracle/, the std-parallel row-parallel
integer kernels) timed on this host's cores on the same inputs.

`configs` carries every BASELINE configuration measured in the same run:
per kernel the median launch time over >= 50 graph replays with the weights
rotated (HBM, the main figure) and with one copy (MALL-warm), the roofline
fraction, whether the output is bit-identical to the oracle, and the oracle's
CPU time on the same inputs.

Other workloads (`--workload NAME`) time one configuration alone; they are
what the rocprofv3 profiles run.
"""
import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "vitni-tensor_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "Q4_K decode GEMV GB/s & % HBM peak; prefill i8-MFMA util; bit-exact"
HBM_PEAK_GBS = 8000.0
MALL_BYTES = 256 << 20
ROTATE_MIN_BYTES = 600 << 20

WORKLOADS = {
    "q4k_gemv_ffn_pair": ["q4k_11008x4096", "q4k_4096x11008"],
    "q8_0_gemv": ["q8_0_4096x4096"],
    "q4k_gemv_11008x4096": ["q4k_11008x4096"],
    "q4k_gemv_4096x11008": ["q4k_4096x11008"],
    "q6k_gemv_lm_head": ["q6k_32000x4096"],
    "q4k_gemm_prefill": ["q4k_gemm_14336x4096_m512"],
    "e2e_decode": [],  # config 5: libvtq_runtime decode of the random-init 1.1B Llama
}
KERNEL_NAME = {12: "kquant_rows_kernel<Q4K>", 14: "kquant_rows_kernel<Q6K>", 8: "q8_lds_kernel<16>"}
INT8_MFMA_PEAK_TOPS = 5000.0


CPU_THREAD_CAP = 16  # the GPU box's CPU share for one GPU (OMP_NUM_THREADS there is 16)
LAUNCHES_PER_REPLAY = 100  # back-to-back launches per graph replay in the per-kernel medians


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--workload", default="q4k_gemv_ffn_pair", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-rotate", action="store_true", help="reuse one weight copy (MALL-warm figure)")
    ap.add_argument("--eager", action="store_true", help="time eager launches instead of a replayed HIP graph")
    ap.add_argument("--reps", type=int, default=50, help="graph replays per median")
    ap.add_argument("--no-configs", action="store_true", help="skip the per-config figures of the default line")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="only run 20 device-to-device copies of this many MiB (HBM counter calibration)")
    return ap.parse_args()


def cpu_threads():
    return min(len(os.sched_getaffinity(0)), CPU_THREAD_CAP)


def calibrate_copy(mib):
    """Plain device copies of a known size: the reference point that scales
    rocprofv3's FETCH_SIZE / WRITE_SIZE counters to bytes."""
    import torch

    n = mib << 20
    src = torch.ones(n, dtype=torch.uint8, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(20):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "device-to-device copy", "bytes_read": n, "bytes_written": n,
                      "copies": 20}), flush=True)


class Timer:
    """Back-to-back launches captured in one HIP graph (unless eager) and
    replayed; HIP events on the launch stream bracket each replay."""

    def __init__(self, eager=False):
        import torch

        self.torch = torch
        self.eager = eager
        self.stream = torch.cuda.current_stream()

    def per_launch_us(self, body, n, reps):
        """[per-launch microseconds of each of `reps` replays of n launches]."""
        torch = self.torch
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        out = []
        if self.eager:
            for _ in range(reps):
                torch.cuda.synchronize()
                e0.record(self.stream)
                for k in range(n):
                    body(k, self.stream.cuda_stream)
                e1.record(self.stream)
                torch.cuda.synchronize()
                out.append(e0.elapsed_time(e1) / n * 1e3)
            return out
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            cs = torch.cuda.current_stream().cuda_stream
            for k in range(n):
                body(k, cs)
        g.replay()
        torch.cuda.synchronize()
        for _ in range(reps):
            e0.record(self.stream)
            g.replay()
            e1.record(self.stream)
            torch.cuda.synchronize()
            out.append(e0.elapsed_time(e1) / n * 1e3)
        del g
        return out


def stream_ceiling(dw, timer, reps):
    """A plain device-to-device copy (torch copy_) of the rotated weight
    copies into one destination, read + write bytes counted: the HBM rate of
    the simplest library kernel on buffers of this size, launch floor
    included: a measured stream peak beside the published one."""
    import torch

    flat = [w for copies in dw for w in copies]
    dst = torch.empty_like(flat[0])
    us = statistics.median(timer.per_launch_us(
        lambda k, cs: dst[: flat[k % len(flat)].numel()].copy_(flat[k % len(flat)]), LAUNCHES_PER_REPLAY, reps))
    nbytes = 2 * statistics.mean(w.numel() for w in flat)
    return {"kernel": "device-to-device copy of the rotated weight copies (graph-replayed), read + write",
            "bytes_per_launch": int(nbytes), "us_per_launch": round(us, 3),
            "gb_s": round(nbytes / us / 1e3, 1), "frac_of_peak": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)}


READ_WORKGROUPS = (1024, 2048, 4096, 8192)


def read_ceiling(nbytes, timer, reps):
    """A hand-written read-only stream (libvtq_probe's stream_read_kernel:
    grid-stride 16-byte loads, one in flight per thread, no writes) over
    `nbytes` rotated over > 600 MB of copies, graph-replayed like the GEMVs:
    the read rate a plain access pattern reaches on buffers of this size,
    launch floor included.  The best of a few grid sizes is kept."""
    import torch

    from vtq import probe

    n = (nbytes + 15) // 16 * 16
    copies = max(2, -(-ROTATE_MIN_BYTES // n))
    bufs = [torch.ones(n, dtype=torch.uint8, device="cuda:0") for _ in range(copies)]
    sink = torch.zeros(max(READ_WORKGROUPS), dtype=torch.int32, device="cuda:0")
    per_wg = {}
    for wg in READ_WORKGROUPS:
        per_wg[wg] = statistics.median(timer.per_launch_us(
            lambda k, cs, wg=wg: probe.stream_read(bufs[k % copies].data_ptr(), n, wg, sink.data_ptr(), cs),
            LAUNCHES_PER_REPLAY, reps))
    wg = min(per_wg, key=per_wg.get)
    us = per_wg[wg]
    del bufs, sink
    torch.cuda.empty_cache()
    return {"kernel": "stream_read_kernel (libvtq_probe): read-only grid-stride 16-byte loads of rotated copies, "
                      "graph-replayed", "bytes_per_launch": n, "weight_copies_rotated": copies, "workgroups": wg,
            "us_per_launch": round(us, 3), "us_per_launch_by_workgroups": {str(k): round(v, 3) for k, v in per_wg.items()},
            "gb_s": round(n / us / 1e3, 1), "frac_of_peak": round(n / us / 1e3 / HBM_PEAK_GBS, 4)}


def gemm_counters():
    """The committed rocprofv3 SQ-counter summary of the prefill GEMM
    (profiles/q4k_gemm_prefill_sq_counters.json): MFMA busy fraction of the
    matrix cores over the kernel's duration, with the command that made it."""
    path = os.path.join(ROOT, "profiles", "q4k_gemm_prefill_sq_counters.json")
    if not os.path.exists(path):
        return None
    d = json.load(open(path))
    return {"mfma_busy_frac": d["derived"]["mfma_busy_frac"],
            "valu_mfma_coexec_frac_of_mfma_busy": d["derived"]["valu_mfma_coexec_frac_of_mfma_busy"],
            "kernel": d["kernel"], "source": "profiles/q4k_gemm_prefill_sq_counters.json",
            "command": d["command"]}


def mfma_ceiling(m, k_, nn, timer, reps):
    """hipBLASLt's int8 GEMM (torch._int_mm) at the prefill shape: the int8
    rate a vendor GEMM reaches (a plain int32 product, not the reference's
    Q4_K arithmetic)."""
    import torch

    if not hasattr(torch, "_int_mm"):
        return {"unavailable": "torch._int_mm missing"}
    a = torch.randint(-127, 128, (m, k_), dtype=torch.int8, device="cuda:0")
    b = torch.randint(-127, 128, (k_, nn), dtype=torch.int8, device="cuda:0")
    try:
        for _ in range(3):
            torch._int_mm(a, b)
        torch.cuda.synchronize()
        us = statistics.median(Timer(eager=True).per_launch_us(lambda k, cs: torch._int_mm(a, b), 10, max(5, reps // 5)))
    except RuntimeError as e:  # not every build ships the int8 GEMM
        return {"unavailable": str(e)[:120]}
    tops = 2.0 * m * k_ * nn / us / 1e6
    return {"kernel": f"torch._int_mm int8 {m}x{k_} @ {k_}x{nn} -> int32 (hipBLASLt)",
            "us_per_launch": round(us, 3), "tops": round(tops, 1), "frac_of_peak": round(tops / INT8_MFMA_PEAK_TOPS, 4)}


def cpu_time(fn, seconds, min_runs=3, max_runs=200):
    """Median wall time of fn() after one warm-up, bounded to ~`seconds`."""
    fn()
    times = []
    t_end = time.perf_counter() + seconds
    while len(times) < min_runs or (time.perf_counter() < t_end and len(times) < max_runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


class Linear:
    """One BASELINE linear configuration resident on the GPU: x, the weight
    copies rotated over > 600 MB, y; launched through vtq_linear_device."""

    def __init__(self, ctx, cfg, rotate=True):
        import torch

        self.ctx, self.c = ctx, cfg
        self.x, self.w = cfg.make()
        self.copies = 1 if not rotate else max(2, -(-ROTATE_MIN_BYTES // cfg.weight_bytes()))
        dev = torch.device("cuda:0")
        self.dx = torch.from_numpy(self.x).to(dev)
        self.dw = [torch.from_numpy(self.w).to(dev) for _ in range(self.copies)]
        self.dy = torch.empty(cfg.batch * cfg.out_feat, dtype=torch.float32, device=dev)

    def launch(self, k, stream, copy=None):
        c = self.c
        w = self.dw[(k if copy is None else copy) % self.copies]
        self.ctx.linear_device(c.ggml_type, 0, self.dx.data_ptr(), w.data_ptr(), w.numel(), self.dy.data_ptr(),
                               c.batch, c.in_feat, c.out_feat, stream)

    def bit_exact(self, threads):
        import numpy as np
        import torch

        import oracle

        c = self.c
        self.dy.fill_(float("nan"))
        self.launch(0, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        want = oracle.linear_dispatch(c.ggml_type, 0, self.x, self.w, c.batch, c.in_feat, c.out_feat, threads)
        return bool(np.array_equal(self.dy.cpu().numpy().view(np.uint32), want.view(np.uint32)))

    def release(self):
        import torch

        del self.dx, self.dw, self.dy
        torch.cuda.empty_cache()


def config_figures(ctx, cfg, timer, reps, cpu_seconds, with_cpu):
    """Per-config figures: median launch time over `reps` graph replays of
    100 back-to-back launches, weights rotated (HBM) and one copy (MALL-warm);
    roofline fraction; bit-exactness vs the oracle; the oracle's CPU time."""
    import oracle

    L = Linear(ctx, cfg)
    threads = cpu_threads()
    exact = L.bit_exact(threads)
    flushed = timer.per_launch_us(lambda k, s: L.launch(k, s), LAUNCHES_PER_REPLAY, reps)
    warm = timer.per_launch_us(lambda k, s: L.launch(k, s, copy=0), LAUNCHES_PER_REPLAY, reps)
    us, us_warm = statistics.median(flushed), statistics.median(warm)
    gemm = cfg.batch >= 32
    out = {"shape": f"{cfg.out_feat}x{cfg.in_feat} batch {cfg.batch}", "dtype": {12: "Q4_K", 14: "Q6_K",
                                                                                  8: "Q8_0"}[cfg.ggml_type],
           "us_per_launch_median": round(us, 3), "us_per_launch_min": round(min(flushed), 3),
           "us_per_launch_mall_warm_median": round(us_warm, 3), "replays": reps,
           "launches_per_replay": LAUNCHES_PER_REPLAY,
           "weight_copies_rotated": L.copies, "bit_exact_vs_oracle": exact}
    if gemm:
        ops = 2.0 * cfg.batch * cfg.out_feat * cfg.in_feat
        out.update({"bound": "mfma", "tops": round(ops / us / 1e6, 1), "peak_tops": INT8_MFMA_PEAK_TOPS,
                    "frac": round(ops / us / 1e6 / INT8_MFMA_PEAK_TOPS, 4),
                    "tops_mall_warm": round(ops / us_warm / 1e6, 1),
                    "kernel": "q4k_gemm_pw_kernel (+ act_quant_tiles_kernel)"})
        mc = gemm_counters()
        if mc:
            out["mfma_util_rocprof"] = mc
    else:
        nb = cfg.algorithmic_bytes()
        out.update({"bound": "hbm", "algorithmic_bytes": nb, "gb_s": round(nb / us / 1e3, 1),
                    "peak_gb_s": HBM_PEAK_GBS, "frac": round(nb / us / 1e3 / HBM_PEAK_GBS, 4),
                    "gb_s_mall_warm": round(nb / us_warm / 1e3, 1),
                    "kernel": KERNEL_NAME.get(cfg.ggml_type, "?")})
        rc = read_ceiling(nb, timer, reps)
        out["read_ceiling"] = {"gb_s": rc["gb_s"], "us_per_launch": rc["us_per_launch"],
                               "workgroups": rc["workgroups"]}
        out["frac_of_measured_read"] = round(nb / us / 1e3 / rc["gb_s"], 4)
    if with_cpu:
        sec, n = cpu_time(lambda: oracle.linear_dispatch(cfg.ggml_type, 0, L.x, L.w, cfg.batch, cfg.in_feat,
                                                         cfg.out_feat, threads), cpu_seconds)
        if gemm:
            out["cpu"] = {"tops": round(2.0 * cfg.batch * cfg.out_feat * cfg.in_feat / sec / 1e12, 4),
                          "ms_per_call": round(sec * 1e3, 2), "cores": threads, "runs": n}
        else:
            out["cpu"] = {"gb_s": round(cfg.algorithmic_bytes() / sec / 1e9, 3), "ms_per_call": round(sec * 1e3, 3),
                          "cores": threads, "runs": n}
    L.release()
    return out


E2E_WEIGHT_BYTES = 22 * 24772608 + 53760000  # per step: every layer's Q4_K matrices + the Q6_K head


def e2e_figures(reps, with_cpu):
    """Config 5: inference::run_quantized of the 1.1B Llama (128 prompt ids
    + 64 new tokens) through libvtq_runtime.  tokens_per_s_median is the
    run's positions (prompt + new) per second, median over `reps` runs of
    the default run (each run is what run_quantized returns: tokens and
    receipt digest), which takes the prompt in one batched pass and then
    decodes step by step; the prompt pass is timed alone (a run with no new
    tokens), the decode rate is the new tokens over the rest of the run, and
    the run with every position stepped (run_quantized's loop) is timed
    beside it.  One more run of each fetches every position's logits, which
    with the digests are compared with the oracle's."""
    import numpy as np

    import oracle
    from vtq import runtime, synth

    blob, prompt = synth.e2e_inputs()
    wh = runtime.blake3(blob)
    model = runtime.Model(blob)
    steps = synth.E2E_PROMPT + synth.E2E_NEW

    def timed(n_new, stepwise):
        model.run(prompt[:4], 4, wh, want_logits=False, stepwise=stepwise)  # weights resident, kernels loaded
        model.run(prompt, n_new, wh, want_logits=False, stepwise=stepwise)
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            model.run(prompt, n_new, wh, want_logits=False, stepwise=stepwise)
            ts.append(time.perf_counter() - t0)
        return ts

    times = timed(synth.E2E_NEW, False)
    toks, digest, _ = model.run(prompt, synth.E2E_NEW, wh, want_logits=False)
    digest_v1 = model.digest_v1
    prompt_times = timed(0, False)
    step_times = timed(synth.E2E_NEW, True)
    toks_l, digest_l, logits = model.run(prompt, synth.E2E_NEW, wh)
    dv1_l = model.digest_v1
    toks_s, digest_s, logits_s = model.run(prompt, synth.E2E_NEW, wh, stepwise=True)
    dv1_s = model.digest_v1
    model.close()
    sec, psec, ssec = statistics.median(times), statistics.median(prompt_times), statistics.median(step_times)
    dsec = max(sec - psec, 1e-9)
    out = {"model": "llama-1.1B-shape", **synth.LLAMA_1B1, "prompt": synth.E2E_PROMPT, "new_tokens": synth.E2E_NEW,
           "prompt_mode": "batched prompt pass, then one decode step per new token (vtqrt_run's default)",
           "tokens_per_s_median": round(steps / sec, 2), "tokens_per_s_best": round(steps / min(times), 2),
           "ms_per_run_median": round(sec * 1e3, 3), "ms_per_token_median": round(sec / steps * 1e3, 4),
           "prompt_pass_ms_median": round(psec * 1e3, 3),
           "prompt_tokens_per_s": round(synth.E2E_PROMPT / psec, 1),
           "decode_tokens_per_s": round(synth.E2E_NEW / dsec, 2),
           "decode_gb_s": round(E2E_WEIGHT_BYTES * synth.E2E_NEW / dsec / 1e9, 1),
           "decode_frac": round(E2E_WEIGHT_BYTES * synth.E2E_NEW / dsec / 1e9 / HBM_PEAK_GBS, 4),
           "stepwise_tokens_per_s_median": round(steps / ssec, 2),
           "stepwise_ms_per_run_median": round(ssec * 1e3, 3),
           "stepwise_gb_s": round(E2E_WEIGHT_BYTES * steps / ssec / 1e9, 1),
           "stepwise_frac": round(E2E_WEIGHT_BYTES * steps / ssec / 1e9 / HBM_PEAK_GBS, 4),
           "runs": reps, "receipt_digest": digest,
           "receipt_digest_v1": digest_v1, "weight_bytes_per_step": E2E_WEIGHT_BYTES,
           "ceiling_tokens_per_s": round(HBM_PEAK_GBS * 1e9 / E2E_WEIGHT_BYTES, 1)}
    threads = cpu_threads()
    om = oracle.Model(blob)
    t0 = time.perf_counter()
    o_toks, o_digest, o_logits = om.run(prompt, synth.E2E_NEW, wh, threads=threads)
    cpu_sec = time.perf_counter() - t0
    same = lambda t, d, dv1, lg: bool(  # noqa: E731
        d == o_digest and dv1 == om.digest_v1 and np.array_equal(t, o_toks)
        and np.array_equal(lg.view(np.uint32), o_logits.view(np.uint32)))
    out["bit_exact_vs_oracle"] = bool(digest == o_digest and digest_v1 == om.digest_v1 and np.array_equal(toks, o_toks)
                                      and same(toks_l, digest_l, dv1_l, logits) and same(toks_s, digest_s, dv1_s, logits_s))
    if with_cpu:
        out["cpu"] = {"tokens_per_s": round(steps / cpu_sec, 3), "cores": threads,
                      "sample": f"the same 192-step run on oracle/vtq_oracle_e2e.c ({cpu_sec:.1f} s)"}
    return out, steps, sec, toks


def run_e2e(args):
    """--workload e2e_decode: config 5 alone, as its own JSON line."""
    from vtq import synth

    fig, steps, sec, toks = e2e_figures(max(3, min(args.reps, 20)), not args.no_cpu)
    step_s = sec / steps
    out = {
        "metric": "E2E run tokens/s (config 5: the 128-id prompt in one batched pass, then 64 decode steps; "
                  "positions per second), receipt digest bit-exact",
        "value": round(steps / sec, 2), "unit": "tokens/s", "n_gpus": 1, "steps": steps, "warmup": 1,
        "ms_per_step": round(step_s * 1e3, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8", "data": "synthetic random-init Llama GGUF (vtqs_llama_gguf, seeded) and prompt ids",
        "config": {"workload": "e2e_decode", **fig, "generated_tokens": [int(t) for t in toks[:8]]},
        # the decode steps of the run (new tokens): one weight pass each
        "roofline": {"bound": "hbm", "kernel": "whole decode step", "achieved": fig["decode_gb_s"],
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": fig["decode_frac"],
                     "traffic": None, "bytes_per_step": E2E_WEIGHT_BYTES},
    }
    if "cpu" in fig:
        out["cpu_baseline"] = {"value": fig["cpu"]["tokens_per_s"], "unit": "tokens/s", "cores": fig["cpu"]["cores"],
                               "kind": "port", "sample": fig["cpu"]["sample"]}
    print(json.dumps(out), flush=True)


def main():
    args = parse()
    if args.calibrate_copy_mib:
        calibrate_copy(args.calibrate_copy_mib)
        return
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); the hot path shards by "
              f"output rows with no cross-device arithmetic, but multi-GPU runs are out of scope for this build.",
              file=sys.stderr)
        sys.exit(2)
    if args.workload == "e2e_decode":
        run_e2e(args)
        return

    import torch

    import oracle
    import vtq
    from vtq import synth

    torch.cuda.set_device(torch.device("cuda:0"))
    ctx = vtq.Context(0)
    timer = Timer(eager=args.eager)
    cfgs = [synth.CONFIGS[n] for n in WORKLOADS[args.workload]]
    lins = [Linear(ctx, c, rotate=not args.no_rotate) for c in cfgs]
    threads = cpu_threads()
    bit_exact = all(L.bit_exact(threads) for L in lins)

    def step(k, s):
        for L in lins:
            L.launch(k, s)

    for k in range(args.warmup):
        step(k, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    # the main figure: exactly --steps steps, one replay
    ms_per_step = timer.per_launch_us(step, args.steps, 1)[0] * 1e-3
    # per-kernel launch times: median over --reps replays of 100 launches
    launch_us = [statistics.median(timer.per_launch_us(lambda k, s, L=L: L.launch(k, s), LAUNCHES_PER_REPLAY,
                                                       args.reps)) for L in lins]
    step_bytes = sum(c.algorithmic_bytes() for c in cfgs)
    step_ops = sum(2.0 * c.batch * c.out_feat * c.in_feat for c in cfgs)
    dom = max(range(len(cfgs)), key=lambda i: launch_us[i])  # the dominant (slowest) kernel of the step
    dc = cfgs[dom]
    gemm = dc.batch >= 32
    # GEMV workloads are quoted in GB/s of algorithmic bytes, the prefill GEMM in int8 TOPS
    value = step_ops / (ms_per_step * 1e-3) / 1e12 if gemm else step_bytes / (ms_per_step * 1e-3) / 1e9
    value_unit = "TOPS" if gemm else "GB/s"
    if gemm:
        ops = 2.0 * dc.batch * dc.out_feat * dc.in_feat
        achieved, peak, unit = ops / launch_us[dom] / 1e6, INT8_MFMA_PEAK_TOPS, "TOPS"
    else:
        achieved, peak, unit = dc.algorithmic_bytes() / launch_us[dom] / 1e3, HBM_PEAK_GBS, "GB/s"
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic.json")
    tkey = {"q4k_11008x4096": "q4k_gemv_11008x4096", "q4k_4096x11008": "q4k_gemv_4096x11008",
            "q6k_32000x4096": "q6k_gemv_lm_head", "q8_0_4096x4096": "q8_0_gemv",
            "q4k_gemm_14336x4096_m512": "q4k_gemm_prefill"}[dc.name]
    if os.path.exists(tpath):
        t = json.load(open(tpath)).get(tkey)
        if t:
            traffic = t.get("hbm_bytes_per_launch")
    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": value_unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8" if cfgs[0].ggml_type in (12, 14) else "f32",
        "data": "synthetic (vtq_synth SplitMix64, seeded per config; GGUF blocks as BASELINE.json)",
        "config": {
            "workload": args.workload,
            "shapes": [f"{c.out_feat}x{c.in_feat} batch {c.batch} {vtq.TYPE_NAMES[c.ggml_type]}" for c in cfgs],
            "bytes_per_step": step_bytes,
            "weight_copies_rotated": lins[0].copies,
            "rotated_bytes": sum(L.copies * L.c.weight_bytes() for L in lins),
            "bit_exact_vs_oracle": bit_exact,
        },
        "roofline": {
            "bound": "mfma" if gemm else "hbm",
            "kernel": f"{'q4k_gemm_pw_kernel' if gemm else KERNEL_NAME.get(dc.ggml_type, '?')} "
                      f"{dc.out_feat}x{dc.in_feat} batch {dc.batch} (the step's slowest launch)",
            "achieved": round(achieved, 2),
            "peak": peak,
            "unit": unit,
            "frac": round(achieved / peak, 4),
            "traffic": traffic,
            "launch_us_median": [round(v, 3) for v in launch_us],
            "bytes_per_launch": [c.algorithmic_bytes() for c in cfgs],
            "replays_per_median": args.reps,
            "launches_per_replay": LAUNCHES_PER_REPLAY,
            "pair_frac": round(step_bytes / (sum(launch_us) * 1e-6) / 1e9 / HBM_PEAK_GBS, 4) if not gemm else None,
        },
    }
    ceilings = {"stream": stream_ceiling([L.dw for L in lins], timer, args.reps)}
    if gemm:
        mc = gemm_counters()
        if mc:
            out["roofline"]["mfma_util_rocprof"] = mc
    if not args.no_cpu:
        def cpu_step():
            for L in lins:
                oracle.linear_dispatch(L.c.ggml_type, 0, L.x, L.w, L.c.batch, L.c.in_feat, L.c.out_feat, threads)

        sec, n = cpu_time(cpu_step, args.cpu_seconds, min_runs=10)
        out["cpu_baseline"] = {
            "value": round(step_ops / sec / 1e12 if gemm else step_bytes / sec / 1e9, 4 if gemm else 3),
            "unit": value_unit, "cores": threads, "kind": "port",
            "sample": f"full workload, median of {n} steps after 1 warm-up ({sec * 1e3:.1f} ms/step); "
                      f"oracle/vtq_oracle.c row-parallel integer kernels, grain ceil(out/(4*threads)) as "
                      f"src/ops/quant.rs:1171; threads = online cores capped at {CPU_THREAD_CAP}, the GPU box's "
                      f"CPU share per GPU"}
    for L in lins:
        L.release()
    if not gemm:
        # the same bytes read by a plain read-only stream: the measured ceiling of this access size
        rd = {}
        for c in cfgs:
            rd.setdefault(c.algorithmic_bytes(), read_ceiling(c.algorithmic_bytes(), timer, args.reps))
        ceilings["read"] = list(rd.values())
        rdom = rd[dc.algorithmic_bytes()]
        out["roofline"]["measured_read_ceiling_gb_s"] = rdom["gb_s"]
        out["roofline"]["frac_of_measured_read"] = round(achieved / rdom["gb_s"], 4)
    if args.workload == "q4k_gemv_ffn_pair" and not args.no_configs:
        # every BASELINE configuration in the same run
        figs = {}
        for name in ("q8_0_4096x4096", "q4k_11008x4096", "q4k_4096x11008", "q6k_32000x4096",
                     "q4k_gemm_14336x4096_m512"):
            figs[name] = config_figures(ctx, synth.CONFIGS[name], timer, args.reps, 2.0, not args.no_cpu)
            print(f"bench: {name} done", file=sys.stderr, flush=True)
        fig5, _, _, _ = e2e_figures(20, not args.no_cpu)
        figs["e2e_decode_llama_1b1"] = fig5
        out["configs"] = figs
        out["config"]["bit_exact_vs_oracle_all_configs"] = all(f["bit_exact_vs_oracle"] for f in figs.values())
        g = synth.CONFIGS["q4k_gemm_14336x4096_m512"]
        ceilings["mfma"] = mfma_ceiling(g.batch, g.in_feat, g.out_feat, timer, args.reps)
    elif gemm:
        ceilings["mfma"] = mfma_ceiling(dc.batch, dc.in_feat, dc.out_feat, timer, args.reps)
    out["measured_ceilings"] = ceilings
    ctx.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
