"""Benchmark of the quantized linear hot path on one MI355X.

Default workload: one step = the Q4_K decode GEMV
pair of a Llama-7B FFN, 11008x4096 then 4096x11008, batch 1, exact-integer
regime, through libvtq's device-pointer entry point with inputs resident in
HBM.  Weights rotate over enough copies (> 512 MB) that every launch reads
them from HBM, not from the 256 MB MALL.

Prints ONE JSON line (rank 0).  `value` is whole-step throughput in GB/s of
algorithmic bytes (packed weights + fp32 x in + fp32 y out).  `roofline`
describes the dominant kernel: its average launch duration is K back-to-back
launches bracketed by HIP events on the launch stream.  `cpu_baseline` is the pinned C restatement of
the reference path (oracle/, the std-parallel row-parallel integer kernels)
timed on this host's cores on the same inputs.

Other configs (`--config NAME`) are for profiling; the main line is the
default one.
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
KERNEL_NAME = {12: "kquant_rows_kernel<Q4K>", 14: "kquant_rows_kernel<Q6K>", 8: "canon_pc_kernel<DecQ8_0>"}
INT8_MFMA_PEAK_TOPS = 5000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="q4k_gemv_ffn_pair", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-rotate", action="store_true", help="reuse one weight copy (MALL-warm figure)")
    ap.add_argument("--eager", action="store_true", help="time eager launches instead of a replayed HIP graph")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="only run 20 device-to-device copies of this many MiB (HBM counter calibration)")
    return ap.parse_args()


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


def measured_ceilings(dw, step_bytes_per_launch, gemm_shape, steps):
    """Reference points measured on this GPU in the same run (BASELINE.md asks
    for a measured stream peak and MFMA peak beside the published ones):
    * stream: a plain device-to-device copy (torch copy_) of each rotated
      weight copy into one destination, read + write bytes counted: the HBM
      rate of the simplest library kernel on buffers of this size, launch
      floor included;
    * mfma: hipBLASLt's int8 GEMM (torch._int_mm) at the prefill shape, the
      int8 rate a vendor GEMM reaches (it computes a plain int32 product, not
      the reference's Q4_K arithmetic)."""
    import torch

    out = {}
    flat = [w for copies in dw for w in copies]
    dst = torch.empty_like(flat[0])
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    n = max(steps, 20)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for k in range(n):
            dst[: flat[k % len(flat)].numel()].copy_(flat[k % len(flat)])
    g.replay()
    torch.cuda.synchronize()
    e0.record()
    g.replay()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) / n * 1e3
    nbytes = 2 * statistics.mean(w.numel() for w in flat)
    out["stream"] = {"kernel": "device-to-device copy of the rotated weight copies (graph-replayed), read + write",
                     "bytes_per_launch": int(nbytes), "us_per_launch": round(us, 3),
                     "gb_s": round(nbytes / us / 1e3, 1), "frac_of_peak": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)}
    if gemm_shape is not None and hasattr(torch, "_int_mm"):
        m, k_, nn = gemm_shape
        a = torch.randint(-127, 128, (m, k_), dtype=torch.int8, device=flat[0].device)
        b = torch.randint(-127, 128, (k_, nn), dtype=torch.int8, device=flat[0].device)
        try:
            for _ in range(3):
                torch._int_mm(a, b)
            torch.cuda.synchronize()
            e0.record()
            for _ in range(20):
                torch._int_mm(a, b)
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) / 20 * 1e3
            tops = 2.0 * m * k_ * nn / us / 1e6
            out["mfma"] = {"kernel": f"torch._int_mm int8 {m}x{k_} @ {k_}x{nn} -> int32 (hipBLASLt)",
                           "us_per_launch": round(us, 3), "tops": round(tops, 1),
                           "frac_of_peak": round(tops / INT8_MFMA_PEAK_TOPS, 4)}
        except RuntimeError as e:  # not every build ships the int8 GEMM
            out["mfma"] = {"unavailable": str(e)[:120]}
    return out


def cpu_baseline(cfgs, inputs, seconds):
    """The reference path restated in C (oracle), row-parallel on this host's cores."""
    import oracle

    threads = min(len(os.sched_getaffinity(0)), 16)
    total_bytes = sum(c.algorithmic_bytes() for c in cfgs)

    def step():
        for c, (x, w) in zip(cfgs, inputs):
            oracle.linear_dispatch(c.ggml_type, 0, x, w, c.batch, c.in_feat, c.out_feat, threads)

    for _ in range(2):
        step()
    times = []
    t_end = time.perf_counter() + seconds
    while len(times) < 10 or (time.perf_counter() < t_end and len(times) < 200):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {
        "value": round(total_bytes / med / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"full workload, median of {len(times)} steps after 2 warm-ups "
                  f"({med * 1e3:.1f} ms/step); oracle/vtq_oracle.c row-parallel integer kernels, "
                  f"grain ceil(out/(4*threads)) as src/ops/quant.rs:1171",
    }


def run_e2e(args):
    """Config 5: inference::run_quantized of the 1.1B Llama (128 prompt ids +
    64 new tokens) through libvtq_runtime, weights resident in HBM.  value =
    decode steps per second over all 192 steps; the receipt digest and every
    step's logits are checked against the CPU oracle."""
    import numpy as np

    import oracle
    from vtq import runtime, synth

    cfg = synth.LLAMA_1B1
    blob, prompt = synth.e2e_inputs()
    wh = runtime.blake3(blob)
    model = runtime.Model(blob)
    steps = synth.E2E_PROMPT + synth.E2E_NEW
    model.run(prompt[:4], 4, wh, want_logits=False)  # warm-up: weights resident, kernels loaded
    # timed: run_quantized's own outputs (tokens and receipt digest); the
    # per-step logits are fetched in a separate, untimed run for the check
    times = []
    for _ in range(max(1, min(args.steps, 3))):
        t0 = time.perf_counter()
        toks, digest, _ = model.run(prompt, synth.E2E_NEW, wh, want_logits=False)
        times.append(time.perf_counter() - t0)
    toks_l, digest_l, logits = model.run(prompt, synth.E2E_NEW, wh)
    model.close()
    sec = min(times)
    threads = min(len(os.sched_getaffinity(0)), 16)
    om = oracle.Model(blob)
    t0 = time.perf_counter()
    o_toks, o_digest, o_logits = om.run(prompt, synth.E2E_NEW, wh, threads=threads)
    cpu_sec = time.perf_counter() - t0
    bit_exact = (digest == o_digest and digest_l == o_digest and bool(np.array_equal(toks, toks_l))
                 and bool(np.array_equal(logits.view(np.uint32), o_logits.view(np.uint32))))
    w_bytes = 22 * 24772608 + 53760000  # per step: every layer's Q4_K matrices + the Q6_K head
    step_s = sec / steps
    out = {
        "metric": "E2E decode tokens/s (config 5), receipt digest bit-exact",
        "value": round(steps / sec, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": 1,
        "ms_per_step": round(step_s * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic random-init Llama GGUF (vtqs_llama_gguf, seeded) and prompt ids",
        "config": {"workload": "e2e_decode", "model": "llama-1.1B-shape", **cfg, "prompt": synth.E2E_PROMPT,
                   "new_tokens": synth.E2E_NEW, "receipt_digest": digest, "bit_exact_vs_oracle": bit_exact,
                   "generated_tokens": [int(t) for t in toks[:8]]},
        "roofline": {"bound": "hbm", "kernel": "whole decode step", "achieved": round(w_bytes / step_s / 1e9, 2),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(w_bytes / step_s / 1e9 / HBM_PEAK_GBS, 4),
                     "traffic": None, "bytes_per_step": w_bytes,
                     "ceiling_tokens_per_s": round(HBM_PEAK_GBS * 1e9 / w_bytes, 1)},
        "cpu_baseline": {"value": round(steps / cpu_sec, 3), "unit": "tokens/s", "cores": threads, "kind": "port",
                         "sample": f"the same 192-step run on oracle/vtq_oracle_e2e.c ({cpu_sec:.1f} s), linears "
                                   f"row-parallel on {threads} threads"},
    }
    print(json.dumps(out), flush=True)


def main():
    args = parse()
    if args.calibrate_copy_mib:
        calibrate_copy(args.calibrate_copy_mib)
        return
    if args.workload == "e2e_decode" and args.gpus == 1:
        run_e2e(args)
        return
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); the hot path shards by "
              f"output rows with no cross-device arithmetic, but multi-GPU runs are out of scope for this build.",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import vtq
    from vtq import synth

    cfgs = [synth.CONFIGS[n] for n in WORKLOADS[args.workload]]
    inputs = [c.make() for c in cfgs]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    ctx = vtq.Context(0)
    stream = torch.cuda.current_stream()
    sh = stream.cuda_stream

    step_weight_bytes = sum(c.weight_bytes() for c in cfgs)
    copies = 1 if args.no_rotate else max(2, -(-ROTATE_MIN_BYTES // step_weight_bytes))
    dx = [torch.from_numpy(x).to(dev) for x, _ in inputs]
    dw = [[torch.from_numpy(w).to(dev) for _ in range(copies)] for _, w in inputs]
    dy = [torch.empty(c.batch * c.out_feat, dtype=torch.float32, device=dev) for c in cfgs]

    def launch(i, copy, sh):
        c = cfgs[i]
        ctx.linear_device(c.ggml_type, 0, dx[i].data_ptr(), dw[i][copy].data_ptr(), dw[i][copy].numel(),
                          dy[i].data_ptr(), c.batch, c.in_feat, c.out_feat, sh)

    def step(k, sh):
        for i in range(len(cfgs)):
            launch(i, k % copies, sh)

    # parity of what is timed (outside the timed region)
    import oracle

    step(0, sh)
    torch.cuda.synchronize()
    bit_exact = True
    for i, c in enumerate(cfgs):
        x, w = inputs[i]
        want = oracle.linear_dispatch(c.ggml_type, 0, x, w, c.batch, c.in_feat, c.out_feat,
                                      min(len(os.sched_getaffinity(0)), 16))
        bit_exact &= bool(np.array_equal(dy[i].cpu().numpy().view(np.uint32), want.view(np.uint32)))

    for k in range(args.warmup):
        step(k, sh)
    torch.cuda.synchronize()

    def timed_us(body):
        """Average GPU time of one body(k, stream) over args.steps calls, the
        calls issued back to back.  Unless --eager, the calls are captured in
        a HIP graph and replayed, so host launch overhead cannot leave the GPU
        idle between kernels of a few microseconds."""
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        if args.eager:
            torch.cuda.synchronize()
            e0.record(stream)
            for k in range(args.steps):
                body(k, sh)
            e1.record(stream)
        else:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                cs = torch.cuda.current_stream().cuda_stream
                for k in range(args.steps):
                    body(k, cs)
            g.replay()
            torch.cuda.synchronize()
            e0.record(stream)
            g.replay()
            e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / args.steps * 1e3

    # whole-step throughput: K steps back to back
    ms_per_step = timed_us(step) * 1e-3
    # per-kernel average launch duration: K back-to-back launches of each config alone
    launch_us = [timed_us(lambda k, s, i=i: launch(i, k % copies, s)) for i in range(len(cfgs))]

    step_bytes = sum(c.algorithmic_bytes() for c in cfgs)
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    mean_launch_us = statistics.mean(launch_us)
    per_launch_bytes = step_bytes / len(cfgs)
    achieved = per_launch_bytes / (mean_launch_us * 1e-6) / 1e9
    gemm = cfgs[0].batch >= 32
    step_ops = sum(2 * c.batch * c.out_feat * c.in_feat for c in cfgs)

    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(tpath):
        t = json.load(open(tpath)).get(args.workload)
        if t:
            traffic = t.get("hbm_bytes_per_launch")

    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
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
            "weight_copies_rotated": copies,
            "rotated_bytes": copies * step_weight_bytes,
            "bit_exact_vs_oracle": bit_exact,
        },
        "roofline": {
            "bound": "mfma" if gemm else "hbm",
            "kernel": "q4k_gemm_kernel (+ act_quant_tiles_kernel)" if gemm else KERNEL_NAME.get(cfgs[0].ggml_type, "?"),
            "achieved": round(step_ops / len(cfgs) / (mean_launch_us * 1e-6) / 1e12, 2) if gemm else round(achieved, 2),
            "peak": INT8_MFMA_PEAK_TOPS if gemm else HBM_PEAK_GBS,
            "unit": "TOPS" if gemm else "GB/s",
            "frac": round(step_ops / len(cfgs) / (mean_launch_us * 1e-6) / 1e12 / INT8_MFMA_PEAK_TOPS, 4) if gemm
            else round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "launch_us_mean": [round(v, 3) for v in launch_us],
            "bytes_per_launch": [c.algorithmic_bytes() for c in cfgs],
        },
    }
    out["measured_ceilings"] = measured_ceilings(
        dw, step_bytes / len(cfgs), (cfgs[0].batch, cfgs[0].in_feat, cfgs[0].out_feat) if gemm else None, args.steps)
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(cfgs, inputs, args.cpu_seconds)
    ctx.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
