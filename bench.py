"""Benchmark of the EXL3 packed-weight linear layer on one MI355X.

Headline (the `value`): decode-time GEMV, k=14336 in x n=4096 out at 4 bits per
weight (mul1 codebook), batch 1, fp16 activations N(0,1), fused su/H128/sv --
algorithmic HBM GB/s = (packed trellis + su + sv + x + y bytes) / time.
Also measured in the same run: batch 2/4/8, a seeded 8-request admission trace
(active rows uniform in 1..8 per step) and the M=512 prefill GEMM (TFLOP/s).

Every step uses the next of 18 distinct copies of the weights (> 512 MB) so the
256 MB Infinity Cache cannot serve repeats.  Inputs are resident in HBM before
the timed region.  Each timed region replays a HIP graph of back-to-back layer
calls (one kernel each at batch <= 8), bracketed by HIP events on the replay
stream, so the per-call time is the kernel's launch-to-launch time without
Python launch cost; the roofline figure divides the algorithmic bytes by it.

CPU baseline: the oracle's restatement of ggml_exl3_mul_mat (the reference CPU
layer, same thread partition) on the same batch-1 layer, timed on this host.
"""
import argparse
import json
import os
import sys
import statistics
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "tests"))

HBM_PEAK_GBPS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2516.6   # dense fp16 MFMA, 256 CU x 4096 flop/clk x 2.4 GHz
K_IN, N_OUT, BITS, CB = 14336, 4096, 4, 2
COPIES = 18


def algo_bytes(k, n, bits, rows):
    return k * n * bits // 8 + 2 * k + 2 * n + 2 * k * rows + 2 * n * rows


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only-gemv", action="store_true", help="headline GEMV only (for profiling)")
    ap.add_argument("--only-gemm", action="store_true", help="M=512 GEMM only (for profiling)")
    ap.add_argument("--calib-copy", action="store_true",
                    help="only time a plain device copy of COPY_BYTES (scales the HBM byte counters)")
    return ap.parse_args()


COPY_BYTES = 64 << 20


def calib_copy(args):
    """Plain device-to-device copy of a known size: its FETCH_SIZE / WRITE_SIZE
    readings per dispatch, divided into COPY_BYTES, give the factors that turn
    those counters into HBM bytes for the GEMV."""
    import torch
    dev = torch.device("cuda", 0)
    src = torch.empty(COPY_BYTES // 4, dtype=torch.int32, device=dev).fill_(7)
    dst = torch.empty_like(src)
    for _ in range(args.warmup):
        dst.copy_(src)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(args.steps):
        dst.copy_(src)
    b.record()
    torch.cuda.synchronize()
    us = a.elapsed_time(b) * 1e3 / args.steps
    print(json.dumps({"calib_copy_bytes": COPY_BYTES, "us_per_copy": round(us, 2),
                      "gbps_read_plus_write": round(2 * COPY_BYTES / (us * 1e-6) / 1e9, 1)}), flush=True)


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}); "
              "the EXL3 layer is not sharded across GPUs here.", file=sys.stderr)
        sys.exit(2)
    if args.calib_copy:
        calib_copy(args)
        return

    import numpy as np
    import torch

    import conftest
    import synth

    amd = conftest.load_amd()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream()

    # ---- synthetic layer, 18 resident copies
    p = synth.packed_tiles(77, K_IN, N_OUT, BITS)
    su, sv = synth.layer_scales(77, K_IN, N_OUT)
    rec = torch.from_numpy(synth.pack_records(p, su, sv, BITS).view(np.uint8).copy()).to(dev)
    copies = [rec] + [rec.clone() for _ in range(COPIES - 1)]
    del p
    xs = {r: torch.from_numpy(synth.activations(1000 + r, r, K_IN)).to(dev) for r in (1, 2, 4, 8)}
    x512 = torch.from_numpy(synth.activations(5000, 512, K_IN)).to(dev)
    row_set = list(range(1, 9)) + [512]
    ys = {r: torch.empty((r, N_OUT), dtype=torch.float16, device=dev) for r in row_set}
    ws = {r: amd.new_workspace(K_IN, N_OUT, r) for r in row_set}
    torch.cuda.synchronize()

    def call(i, rows, x):
        amd.mul_mat(copies[i % COPIES], BITS, K_IN, N_OUT, x, codebook=CB, y=ys[rows], workspace=ws[rows])

    def capture(rows, x):
        """One HIP graph holding COPIES launches, one per weight copy: replays
        measure the kernels back to back, free of Python launch cost."""
        for i in range(2):
            call(i, rows, x)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(COPIES):
                call(i, rows, x)
        torch.cuda.synchronize()
        return g

    def timed(rows, x, steps, warmup):
        """Average time of one layer call over >= steps launches (graph replays,
        HIP events on the replay stream around the whole timed region)."""
        g = capture(rows, x)
        reps = max(1, -(-steps // COPIES))
        for _ in range(max(1, -(-warmup // COPIES))):
            g.replay()
        torch.cuda.synchronize()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(reps):
            g.replay()
        stop.record(stream)
        torch.cuda.synchronize()
        return start.elapsed_time(stop) / (reps * COPIES), reps * COPIES

    if args.only_gemm:
        msg, n = timed(512, x512, max(10, args.steps // 10), max(3, args.warmup // 4))
        print(json.dumps({"gemm_m512_us": round(msg * 1e3, 2), "launches": n,
                          "tflops": round(2.0 * 512 * K_IN * N_OUT / (msg * 1e-3) / 1e12, 1)}), flush=True)
        return

    # ---- headline: batch 1
    ms1, launches1 = timed(1, xs[1], args.steps, args.warmup)
    b1 = algo_bytes(K_IN, N_OUT, BITS, 1)
    value = b1 / (ms1 * 1e-3) / 1e9
    achieved = value   # one kernel per layer call: the step time is the kernel's launch-to-launch time

    extra = {}
    if not args.only_gemv:
        for r in (2, 4, 8):
            ms, _ = timed(r, xs[r], args.steps, args.warmup)
            gbps = algo_bytes(K_IN, N_OUT, BITS, r) / (ms * 1e-3) / 1e9
            extra[f"gemv_rows{r}"] = {"gbps": round(gbps, 1), "kernel_us": round(ms * 1e3, 2),
                                      "frac_hbm": round(gbps / HBM_PEAK_GBPS, 4)}
        # admission trace: 8 requests, active rows uniform in 1..8 per step (seeded), one graph
        trace = (synth.splitmix64(8080, args.steps) % np.uint64(8)).astype(int) + 1
        for i in range(8):
            call(i, i + 1, xs8_slice(xs, i + 1))
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(args.steps):
                call(i, int(trace[i]), xs8_slice(xs, int(trace[i])))
        g.replay()
        torch.cuda.synchronize()
        s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s_ev.record(stream)
        g.replay()
        e_ev.record(stream)
        torch.cuda.synchronize()
        tms = s_ev.elapsed_time(e_ev)
        tbytes = sum(algo_bytes(K_IN, N_OUT, BITS, int(r)) for r in trace)
        extra["gemv_admission_trace"] = {"gbps": round(tbytes / (tms * 1e-3) / 1e9, 1),
                                         "mean_rows": float(np.mean(trace)), "steps": args.steps}
        # prefill GEMM, M = 512
        gsteps = max(10, args.steps // 10)
        msg, _ = timed(512, x512, gsteps, max(3, args.warmup // 4))
        flops = 2.0 * 512 * K_IN * N_OUT
        tflops = flops / (msg * 1e-3) / 1e12
        extra["gemm_m512"] = {"tflops": round(tflops, 1), "call_us": round(msg * 1e3, 1),
                              "frac_mfma": round(tflops / MFMA_F16_PEAK_TFLOPS, 4)}

    traffic = None
    tfile = ROOT / "profiles" / "traffic_gemv_k14336_n4096_b1.json"
    if tfile.exists():
        traffic = json.loads(tfile.read_text()).get("hbm_bytes_per_launch")

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(np, synth)

    line = {
        "metric": "packed-GEMV HBM GB/s (% of peak) at bs 1/8; batch-512 GEMM TFLOPS (% MFMA)",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": launches1,
        "warmup": args.warmup,
        "ms_per_step": round(ms1, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": "EXL3 GEMV k=14336 in x n=4096 out, 4 bpw mul1 trellis, batch 1, fp16 x, "
                               "fused su/H128/sv, 18 rotated weight copies",
                   "k": K_IN, "n": N_OUT, "bits": BITS, "rows": 1, "weight_copies": COPIES},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic,
                     "kernel": "exl3k::gemv_kernel<4,2>", "kernel_us_mean": round(ms1 * 1e3, 3),
                     "algorithmic_bytes": b1},
        "cpu_baseline": cpu,
    }
    line.update(extra)
    print(json.dumps(line), flush=True)


def xs8_slice(xs, r):
    return xs[8][:r]


def cpu_baseline(np, synth):
    from oracle_lib import Oracle
    orc = Oracle()
    p = synth.packed_tiles(77, K_IN, N_OUT, BITS)
    su, sv = synth.layer_scales(77, K_IN, N_OUT)
    rec = synth.pack_records(p, su, sv, BITS)
    x = synth.activations(1001, 1, K_IN)
    cores = len(os.sched_getaffinity(0))
    b1 = algo_bytes(K_IN, N_OUT, BITS, 1)

    def med(threads, reps):
        orc.mul_mat(rec, BITS, CB, K_IN, N_OUT, x, threads=threads)
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            orc.mul_mat(rec, BITS, CB, K_IN, N_OUT, x, threads=threads)
            ts.append(time.perf_counter() - t0)
        return statistics.median(ts)

    t_all = med(cores, 5)
    t_one = med(1, 3)
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(b1 / t_all / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"full k=14336 x n=4096 4-bpw layer, batch 1, oracle restatement of ggml_exl3_mul_mat, "
                      f"{cores} threads (ggml nb partition), median of 5 after 1 warm-up; cpu {cpu_model}",
            "ms": round(t_all * 1e3, 2), "single_thread_gbps": round(b1 / t_one / 1e9, 3),
            "single_thread_ms": round(t_one * 1e3, 1)}


if __name__ == "__main__":
    main()
