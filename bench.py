"""Benchmark of the EXL3 packed-weight linear layer on one MI355X.

Headline (the `value`): decode-time GEMV, k=14336 in x n=4096 out at 4 bits per
weight (mul1 codebook), batch 1, fp16 activations N(0,1), fused su/H128/sv --
algorithmic HBM GB/s = (packed trellis + su + sv + x + y bytes) / time.
Also measured in the same run: batch 2/4/8, a seeded 8-request admission trace
(active rows uniform in 1..8 per step), the M=512 prefill GEMM (TFLOP/s), the
k=2048 x n=6144 layer at batch 1, the projection set of the 2B hybrid model at
batch 8 (mixed 3/4/6 bits), the dequant-only sweep over that model's 151 weight
matrices (mixed 2..6 bits) and GET_ROWS of 8 tokens on a vocabulary-head shard.

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
    ap.add_argument("--only-c1", action="store_true", help="the k=2048 x n=6144 batch-1 GEMV only (for profiling)")
    ap.add_argument("--only-rows", type=int, default=0, help="one C3 row count only (for profiling)")
    ap.add_argument("--no-extra", action="store_true", help="skip the C1/C2/C4/GET_ROWS lines")
    ap.add_argument("--calib-copy", action="store_true",
                    help="only time a plain device copy of COPY_BYTES (scales the HBM byte counters)")
    ap.add_argument("--dense-gemm", action="store_true",
                    help="only time the library's dense fp16 GEMM of the M=512 shape (for profiling)")
    ap.add_argument("--stamps", action="store_true",
                    help="GEMV phase stamps from libexl3_hip_stamps.so: the C3 layer at --only-rows rows "
                         "(default 1), or the k=2048 x n=6144 layer with --only-c1")
    return ap.parse_args()


COPY_BYTES = 64 << 20
SETTLE_MS = 25


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


STAMP_PHASES = ["start", "prep barrier passed", "main loops done (all waves)", "partial ready",
                "summing: other splits' words read", "summing: y issued", "summing: exchange cleared"]


def phase_stamps(args):
    """Where one GEMV call's time goes, from the diagnostic twin of the library
    (libexl3_hip_stamps.so: the same kernels plus one 64-bit store of the
    100 MHz s_memrealtime counter by thread 0 of every workgroup at each phase).
    A graph of back-to-back calls over rotated weight copies runs as in the
    timed bench; the stamps of its last call are read back and reported in us
    from the first workgroup's start, p50 / p90 / max over the workgroups of
    each kind: all, a CU's first and second workgroup (blocks below and above
    half the grid when the grid is two per CU), the summing workgroups."""
    import ctypes
    import importlib.util

    import numpy as np
    import torch

    import synth
    spec = importlib.util.spec_from_file_location("exl3_amd_stamps", ROOT / "xiaomi-hexagon-exl3_amd" / "exl3_amd.py")
    amd = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(amd)
    amd._LIB = amd.load(ROOT / "xiaomi-hexagon-exl3_amd" / "libexl3_hip_stamps.so")
    read = amd._LIB.exl3_hip_debug_gemv_stamps
    read.restype, read.argtypes = ctypes.c_int, [ctypes.c_void_p, ctypes.c_size_t]
    k, n, copies = (2048, 6144, 48) if args.only_c1 else (K_IN, N_OUT, COPIES)
    rows = args.only_rows or 1
    dev = torch.device("cuda", 0)
    p = synth.packed_tiles(77, k, n, BITS)
    su, sv = synth.layer_scales(77, k, n)
    rec = torch.from_numpy(synth.pack_records(p, su, sv, BITS).view(np.uint8).copy()).to(dev)
    recs = [rec] + [rec.clone() for _ in range(copies - 1)]
    x = torch.from_numpy(synth.activations(1000 + rows, rows, k)).to(dev)
    y = torch.empty((rows, n), dtype=torch.float16, device=dev)
    ws = amd.new_workspace(k, n, rows)
    turn = [0]

    def fn():
        amd.mul_mat(recs[turn[0] % copies], BITS, k, n, x, codebook=CB, y=y, workspace=ws)
        turn[0] += 1
    ms = graph_time(torch, torch.cuda.current_stream(), fn, 2 * copies)
    torch.cuda.synchronize()
    st = np.zeros((8192, 8), dtype=np.uint64)
    if read(st.ctypes.data, st.size) != 0:
        raise RuntimeError("reading the phase stamps failed")
    used = np.nonzero(st[:, 0])[0]
    if used.size == 0:
        raise RuntimeError(f"rows {rows}: the call ran no GEMV workgroup (above the GEMV's row range?)")
    G, nbs = int(used.max()) + 1, n // 128
    splits = G // nbs
    t0 = int(st[:G, 0].min())
    us = (st[:G].astype(np.int64) - t0) / 100.0   # 100 MHz ticks -> us

    def q(v):
        return [round(float(np.percentile(v, 50)), 2), round(float(np.percentile(v, 90)), 2), round(float(v.max()), 2)]
    summing = np.arange(G) >= (splits - 1) * nbs
    first = np.arange(G) < G // 2
    out = {"workload": f"EXL3 GEMV k={k} x n={n}, 4 bpw, rows {rows}", "workgroups": G, "splits": splits,
           "call_us_stamps_build": round(ms * 1e3, 2), "unit": "us from the first workgroup's start, p50/p90/max",
           "phases": {}}
    for ph, name in enumerate(STAMP_PHASES):
        if ph < 4:
            out["phases"][name] = {"all": q(us[:, ph]), "first_on_cu": q(us[first, ph]),
                                   "second_on_cu": q(us[~first, ph]), "summing": q(us[summing, ph])}
        else:
            out["phases"][name] = {"summing": q(us[summing, ph])}
    print(json.dumps({"gemv_phase_stamps": out}), flush=True)


DENSE_COPIES = 5   # dense fp16 copies of the 4096 x 14336 weight, 117 MB each: 587 MB rotated


def dense_gemm(torch, stream, steps):
    """The M=512 product on dense fp16 weights through torch.matmul (hipBLASLt on
    ROCm): x[512, k] @ W[n, k]^T, rotating through DENSE_COPIES weight copies as
    the EXL3 calls rotate through theirs, so that each call reads its weights
    from HBM.  Not the EXL3 layer (no decode, no rotations, 4x the weight bytes):
    the rate the vendor's tuned library reaches on an fp16 GEMM of this shape on
    the same GPU, beside the EXL3 GEMM's."""
    gen = torch.Generator(device="cuda").manual_seed(11)
    x = torch.randn(512, K_IN, generator=gen, dtype=torch.float16, device="cuda")
    w = [torch.randn(N_OUT, K_IN, generator=gen, dtype=torch.float16, device="cuda") for _ in range(DENSE_COPIES)]
    y = torch.empty(512, N_OUT, dtype=torch.float16, device="cuda")
    turn = [0]

    def fn():
        torch.matmul(x, w[turn[0] % DENSE_COPIES].t(), out=y)
        turn[0] += 1
    for _ in range(2 * DENSE_COPIES):
        fn()
    per_graph = max(DENSE_COPIES * 4, steps // DENSE_COPIES * DENSE_COPIES)
    ms = graph_time(torch, stream, fn, per_graph)
    del w
    return {"call_us": round(ms * 1e3, 1), "tflops": round(2.0 * 512 * K_IN * N_OUT / (ms * 1e-3) / 1e12, 1),
            "weight_copies": DENSE_COPIES}


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
    if args.stamps:
        phase_stamps(args)
        return

    import numpy as np
    import torch

    import conftest
    import synth

    amd = conftest.load_amd()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream()
    if args.only_c1:
        print(json.dumps(extra_configs(amd, torch, np, synth, stream, args, only_c1=True)), flush=True)
        return
    if args.dense_gemm:
        print(json.dumps({"dense_fp16_gemm_m512": dense_gemm(torch, stream, args.steps)}), flush=True)
        return

    # ---- synthetic layer, 18 resident copies
    p = synth.packed_tiles(77, K_IN, N_OUT, BITS)
    su, sv = synth.layer_scales(77, K_IN, N_OUT)
    rec = torch.from_numpy(synth.pack_records(p, su, sv, BITS).view(np.uint8).copy()).to(dev)
    copies = [rec] + [rec.clone() for _ in range(COPIES - 1)]
    del p
    xs = {r: torch.from_numpy(synth.activations(1000 + r, r, K_IN)).to(dev)
          for r in (1, 2, 4, 8, 12, 14, 16, 24, 32, 33, 64, 128)}
    x512 = torch.from_numpy(synth.activations(5000, 512, K_IN)).to(dev)
    row_set = list(range(1, 9)) + [12, 14, 16, 24, 32, 33, 64, 128, 512]
    ys = {r: torch.empty((r, N_OUT), dtype=torch.float16, device=dev) for r in row_set}
    ws = {r: amd.new_workspace(K_IN, N_OUT, r) for r in row_set}
    torch.cuda.synchronize()

    def call(i, rows, x):
        amd.mul_mat(copies[i % COPIES], BITS, K_IN, N_OUT, x, codebook=CB, y=ys[rows], workspace=ws[rows])

    settled = []

    def settle_clocks(rows, x):
        """Once per process, before the first timed configuration: SETTLE_MS of
        untimed layer calls, so that the first measurement does not start from an
        idle GPU's clocks (the later ones follow the earlier measurements)."""
        if settled:
            return
        settled.append(True)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(50):
                call(i, rows, x)
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < SETTLE_MS * 1e-3:
            g.replay()
            torch.cuda.synchronize()

    def timed(rows, x, steps, warmup):
        """Mean time of one layer call over exactly `steps` launches: `warmup`
        untimed launches, then one HIP graph of `steps` launches (rotating through
        the weight copies, free of Python launch cost) replayed once between HIP
        events on the launch stream, synchronized on both sides."""
        for i in range(2):
            call(i, rows, x)
        torch.cuda.synchronize()

        def graph_of(count):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for i in range(count):
                    call(i, rows, x)
            return g

        gw, gt = graph_of(max(1, warmup)), graph_of(steps)
        torch.cuda.synchronize()
        settle_clocks(rows, x)
        gw.replay()
        torch.cuda.synchronize()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        gt.replay()
        stop.record(stream)
        torch.cuda.synchronize()
        return start.elapsed_time(stop) / steps, steps

    if args.only_rows:
        r = args.only_rows
        xr = torch.from_numpy(synth.activations(1000 + r, r, K_IN)).to(dev)
        ys[r] = torch.empty((r, N_OUT), dtype=torch.float16, device=dev)
        ws[r] = amd.new_workspace(K_IN, N_OUT, r)
        msr, n = timed(r, xr, args.steps, args.warmup)
        print(json.dumps({"rows": r, "call_us": round(msr * 1e3, 2), "launches": n,
                          "gbps": round(algo_bytes(K_IN, N_OUT, BITS, r) / (msr * 1e-3) / 1e9, 1)}), flush=True)
        return

    if args.only_gemm:
        msg, n = timed(512, x512, max(36, args.steps // 2), max(18, args.warmup))
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
        for r in (2, 4, 8, 12, 14):   # 12, 14: continuous batching past 8 requests (GEMV up to 14 rows)
            ms, _ = timed(r, xs[r], args.steps, args.warmup)
            gbps = algo_bytes(K_IN, N_OUT, BITS, r) / (ms * 1e-3) / 1e9
            extra[f"gemv_rows{r}"] = {"gbps": round(gbps, 1), "call_us": round(ms * 1e3, 2),
                                      "frac_hbm": round(gbps / HBM_PEAK_GBPS, 4)}
        for r in (16, 24, 32, 33, 64, 128):   # past the GEMV: the GEMM's 32-, 64- and 128-row tiles
            ms, _ = timed(r, xs[r], max(36, args.steps // 2), args.warmup)
            gbps = algo_bytes(K_IN, N_OUT, BITS, r) / (ms * 1e-3) / 1e9
            tflops = 2.0 * r * K_IN * N_OUT / (ms * 1e-3) / 1e12
            extra[f"gemm_rows{r}"] = {"call_us": round(ms * 1e3, 2), "gbps": round(gbps, 1),
                                      "tflops": round(tflops, 1)}
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
        gsteps = max(36, args.steps // 2)
        msg, _ = timed(512, x512, gsteps, max(18, args.warmup))
        flops = 2.0 * 512 * K_IN * N_OUT
        tflops = flops / (msg * 1e-3) / 1e12
        extra["gemm_m512"] = {"tflops": round(tflops, 1), "call_us": round(msg * 1e3, 1),
                              "frac_mfma": round(tflops / MFMA_F16_PEAK_TFLOPS, 4),
                              "dense_fp16_library": dense_gemm(torch, stream, gsteps)}

    if not args.only_gemv and not args.no_extra:
        extra.update(extra_configs(amd, torch, np, synth, stream, args))

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
                     "kernel": "exl3k::gemv_kernel<4,2,0>", "us_per_launch": round(ms1 * 1e3, 3),
                     "algorithmic_bytes": b1},
        "cpu_baseline": cpu,
    }
    line.update(extra)
    print(json.dumps(line), flush=True)


def xs8_slice(xs, r):
    return xs[8][:r]


def graph_time(torch, stream, fn, per_graph, replays=5, warm_ms=10.0):
    """ms of one fn() call: a HIP graph holding per_graph calls (fn may rotate
    through weight copies), replayed untimed for warm_ms (steady clocks after the
    previous configuration), then `replays` times between HIP events; the median
    replay over per_graph."""
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(per_graph):
            fn()
    t0 = time.perf_counter()
    g.replay()
    torch.cuda.synchronize()
    while time.perf_counter() - t0 < warm_ms * 1e-3:
        g.replay()
        torch.cuda.synchronize()
    times = []
    for _ in range(replays):
        s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s_ev.record(stream)
        g.replay()
        e_ev.record(stream)
        torch.cuda.synchronize()
        times.append(s_ev.elapsed_time(e_ev) / per_graph)
    return sorted(times)[len(times) // 2]


def extra_configs(amd, torch, np, synth, stream, args, only_c1=False):
    out = {}
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev)

    def rand_u16(seed, count):
        g.manual_seed(seed)
        return torch.randint(-32768, 32768, (count,), generator=g, device=dev, dtype=torch.int32).to(torch.int16)

    def records(seed, k, n, bits):
        p = rand_u16(seed, k * n * bits // 16)
        su = torch.where(rand_u16(seed + 1, k) < 0, -1.0, 1.0).to(torch.float16)
        sv = (torch.where(rand_u16(seed + 2, n) < 0, -1.0, 1.0) *
              (0.5 + (rand_u16(seed + 3, n).float() + 32768) / 65536) / (k ** 0.5)).to(torch.float16)
        return amd.pack_records(p, su, sv, bits, k, n)

    # C1: k=2048 in x n=6144 out, 4 bits, batch 1 (48 weight copies, 302 MB: past the 256 MB MALL)
    k, n, bits = 2048, 6144, 4
    copies = [records(100 + i, k, n, bits) for i in range(48)]
    x = torch.from_numpy(synth.activations(1100, 1, k)).to(dev)
    y = torch.empty((1, n), dtype=torch.float16, device=dev)
    ws = amd.new_workspace(k, n, 1)
    it = iter(range(1 << 30))
    ms = graph_time(torch, stream, lambda: amd.mul_mat(copies[next(it) % 48], bits, k, n, x, y=y, workspace=ws), 96)
    out["c1_gemv_k2048_n6144_b1"] = {"gbps": round(algo_bytes(k, n, bits, 1) / (ms * 1e-3) / 1e9, 1),
                                     "call_us": round(ms * 1e3, 2), "frac_hbm": round(
                                         algo_bytes(k, n, bits, 1) / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
                                     "note": "graph replay, 48 weight copies"}
    del copies
    if only_c1:
        return out

    # the same 4096 x 14336 weight in the other orientation (k=4096 in x n=14336 out, an MLP's
    # gate/up shape): GEMV at rows 1 and 8, GEMM at M=512 (20 weight copies, 587 MB)
    k, n, bits = 4096, 14336, 4
    copies = [records(200 + i, k, n, bits) for i in range(20)]
    tr = {}
    for r in (1, 8, 512):
        x = torch.from_numpy(synth.activations(1200 + r, r, k)).to(dev)
        y = torch.empty((r, n), dtype=torch.float16, device=dev)
        ws = amd.new_workspace(k, n, r)
        it = iter(range(1 << 30))
        ms = graph_time(torch, stream,
                        lambda: amd.mul_mat(copies[next(it) % 20], bits, k, n, x, y=y, workspace=ws), 40)
        gbps = algo_bytes(k, n, bits, r) / (ms * 1e-3) / 1e9
        tr[f"rows{r}"] = {"call_us": round(ms * 1e3, 2), "gbps": round(gbps, 1),
                          "frac_hbm": round(gbps / HBM_PEAK_GBPS, 4)}
        if r == 512:
            tflops = 2.0 * r * k * n / (ms * 1e-3) / 1e12
            tr[f"rows{r}"].update({"tflops": round(tflops, 1), "frac_mfma": round(tflops / MFMA_F16_PEAK_TFLOPS, 4)})
    out["k4096_n14336"] = tr
    del copies

    # the vocabulary head as a GEMV: k=2048 in x n=151,936 out, 6 bits, batch 1 (a decode
    # step's output layer; 2 weight copies, 480 MB: past the 256 MB MALL)
    k, n, bits = 2048, 151936, 6
    copies = [records(300 + i, k, n, bits) for i in range(2)]
    x = torch.from_numpy(synth.activations(1300, 1, k)).to(dev)
    y = torch.empty((1, n), dtype=torch.float16, device=dev)
    ws = amd.new_workspace(k, n, 1)
    it = iter(range(1 << 30))
    ms = graph_time(torch, stream, lambda: amd.mul_mat(copies[next(it) % 2], bits, k, n, x, y=y, workspace=ws), 20)
    gbps = algo_bytes(k, n, bits, 1) / (ms * 1e-3) / 1e9
    out["head_k2048_n151936_b1"] = {"call_us": round(ms * 1e3, 2), "gbps": round(gbps, 1),
                                    "frac_hbm": round(gbps / HBM_PEAK_GBPS, 4), "bits": bits,
                                    "note": "graph replay, 2 weight copies"}
    del copies

    # C4: projection set of one decoder layer at batch 8, mixed bits, x ~ N(0, sigma 0.5)
    proj = [("q", 2048, 2048, 6), ("k", 2048, 512, 6), ("v", 2048, 512, 6), ("o", 2048, 2048, 6),
            ("gate", 2048, 6144, 4), ("up", 2048, 6144, 4), ("down", 6144, 2048, 3)]
    sets = [[records(400 + 10 * c + i, kk, nn, bb) for i, (_, kk, nn, bb) in enumerate(proj)] for c in range(12)]
    xs = {kk: torch.from_numpy(synth.activations(4000 + kk, 8, kk, sigma=0.5)).to(dev) for kk in (2048, 6144)}
    ys = {nn: torch.empty((8, nn), dtype=torch.float16, device=dev) for nn in (512, 2048, 6144)}
    ws4 = torch.zeros(max(amd.workspace_bytes(2048, 12288, 8), amd.workspace_bytes(6144, 2048, 8),
                          *(amd.workspace_bytes(kk, nn, 8) for _, kk, nn, _ in proj)), dtype=torch.uint8, device=dev)
    set_bytes = sum(algo_bytes(kk, nn, bb, 8) for _, kk, nn, bb in proj)
    ysg = {name: torch.empty((8, nn), dtype=torch.float16, device=dev) for name, _, nn, _ in proj}
    cnt = iter(range(1 << 30))

    def layer_single():
        c = next(cnt) % 12
        for i, (_, kk, nn, bb) in enumerate(proj):
            amd.mul_mat(sets[c][i], bb, kk, nn, xs[kk], y=ys[nn], workspace=ws4)

    def layer_grouped():   # q/k/v and gate/up share their input: one launch each
        c = next(cnt) % 12
        st = sets[c]
        amd.mul_mat_group([(st[0], 2048, ysg["q"]), (st[1], 512, ysg["k"]), (st[2], 512, ysg["v"])], 6, 2048,
                          xs[2048], workspace=ws4)
        amd.mul_mat(st[3], 6, 2048, 2048, xs[2048], y=ysg["o"], workspace=ws4)
        amd.mul_mat_group([(st[4], 6144, ysg["gate"]), (st[5], 6144, ysg["up"])], 4, 2048, xs[2048], workspace=ws4)
        amd.mul_mat(st[6], 3, 6144, 2048, xs[6144], y=ysg["down"], workspace=ws4)
    ms1 = graph_time(torch, stream, layer_single, 24)
    ms = graph_time(torch, stream, layer_grouped, 24)
    out["c4_projection_set_b8"] = {"gbps": round(set_bytes / (ms * 1e-3) / 1e9, 1), "layer_us": round(ms * 1e3, 1),
                                   "frac_hbm": round(set_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
                                   "layer_us_one_call_per_matrix": round(ms1 * 1e3, 1),
                                   "bits": {nm: bb for nm, _, _, bb in proj}, "x_sigma": 0.5,
                                   "note": "graph replay; q/k/v and gate/up each one grouped launch (4 launches "
                                           "per layer); 12 copies of the set (> 256 MB)"}
    del sets

    # C2: dequant-only sweep of the 151 matrices (upstream tile layout -> fp16), bit-exactness in tests
    mats = synth.c2_matrices()
    bits_c2 = synth.c2_bits(mats)
    packed = [rand_u16(9000 + i, k2 * n2 * int(b2) // 16) for i, ((k2, n2), b2) in enumerate(zip(mats, bits_c2))]
    # every matrix decodes into its own region of one 2.9 GB output (as a model's
    # dequantized weight set would), so no write is absorbed by a cache
    offs = [0]
    for k2, n2 in mats:
        offs.append(offs[-1] + ((k2 * n2 + 63) // 64) * 64)
    dst = torch.empty(offs[-1], dtype=torch.int16, device=dev)
    outs = [dst[o: o + k2 * n2].view(k2, n2) for o, (k2, n2) in zip(offs, mats)]

    def sweep_each():
        for (k2, n2), b2, p2, o2 in zip(mats, bits_c2, packed, outs):
            amd.decode(p2, int(b2), k2, n2, codebook=CB, out=o2)
    ms_each = graph_time(torch, stream, sweep_each, 1)
    # one exl3_hip_decode_batch call: the matrices of each rate share launches
    batch = [(p2, int(b2), k2, n2, o2) for (k2, n2), b2, p2, o2 in zip(mats, bits_c2, packed, outs)]

    def sweep():
        amd.decode_batch(batch, codebook=CB)
    ms = graph_time(torch, stream, sweep, 1)
    c2_bytes = sum(k2 * n2 * int(b2) // 8 + 2 * k2 * n2 for (k2, n2), b2 in zip(mats, bits_c2))
    wsum = sum(k2 * n2 for k2, n2 in mats)
    out["c2_dequant_sweep"] = {"gbps": round(c2_bytes / (ms * 1e-3) / 1e9, 1), "sweep_ms": round(ms, 3),
                               "frac_hbm": round(c2_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
                               "matrices": len(mats), "weights": wsum,
                               "mean_bpw": round(float(sum(k2 * n2 * int(b2) for (k2, n2), b2 in zip(mats, bits_c2)) / wsum), 3),
                               "bytes": c2_bytes, "sweep_ms_one_call_per_matrix": round(ms_each, 3),
                               "note": "one exl3_hip_decode_batch call (one launch per rate and up to 32 "
                                       "matrices), each matrix into its own output"}
    del packed, dst, batch, outs

    # GET_ROWS: 8 token ids on a 1/8 vocabulary-head shard (k=2048 hidden, 6 bits)
    k, n, bits = 2048, 151936 // 8 // 128 * 128, 6
    rec = records(777, k, n, bits)
    ids = torch.tensor([5, n // 2, n - 1, 1000, 77, 4096, 18000 % n, 123], dtype=torch.int32, device=dev)
    rows = torch.empty((8, k), dtype=torch.float32, device=dev)
    ms = graph_time(torch, stream, lambda: amd.get_rows(rec, bits, k, n, ids, out=rows), 50)
    rbytes = 8 * (k // 128) * (2048 * bits + 512)
    out["get_rows_head_shard"] = {"call_us": round(ms * 1e3, 2), "tokens": 8, "k": k, "n": n, "bits": bits,
                                  "record_gbps": round(rbytes / (ms * 1e-3) / 1e9, 1)}
    return out


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
    t_one = med(1, 5)

    # decode only (the CPU side of the dequant sweep): the oracle's decode_inner on
    # one MLP matrix, on one thread as the reference runs it, and in column slices
    # on all cores (ctypes releases the GIL during each call)
    from concurrent.futures import ThreadPoolExecutor
    kd, nd, bd = 2048, 6144, 4
    pd = synth.packed_tiles(78, kd, nd, bd)
    dbytes = kd * nd * bd // 8 + 2 * kd * nd
    width = max(16, nd // cores // 16 * 16)
    slices = [(f, min(width, nd - f)) for f in range(0, nd, width)]

    def dec_med(threads, reps):
        def once():
            if threads == 1:
                orc.decode_inner(pd, kd, nd, bd, CB)
            else:
                with ThreadPoolExecutor(threads) as ex:
                    list(ex.map(lambda sl: orc.decode_inner(pd, kd, nd, bd, CB, first=sl[0], count=sl[1]), slices))
        once()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            once()
            ts.append(time.perf_counter() - t0)
        return statistics.median(ts)

    td_all = dec_med(cores, 5)
    td_one = dec_med(1, 5)
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
                      f"{cores} threads (ggml nb partition) and 1 thread, median of 5 after 1 warm-up each; "
                      f"cpu {cpu_model}",
            "ms": round(t_all * 1e3, 2), "single_thread_gbps": round(b1 / t_one / 1e9, 3),
            "single_thread_ms": round(t_one * 1e3, 1),
            "decode": {"sample": f"decode_inner restatement, k=2048 x n=6144 at 4 bits (one MLP matrix of the "
                                 f"dequant sweep), {len(slices)} column slices on {cores} threads; median of 5",
                       "gbps": round(dbytes / td_all / 1e9, 3), "ms": round(td_all * 1e3, 2),
                       "single_thread_gbps": round(dbytes / td_one / 1e9, 3),
                       "single_thread_ms": round(td_one * 1e3, 1)}}


if __name__ == "__main__":
    main()
