#!/usr/bin/env python3
"""Benchmark of the MI355X fp8 weight quantizer and its fused dequant GEMV / GEMM.

Headline (one JSON line on stdout): quantize throughput in GB/s of algorithmic
bytes over the full Llama-3.1-8B-shaped bf16 weight set (32 layers of
q/o [4096, 4096], k/v [1024, 4096], gate/up [14336, 4096], down [4096, 14336];
6,979,321,856 elements; N(0, 0.02) with all-zero rows, bf16 subnormals and
out-of-range values injected), E4M3, per-output-channel absmax scales,
backoff 1. One step = one pass of the quantizer over the whole set, inputs
already resident in HBM. Algorithmic bytes per element: 2 (bf16 in) + 1 (code
out), plus 4 per row (f32 scale).

Also reported (under "extras"): E5M2 over the same set; the full Qwen2.5-32B-shaped
quantize (64 layers, 31.2 G elements, layer 0 compared bit for bit with the
oracle); the f32 [2048, 2048] quantize rotated over 32 copies (compared with the
oracle); the fused dequant GEMV at batch 1 on the [14336, 4096] and
[4096, 14336] shapes rotated past the Infinity Cache, next to a plain read of
the same bytes (the one-launch read yardstick), and on the long rows of the
Qwen2.5-7B and -32B down projections ([3584, 18944], [5120, 27648]); the
skinny GEMM at batch 8 and
64 on Qwen2.5-7B shapes; the M = 1024 fp8 x fp8 GEMM on Qwen2.5-32B shapes, each
beside hipBLASLt (torch._scaled_mm) on the same codes; the fp8 decode step; the
quantizer's stream yardstick (the same 2 bytes in and 1 byte out per element
with no arithmetic, reng_hip_stream_narrow) beside the dominant quantize launch.

The CPU baseline is the oracle (a C restatement of reng-fp8's quantizer: two
passes, an IEEE divide per element, <= 8 threads by reng-fp8's split rule)
timed on this host over layers 0-15 of the same set (about 4 s a run, the
median of 3); those layers are also compared bit for bit with the GPU's codes
and scales.

roofline.traffic is the dominant quantize kernel's HBM bytes per launch from two
rocprofv3 counter passes (FETCH_SIZE, WRITE_SIZE) that the default run starts as
child processes over its own quantize part, scaled by a 1 GiB device copy in
the same pass (--no-traffic, or no rocprofv3: the committed summary instead;
roofline.traffic_source says which).

    python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--no-cpu] [--no-extras] [--no-traffic] [--part ...]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "reciprocating-engine_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

METRIC = "quantize GB/s; fp8 GEMV/GEMM % HBM/MFMA roofline, 8B shapes b1-b64"
import reng_ceiling as RC     # noqa: E402  (the package directory is on sys.path above)

MI355X = RC.HardwareSpec.mi355x()
HBM_PEAK = MI355X.hbm_bw     # 8 TB/s HBM3E, bytes/s
MALL_BYTES = MI355X.sram_bytes   # Infinity Cache: timed buffers rotate over more than this

LLAMA_8B = [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
            ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336)]
QWEN_7B = [("q/o", 3584, 3584), ("k/v", 512, 3584), ("gate/up", 18944, 3584), ("down", 3584, 18944)]
# Batch-1 GEMV rows longer than 16 KB: the Qwen2.5-7B and Qwen2.5-32B down projections [N, K].
LONG_ROWS = [(3584, 18944), (5120, 27648)]
QWEN_32B = [("q", 5120, 5120), ("k", 1024, 5120), ("v", 1024, 5120), ("o", 5120, 5120),
            ("gate", 27648, 5120), ("up", 27648, 5120), ("down", 5120, 27648)]


def log(*a):
    print(*a, file=sys.stderr, flush=True)


quant_bytes = RC.quantize_bytes


def make_bf16(torch, rows, cols, gen, inject=True):
    """N(0, 0.02) bf16 bits (int16 view) with the workload's injections."""
    w = (torch.randn(rows, cols, device="cuda", generator=gen) * 0.02).to(torch.bfloat16).view(torch.int16)
    if inject:
        nz = max(1, rows // 1000)                      # all-zero rows, 0.1%
        w[torch.randint(0, rows, (nz,), device="cuda", generator=gen)] = 0
        flat = w.view(-1)
        n = flat.numel()
        ns = max(1, n // 10000)                        # bf16 subnormals, 0.01%
        idx = torch.randint(0, n, (ns,), device="cuda", generator=gen)
        sub = torch.randint(1, 0x80, (ns,), device="cuda", generator=gen, dtype=torch.int32)
        sign = torch.randint(0, 2, (ns,), device="cuda", generator=gen, dtype=torch.int32) << 15
        flat[idx] = (sub | sign).to(torch.int32).to(torch.int16)
        nb = max(1, n // 1000000)                      # out-of-range finite values, 1 ppm
        idx = torch.randint(0, n, (nb,), device="cuda", generator=gen)
        vals = torch.tensor([1e4, -1e4, 3e38, -3e38], device="cuda").to(torch.bfloat16).view(torch.int16)
        flat[idx] = vals[torch.randint(0, 4, (nb,), device="cuda", generator=gen)]
    return w.view(-1)


class WeightSet:
    def __init__(self, torch, shapes, layers, seed):
        gen = torch.Generator(device="cuda")
        gen.manual_seed(seed)
        self.mats = []   # (layer, name, rows, cols, w, codes, scales, exp_bias)
        for layer in range(layers):
            for name, rows, cols in shapes:
                w = make_bf16(torch, rows, cols, gen)
                codes = torch.empty(rows * cols, dtype=torch.uint8, device="cuda")
                scales = torch.empty(rows, dtype=torch.float32, device="cuda")
                eb = torch.zeros(1, dtype=torch.int32, device="cuda")
                self.mats.append((layer, name, rows, cols, w, codes, scales, eb))
        self.elements = sum(m[2] * m[3] for m in self.mats)
        self.bytes = sum(quant_bytes(m[2], m[3]) for m in self.mats)

    def launches(self):
        """The set as the library launches it: matrices grouped by row width,
        32 per launch (the batch descriptors travel in the kernel arguments)."""
        by_cols = {}
        for m in self.mats:
            by_cols.setdefault(m[3], []).append(m)
        out = []
        for cols in sorted(by_cols):
            ms = by_cols[cols]
            for i in range(0, len(ms), 32):
                chunk = ms[i:i + 32]
                out.append((cols, chunk, sum(quant_bytes(m[2], m[3]) for m in chunk)))
        return out


def time_quantize(torch, R, ws, fmt, steps, warmup):
    launches = ws.launches()
    batches = [[(m[4], m[2], m[3], m[5], m[6], m[7]) for m in chunk] for _, chunk, _ in launches]

    # One event before a step's first launch and one after each launch: the
    # launches run back to back on the stream, so launch i spans the event
    # before it to the event after it (half the markers of a start/end pair
    # per launch, each of which is a packet in the queue between kernels).
    def step(evs=None):
        if evs is not None:
            evs[0].record()
        for i, b in enumerate(batches):
            R.quantize_batch(b, fmt, "pcs", 1.0)
            if evs is not None:
                evs[i + 1].record()

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(len(batches) + 1)] for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(steps):
        step(evs[s])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per_launch = [[e[i].elapsed_time(e[i + 1]) * 1e-3 for i in range(len(batches))] for e in evs]
    step_s = wall / steps
    # The dominant kernel: the configuration carrying the most bytes per step.
    by_cfg = {}
    for i, (cols, _, nbytes) in enumerate(launches):
        d = by_cfg.setdefault(cols, {"bytes": 0, "secs": 0.0, "launches": 0})
        d["bytes"] += nbytes * steps
        d["secs"] += sum(per_launch[s][i] for s in range(steps))
        d["launches"] += steps
    dom_cols = max(by_cfg, key=lambda c: by_cfg[c]["bytes"])
    d = by_cfg[dom_cols]
    return {
        "step_s": step_s,
        "gbps": ws.bytes / step_s / 1e9,
        "kernel_sum_s": sum(sum(p) for p in per_launch) / steps,
        "dominant": {"cols": dom_cols, "bytes_per_launch": d["bytes"] / d["launches"],
                     "secs_per_launch": d["secs"] / d["launches"], "launches_per_step": d["launches"] // steps},
        "configs": {str(c): {"GBps": v["bytes"] / v["secs"] / 1e9, "launches_per_step": v["launches"] // steps}
                    for c, v in by_cfg.items()},
    }


def stream_yardstick(torch, R, ws, quant_gbps):
    """The quantizer's memory stream with no arithmetic (reng_hip_stream_narrow:
    2 bytes in, 1 byte out per element) over the set's 58.7 M-element
    matrices (gate, up, down), rotated and replayed from a hipGraph, beside the
    dominant quantize kernel's rate. Run after the quantize timings: it
    overwrites those matrices' codes."""
    big = [m for m in ws.mats if m[2] * m[3] == 14336 * 4096]
    n = 14336 * 4096
    secs = graph_time(torch, lambda i: R.stream_narrow(big[i % len(big)][4], n, big[i % len(big)][5]), 2 * len(big))
    gbps = 3 * n / secs / 1e9
    return {"matrices": len(big), "us_per_matrix": round(secs * 1e6, 2), "GBps": round(gbps, 1),
            "hbm_frac": round(gbps * 1e9 / HBM_PEAK, 4), "quantize_over_stream": round(quant_gbps / gbps, 3)}


def time_oracle_sample(O, host, fmt, runs=3):
    """The oracle's quantize_with over host [(rows, cols, bf16 bits)] matrix by matrix,
    `runs` times; returns (the first run's results, every run's seconds)."""
    times, refs = [], None
    for _ in range(runs):
        t0 = time.perf_counter()
        out = [O.quantize_with(w, r, c, fmt, "pcs", 1.0, thread_cap=8) for r, c, w in host]
        times.append(time.perf_counter() - t0)
        refs = refs or out
    return refs, times


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown CPU"


def cpu_record(O, host, secs, what):
    """cpu_baseline record: GB/s of algorithmic bytes at the median of the timed runs."""
    elems = sum(r * c for r, c, _ in host)
    nbytes = sum(quant_bytes(r, c) for r, c, _ in host)
    med = sorted(secs)[len(secs) // 2]
    threads = max(O.split(r, c) for r, c, _ in host)
    return {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "runs_s": [round(t, 2) for t in secs],
            "sample": (f"{what} ({len(host)} matrices, {elems} elements), the median of {len(secs)} runs "
                       f"({med:.1f} s), the oracle's C restatement of reng-fp8 quantize_with run matrix by "
                       f"matrix with reng-fp8's split rule (<= 8 threads), {cpu_model()}, nproc {os.cpu_count()}")}


def cpu_baseline_and_parity(torch, O, ws, fmt, layers=16):
    import numpy as np

    sample = [m for m in ws.mats if m[0] < layers]
    host = [(m[2], m[3], m[4].cpu().numpy().view(np.uint16)) for m in sample]
    refs, secs = time_oracle_sample(O, host, fmt)
    mismatched = 0
    for m, ref in zip(sample, refs):
        if not (np.array_equal(m[5].cpu().numpy(), ref.codes)
                and np.array_equal(m[6].cpu().numpy().view(np.uint32), ref.scales.view(np.uint32))
                and int(m[7].item()) == ref.exp_bias):
            mismatched += 1
    return (cpu_record(O, host, secs, f"layers 0-{layers - 1} of the same set"),
            {"matrices": len(sample), "mismatched": mismatched})


def graph_time(torch, fn, n_launch, reps=3):
    """Mean seconds per launch of fn(i) for i in 0..n_launch-1 replayed from a hipGraph."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(n_launch):
            fn(i)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    # Capture on the warm-up stream: per-stream buffers the library keeps (the
    # split-K workspace) already exist there, so nothing allocates inside the capture.
    with torch.cuda.graph(g, stream=s):
        for i in range(n_launch):
            fn(i)
    g.replay()
    torch.cuda.synchronize()
    best = None
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        g.replay()
        b.record()
        torch.cuda.synchronize()
        t = a.elapsed_time(b) * 1e-3 / n_launch
        best = t if best is None else min(best, t)
    return best


def cool_down(torch, secs=20.0):
    """Idle the device before a group of GEMV / GEMM timings. Right after the
    Qwen2.5-32B quantize (minutes of full-rate HBM traffic) every launch over
    HBM runs 3-5% slower for a while — measured on MI355X in one process: the
    read yardstick over [4096, 14336] x 10 copies 9.55 us fresh, 9.83 after that
    part, 9.85 after torch.cuda.empty_cache(), 9.52 after 20 s idle (the GEMV
    10.40 / 10.98 / 10.96 / 10.36 us). Later groups follow seconds of their own
    full-rate work, and the MFMA kernels among them lose 5-10% there while
    their read yardsticks do not (skinny M = 64 gate/up 24.8 against 22.5 us,
    the read 10.7-10.8 us both), so each group starts after 10 s idle. The
    timings are of the device's steady state, the same for each kernel and
    its yardstick."""
    torch.cuda.synchronize()
    time.sleep(secs)
    return secs


SETTLE_S = 0.03   # bench.py --settle-ms


def set_settle(secs):
    global SETTLE_S
    SETTLE_S = secs


def settle(torch, R, bufs, nbytes, secs=None):
    """Keep the device reading buffers for `secs` (back-to-back launches
    replayed from a hipGraph) before timing anything over them. After the
    weights are written and the device idles for a moment, launches over them
    run 3-8% slower for the first ~15 ms of continuous work (measured on MI355X
    over [4096, 14336] x 10 copies: the read yardstick 9.84 against 9.58 us, the
    GEMV 11.1 against 10.33); launches issued one by one from the host (idle
    gaps between them) did not end it. Counter passes of rocprofv3 serialize
    every launch, so they run with --settle-ms 0 (no warm-up reads)."""
    secs = SETTLE_S if secs is None else secs
    if secs <= 0:
        return
    sink = torch.empty(R.stream_read_sink_bytes(), dtype=torch.uint8, device="cuda")
    n = nbytes - nbytes % 1024
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(g, stream=s):
        for i in range(4 * len(bufs)):
            R.stream_read(bufs[i % len(bufs)], n, sink)
    torch.cuda.synchronize()
    t0 = time.time()
    while time.time() - t0 < secs:
        for _ in range(8):
            g.replay()
        torch.cuda.synchronize()


def rotation(nbytes, floor=4, cap=1024):
    n = max(floor, -(-2 * MALL_BYTES // max(1, nbytes)))
    return min(cap, n)


def bench_w8a16(torch, R, gen, M, N, K, fmt="e4m3", read_yardstick=False):
    per = N * K
    copies = rotation(per)
    ws = []
    for _ in range(copies):
        w = (torch.randn(N, K, device="cuda", generator=gen) * 0.02).to(torch.bfloat16).view(torch.int16).view(-1)
        q = R.quantize_with(w, N, K, fmt, "pcs")
        ws.append((q.codes, q.scales))
        del w
    x = torch.randn(M, K, device="cuda", generator=gen).to(torch.bfloat16).view(-1)
    y = torch.empty(M * N, dtype=torch.bfloat16, device="cuda")
    settle(torch, R, [c for c, _ in ws], N * K)
    n_launch = max(2 * copies, 40)
    run = lambda i: R.gemm_w8a16(x, ws[i % copies][0], ws[i % copies][1], M, N, K, fmt, y)
    secs = graph_time(torch, run, n_launch)
    csecs = rsecs = None
    if read_yardstick and 16 < M <= 64 and K % 128 == 0:
        # The same product's copy stream alone (global -> LDS ring, codes and
        # activation, no arithmetic): the floor its data movement sets.
        sink1 = torch.zeros(1, dtype=torch.int32, device="cuda")
        csecs = graph_time(torch, lambda i: R.stream_stage(x, ws[i % copies][0], M, N, K, sink1), n_launch)
    if read_yardstick and (N * K) % 1024 == 0:
        # A plain read of the same code bytes, rotated the same way: the
        # fastest one launch of this size reads on this device.
        sink = torch.empty(R.stream_read_sink_bytes(), dtype=torch.uint8, device="cuda")
        rsecs = graph_time(torch, lambda i: R.stream_read(ws[i % copies][0], N * K, sink), n_launch)
    nbytes = RC.w8a16_bytes(M, N, K)
    flops = 2 * M * N * K
    ceil = RC.w8a16_ceiling(MI355X, M, N, K)   # HBM-bound for M <= 64
    rec = {"M": M, "N": N, "K": K, "us": round(secs * 1e6, 2), "GBps": round(nbytes / secs / 1e9, 1),
           "hbm_frac": round(ceil.fraction(secs), 3), "bound": ceil.bottleneck.value,
           "TFLOPs": round(flops / secs / 1e12, 2), "rotated_copies": copies}
    if csecs is not None:
        rec["copy_yardstick"] = {"us": round(csecs * 1e6, 2), "hbm_frac": round(ceil.fraction(csecs), 3),
                                 "kernel_over_copy": round(secs / csecs, 3)}
    if rsecs is not None:
        rec["read_yardstick"] = {"us": round(rsecs * 1e6, 2), "GBps": round(N * K / rsecs / 1e9, 1),
                                 "hbm_frac": round(N * K / rsecs / HBM_PEAK, 3),
                                 "kernel_over_read": round(secs / rsecs, 3)}
    return rec


def launch_floor(torch, R):
    """The cost of a launch that does (almost) nothing, as these replays see
    it: the read yardstick over 64 KB (its full grid of 8 blocks per CU) from a
    hipGraph. Every timed kernel here pays about this much per launch."""
    bufs = [torch.zeros(64 << 10, dtype=torch.uint8, device="cuda") for _ in range(4)]
    sink = torch.empty(R.stream_read_sink_bytes(), dtype=torch.uint8, device="cuda")
    secs = graph_time(torch, lambda i: R.stream_read(bufs[i % 4], 64 << 10, sink), 40)
    return {"us": round(secs * 1e6, 2), "what": "stream_read over 64 KB, 40 launches replayed from a hipGraph"}


def read_fit(torch, R, sizes_mb=(8, 16, 32, 64, 128, 256)):
    """The read yardstick's launch time over sizes, fitted as a fixed part plus
    bytes over a streaming rate (least squares). The fixed part is what any one
    launch of these sizes pays on top of its bytes; the rate is what a plain
    read sustains once it streams."""
    sink = torch.empty(R.stream_read_sink_bytes(), dtype=torch.uint8, device="cuda")
    pts = []
    for mb in sizes_mb:
        n = mb << 20
        copies = rotation(n)
        bufs = [torch.zeros(n, dtype=torch.uint8, device="cuda") for _ in range(copies)]
        settle(torch, R, bufs, n)
        secs = graph_time(torch, lambda i: R.stream_read(bufs[i % copies], n, sink), max(2 * copies, 40))
        pts.append((n, secs))
        del bufs
    k = len(pts)
    sx = sum(p[0] for p in pts); sy = sum(p[1] for p in pts)
    sxx = sum(p[0] * p[0] for p in pts); sxy = sum(p[0] * p[1] for p in pts)
    slope = (k * sxy - sx * sy) / (k * sxx - sx * sx)
    icpt = (sy - slope * sx) / k
    return {"fixed_us": round(icpt * 1e6, 2), "stream_TBps": round(1e-12 / slope, 2),
            "points": [{"MB": n >> 20, "us": round(s * 1e6, 2)} for n, s in pts],
            "what": "stream_read over rotated buffers, t = fixed + bytes / rate"}


def bench_w8a16_tiles(torch, R, gen):
    """More than 64 activation rows (the tiled bf16-MFMA kernel): M = 256 on the
    reference probe's timed shapes (fp8_probe.rs:359-431), the Llama-3.1-8B
    down projection (long K: stream-K) and M = 1024 on the
    Qwen2.5-32B prefill shapes, each beside a bf16 x bf16 torch.matmul
    (hipBLASLt) over the dequantized weight as the library yardstick."""
    out = []
    for M, N, K in ((256, 4096, 4096), (256, 14336, 4096), (256, 4096, 14336), (1024, 5120, 5120),
                    (1024, 27648, 5120), (1024, 5120, 27648)):
        rec = bench_w8a16(torch, R, gen, M, N, K)
        wb = (torch.randn(N, K, device="cuda", generator=gen) * 0.02).to(torch.bfloat16)
        wt = wb.t().contiguous()
        del wb
        x = torch.randn(M, K, device="cuda", generator=gen).to(torch.bfloat16)
        secs = graph_time(torch, lambda i: torch.matmul(x, wt), 10)
        rec["bf16_matmul_us"] = round(secs * 1e6, 2)
        out.append(rec)
        del wt, x
        torch.cuda.empty_cache()
    return out


def bench_fp8_gemm(torch, R, gen, M, N, K):
    """fp8 x fp8 at M = 1024 over rotated weight copies, each copy quantized
    per output channel and the activation per token; beside it hipBLASLt
    (torch._scaled_mm) on the same codes as the library yardstick."""
    per = N * K
    copies = rotation(per)
    ws = []
    for _ in range(copies):
        w = (torch.randn(N, K, device="cuda", generator=gen) * 0.02).to(torch.bfloat16).view(torch.int16).view(-1)
        ws.append(R.quantize_with(w, N, K, "e4m3", "pcs"))
        del w
    x = torch.randn(M, K, device="cuda", generator=gen).to(torch.bfloat16).view(torch.int16).view(-1)
    qa = R.quantize_with(x, M, K, "e4m3", "pcs")     # per-token activation scales
    out = torch.empty(M * N, dtype=torch.bfloat16, device="cuda")
    settle(torch, R, [q.codes for q in ws], N * K)
    secs = graph_time(torch, lambda i: R.gemm_fp8_scaled(qa.codes, "e4m3", qa.scales, ws[i % copies].codes, "e4m3",
                                                         ws[i % copies].scales, M, N, K, out),
                      max(2 * copies, 10))
    flops = 2 * M * N * K
    ceil = RC.fp8_gemm_ceiling(MI355X, M, N, K)   # fp8 MFMA-bound at M = 1024
    rec = {"M": M, "N": N, "K": K, "us": round(secs * 1e6, 1), "TFLOPs": round(flops / secs / 1e12, 1),
           "mfma_frac": round(ceil.fraction(secs), 3), "bound": ceil.bottleneck.value, "rotated_copies": copies}
    # The same e4m3 codes as OCP float8_e4m3fn (codes 0x00-0x77 mean the same value in both).
    a8 = qa.codes.view(torch.float8_e4m3fn).view(M, K)
    b8 = [q.codes.view(torch.float8_e4m3fn).view(N, K).t() for q in ws]   # [K, N], column-major
    one = torch.ones((), device="cuda")
    # Row-wise scales are this product's own semantics (per token, per output
    # channel); one scale per tensor is the library's plainer form, timed too.
    forms = (("rowwise", lambda q: (qa.scales.view(M, 1), q.scales.view(1, N))),
             ("tensorwise", lambda q: (one, one)))
    for name, scales in forms:
        sc = [scales(q) for q in ws]
        key = "hipblaslt" if name == "rowwise" else "hipblaslt_tensorwise"
        try:
            torch._scaled_mm(a8, b8[0], sc[0][0], sc[0][1], out_dtype=torch.bfloat16)
            torch.cuda.synchronize()
        except (RuntimeError, NotImplementedError) as e:
            rec[key] = {"refused": str(e).splitlines()[0][:160]}
            continue
        hsecs = graph_time(torch, lambda i: torch._scaled_mm(a8, b8[i % copies], sc[i % copies][0],
                                                             sc[i % copies][1], out_dtype=torch.bfloat16),
                           max(2 * copies, 10))
        rec[key] = {"us": round(hsecs * 1e6, 1), "ours_over_hipblaslt": round(secs / hsecs, 3)}
        if name == "rowwise":
            # Both products of copy 0 side by side: the library as an
            # independent check of the whole output at full size.
            R.gemm_fp8_scaled(qa.codes, "e4m3", qa.scales, ws[0].codes, "e4m3", ws[0].scales, M, N, K, out)
            ref = torch._scaled_mm(a8, b8[0], sc[0][0], sc[0][1], out_dtype=torch.bfloat16).float()
            d = out.view(M, N).float() - ref
            rec[key]["rel_l2"] = float(d.norm() / ref.norm())
    return rec


def cpu_f32_quantize(x_host, rows, cols):
    """The oracle's quantize_with (reng-fp8's algorithm, <= 8 threads by its
    split rule) on one f32 matrix: microseconds, the median of 5."""
    import oracle as O

    O.quantize_with(x_host, rows, cols, "e4m3", "pcs", 1.0)
    ts = []
    for _ in range(5):
        t0 = time.perf_counter()
        O.quantize_with(x_host, rows, cols, "e4m3", "pcs", 1.0)
        ts.append(time.perf_counter() - t0)
    return sorted(ts)[2] * 1e6


def bench_f32_quantize(torch, R, gen, rows=2048, cols=2048, cpu=False):
    copies = 32
    mats = []
    for _ in range(copies):
        x = torch.randn(rows, cols, device="cuda", generator=gen) * 0.02
        out = torch.rand(rows, cols, device="cuda", generator=gen) < 0.001   # 0.1% outliers x50
        x = torch.where(out, x * 50.0, x).contiguous().view(-1)
        mats.append((x, torch.empty(rows * cols, dtype=torch.uint8, device="cuda"),
                     torch.empty(rows, dtype=torch.float32, device="cuda")))
    secs = graph_time(torch, lambda i: R.quantize_into(mats[i % copies][0], rows, cols, "e4m3", "pcs", 1.0,
                                                       mats[i % copies][1], mats[i % copies][2]), 2 * copies)
    nbytes = quant_bytes(rows, cols, 4)
    rec = {"rows": rows, "cols": cols, "us": round(secs * 1e6, 2), "GBps": round(nbytes / secs / 1e9, 1),
           "hbm_frac": round(nbytes / secs / HBM_PEAK, 3), "rotated_copies": copies}
    # One launch that only reads the same 16.8 MB input, rotated the same way:
    # what a launch of this size costs before any encode or store.
    sink = torch.empty(R.stream_read_sink_bytes(), dtype=torch.uint8, device="cuda")
    rsecs = graph_time(torch, lambda i: R.stream_read(mats[i % copies][0], rows * cols * 4, sink), 2 * copies)
    rec["read_yardstick"] = {"us": round(rsecs * 1e6, 2), "quantize_over_read": round(secs / rsecs, 3)}
    if cpu:
        import numpy as np

        import oracle as O

        torch.cuda.synchronize()
        ref = O.quantize_with(mats[0][0].cpu().numpy(), rows, cols, "e4m3", "pcs", 1.0)
        rec["parity"] = {"matrices": 1, "mismatched": int(not (
            np.array_equal(mats[0][1].cpu().numpy(), ref.codes)
            and np.array_equal(mats[0][2].cpu().numpy().view(np.uint32), ref.scales.view(np.uint32))))}
        us = cpu_f32_quantize(mats[0][0].cpu().numpy(), rows, cols)
        threads = max(1, min(8, (rows * cols) >> 20, rows))   # reng-fp8's split rule
        rec["cpu_baseline"] = {"us": round(us, 1), "GBps": round(nbytes / us / 1e3, 2), "threads": threads,
                               "kind": "port", "sample": "the first of the rotated matrices"}
    return rec


def bench_qwen32b_quantize(torch, R, fmt="e4m3", steps=3, warmup=1, parity=True):
    """The Qwen2.5-32B-shaped quantize: 64 layers of q/o [5120, 5120], k/v
    [1024, 5120], gate/up [27648, 5120], down [5120, 27648] bf16, N(0, 0.02) with
    the same injections, E4M3 per-channel; inputs resident in HBM. Layer 0's
    seven matrices are compared bit for bit with the oracle."""
    import numpy as np

    t0 = time.perf_counter()
    wq = WeightSet(torch, QWEN_32B, 64, seed=4321)
    torch.cuda.synchronize()
    gen_s = time.perf_counter() - t0
    r = time_quantize(torch, R, wq, fmt, steps, warmup)
    dom = r["dominant"]
    rec = {"workload": "Qwen2.5-32B-shaped bf16 set, 64 layers x (q/o [5120,5120], k/v [1024,5120], "
                       "gate/up [27648,5120], down [5120,27648]), N(0,0.02) with the same injections",
           "format": fmt, "scaling": "pcs", "elements": wq.elements, "algorithmic_bytes_per_step": wq.bytes,
           "steps": steps, "ms_per_step": round(r["step_s"] * 1e3, 3), "GBps": round(r["gbps"], 1),
           "hbm_frac": round(r["gbps"] * 1e9 / HBM_PEAK, 4),
           "per_row_width": {c: {"GBps": round(v["GBps"], 1), "hbm_frac": round(v["GBps"] * 1e9 / HBM_PEAK, 4),
                                 "launches_per_step": v["launches_per_step"]} for c, v in r["configs"].items()},
           "dominant": {"cols": dom["cols"], "mean_launch_us": round(dom["secs_per_launch"] * 1e6, 1),
                        "algorithmic_bytes_per_launch": int(dom["bytes_per_launch"])},
           "generated_in_s": round(gen_s, 1)}
    if parity:
        import oracle as O

        layer0 = [m for m in wq.mats if m[0] == 0]
        host = [(m[2], m[3], m[4].cpu().numpy().view(np.uint16)) for m in layer0]
        refs, secs = time_oracle_sample(O, host, fmt)
        bad = 0
        for m, ref in zip(layer0, refs):
            bad += int(not (np.array_equal(m[5].cpu().numpy(), ref.codes)
                            and np.array_equal(m[6].cpu().numpy().view(np.uint32), ref.scales.view(np.uint32))))
        rec["parity"] = {"matrices": 7, "mismatched": bad, "sample": "layer 0 (q, k, v, o, gate, up, down)"}
        rec["cpu_baseline"] = cpu_record(O, host, secs, "layer 0 of the same set (q, k, v, o, gate, up, down)")
    del wq
    torch.cuda.empty_cache()
    return rec


def bench_host_quantize(torch, R, layers=2, fmt="e4m3"):
    """The host-pointer entry Rust's quantize_with calls (reng_hip_quantize_host:
    8 MB row chunks through three pinned slots and streams, host copies in and
    out on thread pools, uploads, quantizes and downloads overlapped):
    Llama-3.1-8B layers 0..layers-1 from host memory, codes and scales back in
    host memory. GB/s of the same algorithmic bytes, PCIe included (never the
    headline value), beside pinned-memory PCIe copies as the yardstick."""
    import numpy as np

    gen = torch.Generator(device="cuda")
    gen.manual_seed(77)
    mats = []
    for _ in range(layers):
        for name, rows, cols in LLAMA_8B:
            mats.append((rows, cols, make_bf16(torch, rows, cols, gen).cpu().numpy().view(np.uint16)))
    for rows, cols, w in mats:   # one untimed pass: staging buffers, threads, first touches
        R.quantize_host(w, rows, cols, fmt, "pcs")
    runs = []
    for _ in range(3):
        t0 = time.perf_counter()
        for rows, cols, w in mats:
            R.quantize_host(w, rows, cols, fmt, "pcs")
        runs.append(time.perf_counter() - t0)
    secs = sorted(runs)[1]
    nbytes = sum(quant_bytes(r, c) for r, c, _ in mats)
    elems = sum(r * c for r, c, _ in mats)
    return {"matrices": len(mats), "algorithmic_bytes": nbytes, "secs": round(secs, 4),
            "runs_s": [round(t, 4) for t in runs],
            "GBps": round(nbytes / secs / 1e9, 2), "layers": layers, "format": fmt,
            "upload_GBps": round(2 * elems / secs / 1e9, 2), "download_GBps": round(elems / secs / 1e9, 2),
            "pcie": pcie_yardstick(torch),
            "note": "host memory in and out, PCIe and host copies included; the median of 3 passes after one "
                    "untimed pass; "
                    "upload / download = the bf16 weights / the codes over the whole pass"}


def pcie_yardstick(torch, nbytes=256 << 20):
    """Pinned host <-> device copies of nbytes, each direction alone and both at
    once (torch copies on two streams): GB/s, the best of 3."""
    h_in = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
    h_out = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
    d_in = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    d_out = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()

    def best(fn):
        ts = []
        for _ in range(3):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            fn()
            torch.cuda.synchronize()
            ts.append(time.perf_counter() - t0)
        return min(ts)

    def up():
        with torch.cuda.stream(s1):
            d_in.copy_(h_in, non_blocking=True)

    def down():
        with torch.cuda.stream(s2):
            h_out.copy_(d_out, non_blocking=True)

    def both():
        up()
        down()

    tu, td, tb = best(up), best(down), best(both)
    return {"bytes": nbytes, "h2d_GBps": round(nbytes / tu / 1e9, 1), "d2h_GBps": round(nbytes / td / 1e9, 1),
            "both_GBps": round(2 * nbytes / tb / 1e9, 1)}


def bench_decode_step(layers=4, positions=512):
    """The fp8 decode step (reng_model::Fp8Decoder) on Llama-3.1-8B-shaped layers:
    bin/reng-fp8-decode-bench in a child process (its own HIP runtime, its own
    device memory); its JSON line, or an error record if it fails."""
    import subprocess

    exe = os.path.join(ROOT, "reciprocating-engine_amd", "bin", "reng-fp8-decode-bench")
    r = subprocess.run([exe, "--layers", str(layers), "--positions", str(positions)], capture_output=True,
                       text=True, timeout=300)
    if r.returncode != 0:
        return {"error": (r.stderr or r.stdout).strip()[-500:]}
    return json.loads(r.stdout.strip().splitlines()[-1])


def cpu_decode_step(positions=512, steps=3):
    """The CPU baseline beside the decode step: one token of a Llama-3.1-8B-shaped
    layer at position positions - 1, in f32 over f32 weights, as the reference's
    CPU decoder layer computes it (layer_cpu, crates/reng-synapse/src/model.rs:
    2903-3100, in the oracle's restatement: its rms_norm, rope and silu; numpy
    matrix-vector products on the host's BLAS threads), the key / value cache
    holding positions - 1 earlier rows. Returns microseconds per layer-step (the
    median of `steps`)."""
    import numpy as np

    import layer as L

    h, inter, nh, nkv, hd, eps = 4096, 14336, 32, 8, 128, 1e-5
    rng = np.random.default_rng(3)
    mat = lambda rows, cols: rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.02)
    w = {"wq": mat(nh * hd, h), "wk": mat(nkv * hd, h), "wv": mat(nkv * hd, h), "wo": mat(h, nh * hd),
         "wg": mat(inter, h), "wu": mat(inter, h), "wd": mat(h, inter)}
    g1 = np.ones(h, dtype=np.float32)
    g2 = np.ones(h, dtype=np.float32)
    p = positions - 1
    kc = rng.standard_normal((positions, nkv * hd), dtype=np.float32)
    vc = rng.standard_normal((positions, nkv * hd), dtype=np.float32)
    sin, cos = L.rope_caches(positions, hd, 500000.0)
    x = rng.standard_normal((1, h), dtype=np.float32)
    scale = np.float32(hd ** -0.5)

    def step():
        n1 = L.rms_norm(x, g1, eps)
        q = L.rope(n1 @ w["wq"].T, sin[p:p + 1], cos[p:p + 1], hd)
        kc[p] = L.rope(n1 @ w["wk"].T, sin[p:p + 1], cos[p:p + 1], hd)[0]
        vc[p] = (n1 @ w["wv"].T)[0]
        a = np.empty((1, nh * hd), dtype=np.float32)
        for hh in range(nh):
            g = hh // (nh // nkv)
            s_ = (kc[:, g * hd:(g + 1) * hd] @ q[0, hh * hd:(hh + 1) * hd]) * scale
            e = np.exp(s_ - s_.max())
            a[0, hh * hd:(hh + 1) * hd] = (e / e.sum()) @ vc[:, g * hd:(g + 1) * hd]
        hres = x + a @ w["wo"].T
        n2 = L.rms_norm(hres, g2, eps)
        return hres + (L.silu(n2 @ w["wg"].T) * (n2 @ w["wu"].T)) @ w["wd"].T

    step()
    ts = []
    for _ in range(steps):
        t0 = time.perf_counter()
        step()
        ts.append(time.perf_counter() - t0)
    return sorted(ts)[len(ts) // 2] * 1e6


def decode_cpu_record():
    us = cpu_decode_step()
    return {"us_per_layer_step": round(us, 1), "threads": int(os.environ.get("OMP_NUM_THREADS", os.cpu_count())),
            "kind": "port", "sample": "one token at position 511 of a Llama-3.1-8B-shaped layer, f32 weights, "
            "the oracle's restatement of layer_cpu with numpy BLAS matrix-vector products (median of 3)"}


def measure_traffic(fmt):
    """HBM bytes per launch of the dominant quantize kernel, measured now: two rocprofv3 --pmc
    passes (FETCH_SIZE, then WRITE_SIZE, one counter each) over this script's quantize part, run as
    child processes with the 1 GiB device-copy calibration; each counter is scaled by what it reads
    for that copy in the same pass. The dominant kernel is the quantize_rows_fast launch form with
    the most bytes over the pass (rows of 4096 on the Llama-3.1-8B set). Returns (bytes, note);
    bytes is None when rocprofv3 is missing or a pass gives no usable counters."""
    import csv
    import glob
    import shutil
    import signal
    import subprocess
    import tempfile

    exe = shutil.which("rocprofv3")
    if exe is None:
        return None, "rocprofv3 not found"
    tmp = tempfile.mkdtemp(prefix="reng_pmc_", dir="/tmp")
    per_launch = {}
    try:
        for ctr, copy_bytes in (("FETCH_SIZE", 1 << 30), ("WRITE_SIZE", 1 << 30)):
            out = os.path.join(tmp, ctr)
            cmd = [exe, "--pmc", ctr, "--output-format", "csv", "-d", out, "-o", "run", "--", sys.executable,
                   os.path.abspath(__file__), "--part", "quantize", "--steps", "1", "--warmup", "1", "--no-cpu",
                   "--no-extras", "--format", fmt, "--copy-calibration"]
            proc = subprocess.Popen(cmd, cwd="/tmp", env=dict(os.environ, TMPDIR="/tmp"), stdout=subprocess.DEVNULL,
                                    stderr=subprocess.DEVNULL, start_new_session=True)
            try:
                proc.wait(timeout=90)   # a pass takes seconds; a stuck one must not hold the bench
            except subprocess.TimeoutExpired:
                os.killpg(proc.pid, signal.SIGKILL)
                proc.wait()
                return None, f"rocprofv3 --pmc {ctr} timed out"
            # rocprofv3 may end with a signal after the program finished and its files are whole:
            # the counter file decides.
            groups = {}
            for path in glob.glob(os.path.join(out, "**", "*counter_collection.csv"), recursive=True):
                with open(path) as f:
                    for r in csv.DictReader(f):
                        if r.get("Counter_Name") != ctr:
                            continue
                        groups.setdefault((r["Kernel_Name"], r["Grid_Size"]), []).append(float(r["Counter_Value"]))
            copies = [max(v) for (name, _), v in groups.items() if "copyBuffer" in name]
            quant = [v for (name, _), v in groups.items() if "quantize_rows_fast" in name]
            if not copies or not quant or max(copies) <= 0:
                return None, f"rocprofv3 --pmc {ctr}: no calibration copy or quantize kernel in the counters"
            scale = copy_bytes / (max(copies) * 1024)
            dom = max(quant, key=sum)
            per_launch[ctr] = sum(dom) / len(dom) * 1024 * scale
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    return int(per_launch["FETCH_SIZE"] + per_launch["WRITE_SIZE"]), (
        "rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE passes over `bench.py --part quantize` in this run, "
        "each scaled by the counter's reading for a 1 GiB device copy")


def read_traffic(kind):
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3 PMC
    summary (profiles/<kind>_traffic.txt: `fetch_bytes` and `write_bytes` lines,
    already scaled by the copy-kernel calibration), or None."""
    p = os.path.join(ROOT, "profiles", f"{kind}_traffic.txt")
    try:
        vals = {}
        for line in open(p):
            if ":" in line and not line.startswith("#"):
                k, v = line.split(":", 1)
                vals[k.strip()] = v.strip()
        return int(float(vals["fetch_bytes"])) + int(float(vals["write_bytes"]))
    except (OSError, KeyError, ValueError):
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--format", default="e4m3")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extras", action="store_true")
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the two rocprofv3 counter passes that measure the dominant kernel's HBM "
                         "traffic (the committed profiles/quantize_traffic.txt is reported instead)")
    ap.add_argument("--part", default="all",
                    choices=["all", "quantize", "gemv", "skinny", "tiles", "prefill", "f32", "decode", "qwen32b",
                             "host"],
                    help="run one part only (for profiling); the JSON line is printed for 'all' and 'quantize'")
    ap.add_argument("--settle-ms", type=float, default=SETTLE_S * 1e3,
                    help="back-to-back reads of each product's weights before it is timed (0 for counter passes)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="copy 1 GiB device-to-device three times first: a kernel of known traffic that "
                         "scales the rocprofv3 FETCH_SIZE / WRITE_SIZE counters")
    args = ap.parse_args()
    set_settle(args.settle_ms / 1e3)
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: this path runs on a single MI355X and has no multi-GPU "
              f"form here (asked for --gpus {args.gpus}, WORLD_SIZE {world}).", file=sys.stderr)
        sys.exit(2)

    import torch

    import reng_hip as R

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.set_device(0)
    R.lib()
    log("device:", R.device_info())
    if args.copy_calibration:
        src = torch.empty(1 << 28, dtype=torch.int32, device="cuda").random_()
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if args.part not in ("all", "quantize"):
        gen = torch.Generator(device="cuda")
        gen.manual_seed(99)
        if args.part == "gemv":
            out = [bench_w8a16(torch, R, gen, 1, 14336, 4096, read_yardstick=True),
                   bench_w8a16(torch, R, gen, 1, 4096, 14336, read_yardstick=True),
                   {"long_rows": [bench_w8a16(torch, R, gen, 1, N, K, read_yardstick=True) for N, K in LONG_ROWS]},
                   {"launch_floor": launch_floor(torch, R)}, {"read_fit": read_fit(torch, R)}]
        elif args.part == "qwen32b":
            out = [bench_qwen32b_quantize(torch, R, args.format, parity=not args.no_cpu)]
        elif args.part == "host":
            out = [bench_host_quantize(torch, R)]
        elif args.part == "skinny":
            out = [bench_w8a16(torch, R, gen, M, N, K, read_yardstick=True) for M in (8, 64) for _, N, K in QWEN_7B]
        elif args.part == "tiles":
            out = bench_w8a16_tiles(torch, R, gen)
        elif args.part == "prefill":
            out = [bench_fp8_gemm(torch, R, gen, 1024, N, K) for N, K in ((5120, 5120), (1024, 5120),
                                                                           (27648, 5120), (5120, 27648))]
        elif args.part == "decode":
            out = [bench_decode_step()]
            if not args.no_cpu:
                out[0]["cpu_baseline"] = decode_cpu_record()
        else:
            out = [bench_f32_quantize(torch, R, gen, cpu=not args.no_cpu)]
        log(json.dumps(out))
        return
    t0 = time.perf_counter()
    ws = WeightSet(torch, LLAMA_8B, 32, seed=1234)
    torch.cuda.synchronize()
    log(f"Llama-3.1-8B set: {len(ws.mats)} matrices, {ws.elements} elements, {ws.bytes / 1e9:.3f} GB "
        f"algorithmic per pass, generated in {time.perf_counter() - t0:.1f} s")

    set_elements, set_bytes = ws.elements, ws.bytes
    res = time_quantize(torch, R, ws, args.format, args.steps, args.warmup)
    log(f"quantize {args.format}: {res['step_s'] * 1e3:.3f} ms/step, {res['gbps']:.1f} GB/s, "
        f"per config {res['configs']}")
    dom = res["dominant"]
    achieved = dom["bytes_per_launch"] / dom["secs_per_launch"] / 1e9
    traffic, traffic_src = None, None
    if args.part == "all" and not args.no_traffic:
        traffic, why = measure_traffic(args.format)
        traffic_src = why if traffic is not None else None
        log(f"traffic per launch: {traffic} B ({why})")
    if traffic is None:
        traffic = read_traffic("quantize")
        traffic_src = "profiles/quantize_traffic.txt (committed rocprofv3 summary)" if traffic is not None else None
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                "frac": round(achieved * 1e9 / HBM_PEAK, 4), "traffic": traffic, "traffic_source": traffic_src,
                "kernel": f"quantize_rows_fast (bf16, {args.format}, rows of {dom['cols']})",
                "algorithmic_bytes_per_launch": int(dom["bytes_per_launch"]),
                "mean_launch_us": round(dom["secs_per_launch"] * 1e6, 1)}

    cpu, parity = None, None
    if not args.no_cpu:
        import oracle as O

        cpu, parity = cpu_baseline_and_parity(torch, O, ws, args.format)
        log(f"cpu baseline {cpu['value']} GB/s; parity {parity}")

    extras = {}
    if not args.no_extras and args.part == "all":
        other = "e5m2" if args.format == "e4m3" else "e4m3"
        r2 = time_quantize(torch, R, ws, other, args.steps, args.warmup)
        extras[f"quantize_{other}_GBps"] = round(r2["gbps"], 1)
        extras[f"quantize_{other}_ms_per_step"] = round(r2["step_s"] * 1e3, 3)
        extras["quantize_stream_yardstick"] = stream_yardstick(torch, R, ws, achieved)
        log("stream yardstick:", extras["quantize_stream_yardstick"])
        del ws
        torch.cuda.empty_cache()
        gen = torch.Generator(device="cuda")
        gen.manual_seed(99)
        extras["quantize_qwen32b"] = bench_qwen32b_quantize(torch, R, args.format, parity=not args.no_cpu)
        log("qwen32b quantize:", extras["quantize_qwen32b"])
        extras["quantize_host_llama8b"] = bench_host_quantize(torch, R)
        log("host-pointer quantize:", extras["quantize_host_llama8b"])
        extras["f32_2048x2048_quantize"] = bench_f32_quantize(torch, R, gen, cpu=not args.no_cpu)
        extras["cool_down_s"] = cool_down(torch)
        extras["gemv_b1_llama8b"] = [bench_w8a16(torch, R, gen, 1, 14336, 4096, read_yardstick=True),
                                     bench_w8a16(torch, R, gen, 1, 4096, 14336, read_yardstick=True)]
        extras["gemv_b1_long_rows"] = [bench_w8a16(torch, R, gen, 1, N, K, read_yardstick=True) for N, K in LONG_ROWS]
        extras["launch_floor"] = launch_floor(torch, R)
        extras["read_fit"] = read_fit(torch, R)
        log("gemv b1:", extras["gemv_b1_llama8b"], "launch floor:", extras["launch_floor"],
            "read fit:", extras["read_fit"], "long rows:", extras["gemv_b1_long_rows"])
        extras["cool_down_s"] += cool_down(torch, 10.0)
        sk = []
        for M in (8, 64):
            for _, N, K in QWEN_7B:
                sk.append(bench_w8a16(torch, R, gen, M, N, K, read_yardstick=True))
        extras["skinny_qwen7b"] = sk
        log("skinny:", sk)
        torch.cuda.empty_cache()
        extras["cool_down_s"] += cool_down(torch, 10.0)
        extras["w8a16_tiles"] = bench_w8a16_tiles(torch, R, gen)
        log("w8a16 tiles:", extras["w8a16_tiles"])
        extras["cool_down_s"] += cool_down(torch, 10.0)
        extras["prefill_fp8_m1024_qwen32b"] = [bench_fp8_gemm(torch, R, gen, 1024, N, K)
                                               for N, K in ((5120, 5120), (1024, 5120), (27648, 5120),
                                                            (5120, 27648))]
        log("prefill fp8:", extras["prefill_fp8_m1024_qwen32b"])
        torch.cuda.empty_cache()
        extras["decode_step_llama8b"] = bench_decode_step()
        if not args.no_cpu and "error" not in extras["decode_step_llama8b"]:
            extras["decode_step_llama8b"]["cpu_baseline"] = decode_cpu_record()
        log("decode step:", extras["decode_step_llama8b"])

    out = {
        "metric": METRIC,
        "value": round(res["gbps"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(res["step_s"] * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": ("Llama-3.1-8B-shaped bf16 weight set, 32 layers x (q/o [4096,4096], "
                                "k/v [1024,4096], gate/up [14336,4096], down [4096,14336]), N(0,0.02) with "
                                "0.1% zero rows, 0.01% bf16 subnormals, 1 ppm out-of-range values"),
                   "elements": set_elements, "format": args.format, "scaling": "pcs", "backoff": 1.0,
                   "algorithmic_bytes_per_step": set_bytes},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "parity": parity,
        "extras": extras,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
