"""Benchmark of welvet's Dense MatVec path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload q4k_4096x14336]

Other workloads (--workload): every packed format at 4096->14336, the
batched prefill GEMM (q4k_prefill_*), MatVecT (<fmt>_t_<in>x<out>) and the
32-layer decode step (decode_32l).

A step is one batch-1 dequant-GEMV launch (y = W x, W packed, x and y f32 in
HBM). Weights are N(0, 0.02) packed by the library's quant.Pack restatement,
x ~ N(0, 1). Consecutive steps rotate over enough uploaded copies of W that
the working set exceeds the 256 MB Infinity Cache, so every step streams W
from HBM. Timing uses HIP events recorded on the stream the kernels run on.

Prints ONE JSON line (the driver's contract) with `roofline` (algorithmic
bytes / average kernel duration against 8 TB/s) and `cpu_baseline` (the CPU
restatement of welvet's Go/SIMD path, timed on this host's cores over a
bounded sample).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MALL_BYTES = 256 << 20

# name: (format, rows=out, cols=in, description)
WORKLOADS = {
    "q4k_4096x14336": ("Q4_K", 14336, 4096, "Q4_K dequant-GEMV 4096->14336 b=1"),
    "q4k_4096x4096": ("Q4_K", 4096, 4096, "Q4_K dequant-GEMV 4096->4096 b=1"),
    "q4k_14336x4096": ("Q4_K", 4096, 14336, "Q4_K dequant-GEMV 14336->4096 b=1"),
    "q4k_4096x6144": ("Q4_K", 6144, 4096, "Q4_K dequant-GEMV 4096->6144 b=1 (a decoder's fused Q|K|V shape)"),
    "q6k_4096x14336": ("Q6_K", 14336, 4096, "Q6_K dequant-GEMV 4096->14336 b=1"),
    "q6k_4096x4096": ("Q6_K", 4096, 4096, "Q6_K dequant-GEMV 4096->4096 b=1"),
    "q6k_14336x4096": ("Q6_K", 4096, 14336, "Q6_K dequant-GEMV 14336->4096 b=1"),
    "q8_0_4096x14336": ("Q8_0", 14336, 4096, "Q8_0 dequant-GEMV 4096->14336 b=1"),
    "q8_0_4096x4096": ("Q8_0", 4096, 4096, "Q8_0 dequant-GEMV 4096->4096 b=1"),
    "q8_0_14336x4096": ("Q8_0", 4096, 14336, "Q8_0 dequant-GEMV 14336->4096 b=1"),
    "q4_0_4096x4096": ("Q4_0", 4096, 4096, "Q4_0 dequant-GEMV 4096->4096 b=1"),
    "ternary_2560x6912": ("NativeTernary", 6912, 2560, "DTypeTernary int8 GEMV 2560->6912 b=1"),
    "ternary_6912x2560": ("NativeTernary", 2560, 6912, "DTypeTernary int8 GEMV 6912->2560 b=1"),
}
# The other narrow weights.Store DTypes on Dense's int8 path, at the ternary pair's shapes.
WORKLOADS.update({
    f"{d.lower()}_{a}x{b}": (f"Native{d}", b, a, f"DType{d} int8 GEMV {a}->{b} b=1")
    for d in ("Int8", "Int4", "Int2", "Binary") for a, b in ((2560, 6912), (6912, 2560))
})
WORKLOADS.update({f"{d.lower()}_14336x4096": (f"Native{d}", 4096, 14336, f"DType{d} int8 GEMV 14336->4096 b=1")
                  for d in ("Int8", "Int4")})
# Every other packed format at the headline shape (row-interleaved where the format has it, else the reference layout).
WORKLOADS.update({
    f"{f.lower()}_4096x14336": (f, 14336, 4096, f"{f} dequant-GEMV 4096->14336 b=1")
    for f in ("Q4_0", "Q4_1", "Q5_0", "Q5_1", "Q2_K", "Q3_K", "Q5_K", "IQ1_S", "IQ2_XXS", "IQ2_XS", "IQ3_XXS",
              "IQ3_S", "IQ4_NL", "IQ4_XS", "TernaryPacked", "BinaryPacked", "AffinePacked")
})
# Batched prefill through the same Dense API (wv_matmul_dev): name -> (format, rows, cols, M, description)
PREFILL = {
    f"q4k_prefill_{i}x{o}_m{m}": ("Q4_K", o, i, m, f"Q4_K prefill GEMM {i}->{o} M={m} (fp16 MFMA)")
    for (i, o) in ((4096, 14336), (14336, 4096)) for m in (32, 128, 512)
}
# The other k-quants, Q8_0 and IQ4_NL on the packed-W MFMA GEMM.
PREFILL.update({
    f"{f.lower().replace('_k', 'k')}_prefill_4096x14336_m{m}": (f, 14336, 4096, m, f"{f} prefill 4096->14336 M={m}")
    for f in ("Q2_K", "Q3_K", "Q5_K", "Q6_K", "Q8_0", "IQ4_NL") for m in (32, 128, 512)
})
# quant.MatVecT (gx += W^T gy, wv_matvec_t_dev) of a Dense layer's weight:
# name -> (format, rows, cols, description); rows = the layer's out, cols = its in.
MATVECT = {
    f"{f.lower()}_t_{i}x{o}": (f, o, i, f"{f} MatVecT of the {i}->{o} weight (gx[{i}] += W^T gy[{o}]) b=1")
    for f in ("Q4_K", "Q6_K", "Q8_0", "Q5_K", "Q3_K", "Q2_K", "Q4_1", "IQ4_NL") for (i, o) in ((4096, 14336), (14336, 4096))
}
# Streaming-read probe (libwv_probe.so): one launch reads MB bytes, one 16 B
# non-temporal load per thread; the 38.5 MB case is the headline GEMV's
# packed bytes, so it gives the single-launch read ceiling of that size.
PROBE = {f"stream_read_{n}": b for n, b in (("38m", 38535168), ("11m", 11010048), ("77m", 77070336))}
MFMA_F16_PEAK_TFLOPS = 2500.0
# 32-layer decoder, hidden 4096, 32/8 heads x 128, SwiGLU 14336, vocab 32000, Q4_K, KV 2048
DECODE = {
    "decode_32l": dict(n_layers=32, hidden=4096, n_heads=32, n_kv_heads=8, head_dim=128, ffn=14336, vocab=32000,
                       kv=2048, distinct_layers=4),
}
# The device prompt forward (wv_decoder_prefill) of the same model: one step
# = one n-token prompt through all layers, its caches written, the next token
# chosen (model/transformer/forward.go:26-90 ForwardTokens).
PROMPT = {f"prompt_32l_{n}": dict(DECODE["decode_32l"], prompt=n) for n in (32, 128, 512, 2047)}
# HBM bytes per decode token: the sum over one token's launches of
# 1.9993 * FETCH_SIZE + WRITE_SIZE (per-launch medians of `rocprofv3 --pmc`
# runs of `bench.py --no-cpu --workload decode_32l`; the launches and
# commands are listed in DECODE_TRAFFIC_SOURCE).
DECODE_TRAFFIC = {"decode_32l": 5_335_726_695}
DECODE_TRAFFIC_SOURCE = "profiles/decode_32l_q4k_kernel_trace.txt"
# Per-dispatch TCC counters of the GEMV kernel (KiB), medians over the timed
# launches of `rocprofv3 --pmc FETCH_SIZE` and `--pmc WRITE_SIZE` runs of
# `bench.py --no-cpu --copy-probe 64 --workload W` (the commands are in the
# PMC_SOURCE files).
# On gfx950 FETCH_SIZE counts one half of the bytes a plain 64 MiB device copy
# reads (32779.5 KiB for 65536 KiB) and WRITE_SIZE all the bytes it writes
# (65536 KiB), so traffic = 1.9993 * FETCH + 1.0 * WRITE, in bytes.
COPY_FETCH_SCALE = 65536.0 / 32779.5
COPY_WRITE_SCALE = 65536.0 / 65536.0
PMC_KIB = {
    "q4k_4096x14336": (18931.62, 56.0),
    "q4k_4096x4096": (5499.5, 16.0),
    "q4k_14336x4096": (19109.5, 16.0),
    "q8_0_4096x4096": (9325.5, 16.0),
    "q8_0_4096x14336": (32456.69, 56.0),
    "q8_0_14336x4096": (32651.12, 16.0),
    "q6k_4096x4096": (7035.0, 16.0),
    "q6k_4096x14336": (24327.5, 56.0),
    "q6k_14336x4096": (24497.5, 16.0),
    "q4_0_4096x4096": (5242.0, 16.0),
    "ternary_2560x6912": (2241.5, 30.84),
    "ternary_6912x2560": (2308.0, 16.0),
}
# Where each PMC_KIB entry comes from: the profile summary of the kernel that
# workload dispatches (k_gemv_q4k serves the headline shape; the other
# k-quant/Q8_0/Q4_0 shapes run k_gemv_rpl; the ternary DType runs k_narrow_i8v).
PMC_SOURCE = {w: f"profiles/{'k_narrow_i8v' if w.startswith('ternary') else 'k_gemv_rpl'}_{w}.txt" for w in PMC_KIB}
PMC_SOURCE["q4k_4096x14336"] = "profiles/k_gemv_q4k_4096x14336.txt"
# HBM bytes per MatVecT step (every kernel of the step: 1.9993 * FETCH_SIZE +
# WRITE_SIZE per dispatch), from the profile summary each workload names.
MATVECT_TRAFFIC = {
    "q4_k_t_4096x14336": 39_431_811,
    "q4_k_t_14336x4096": 39_090_041,
    "q6_k_t_4096x14336": 50_358_658,
    "q6_k_t_14336x4096": 49_952_296,
    "q8_0_t_4096x14336": 68_341_744,
    "q8_0_t_14336x4096": 67_684_058,
}


METRIC = "dequant-GEMV HBM GB/s (% of peak) at 4096->14336 Q4_K b=1; decode tokens/s"


def algorithmic_bytes(packed, rows, cols, ternary):
    """Packed weight bytes in the reference layout (+ the f32 tensor scale of
    the native DTypes) + f32 x + f32 y. Every path reads x as f32: the int8
    path quantizes it on chip."""
    return packed.nbytes + (4 if ternary else 0) + 4 * cols + 4 * rows


def make_weights(fmt, rows, cols, seed=1234):
    rng = np.random.default_rng(seed)
    if fmt == "NativeTernary":
        t = rng.choice(np.array([-1, 0, 1], np.int8), size=rows * cols, p=[0.335, 0.33, 0.335])
        s = np.float32(np.abs(rng.standard_normal(1 << 16).astype(np.float32) * np.float32(0.02)).mean())
        return (t.astype(np.float32) * s).astype(np.float32), rng
    return (rng.standard_normal(rows * cols, dtype=np.float32) * np.float32(0.02)).astype(np.float32), rng


def host_info():
    """nproc, the cores this process may run on, the CPU model, and the threads
    the CPU baseline uses: every core available to the process, capped by the
    host's CPU share for one GPU (OMP_NUM_THREADS, set on the GPU boxes)."""
    nproc = os.cpu_count() or 1
    avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else nproc
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    threads = avail if share <= 0 else max(1, min(avail, share))
    return dict(nproc=nproc, cores_available=avail, cpu_model=model, threads=threads)


def parity_vs(y_gpu, y_ref, exact):
    """GPU output against the CPU restatement's output for the same call: the
    normwise error max|dy| / max|y_ref| and the per-element relative error over
    the elements with |y_ref| > 1e-3 * max|y_ref|."""
    y_gpu = np.asarray(y_gpu, np.float64).reshape(-1)
    y_ref = np.asarray(y_ref, np.float64).reshape(-1)
    scale = float(np.abs(y_ref).max())
    dy = np.abs(y_gpu - y_ref)
    big = np.abs(y_ref) > 1e-3 * scale
    rel = dy[big] / np.abs(y_ref[big])
    out = {"normwise_err": float(dy.max() / scale) if scale > 0 else float(dy.max()),
           "per_element_rel_err_max": float(rel.max()) if rel.size else 0.0,
           "per_element_rel_err_median": float(np.median(rel)) if rel.size else 0.0,
           "elements_compared": int(big.sum()), "outputs": int(y_ref.size)}
    if exact:
        out["bit_exact"] = bool(np.array_equal(y_gpu.astype(np.float32), y_ref.astype(np.float32)))
    return out


def cpu_baseline(packed, x, rows, cols, ternary, nbytes, budget_s, threads, y_gpu=None):
    """CPU restatement of welvet's Go/SIMD Dense path (oracle/), timed here on
    `threads` row-shard threads and on one thread. With `y_gpu`, the result
    also carries the GPU output's parity against the restatement's output."""
    import oracle
    info = host_info()
    op = oracle.Packed(packed.fmt if not ternary else 0, rows, cols, packed.raw, packed.scales, packed.meta,
                       packed.block_weights, packed.mins)

    def timed(fn, budget):
        t0 = time.perf_counter()
        fn()
        one = time.perf_counter() - t0
        n = max(2, min(500, int(budget / max(one, 1e-6))))
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        return n, (time.perf_counter() - t0) / n

    if ternary:
        dt = oracle.DTYPES[packed.name]
        n, sec = timed(lambda: oracle.narrow_i8_forward(dt, packed.raw, np.float32(packed.tensor_scale), rows, cols, x),
                       budget_s)
        par = None
        if y_gpu is not None:
            par = parity_vs(y_gpu, oracle.narrow_i8_forward(dt, packed.raw, np.float32(packed.tensor_scale), rows,
                                                            cols, x)[0], exact=True)
        return dict(value=round(nbytes / sec / 1e9, 3), unit="GB/s", cores=1, kind="port", parity=par,
                    one_thread_value=round(nbytes / sec / 1e9, 3), nproc=info["nproc"],
                    cores_available=info["cores_available"], cpu_model=info["cpu_model"],
                    sample=f"{n} full calls of forwardSIMDNarrowI8 restated (serial, re-expands codes every call, "
                           f"as the reference), {sec * 1e3:.3f} ms/call; the reference path has no threads")
    t0 = time.perf_counter()
    simd = oracle.SimdPath(op)
    cache_s = time.perf_counter() - t0
    y_cpu = simd.matvec(x, nthreads=threads)  # warm
    n, sec = timed(lambda: simd.matvec(x, nthreads=threads), budget_s)
    n1, sec1 = timed(lambda: simd.matvec(x, nthreads=1), budget_s / 3)
    simd.close()
    par = None if y_gpu is None else parity_vs(y_gpu, y_cpu, exact=False)
    return dict(value=round(nbytes / sec / 1e9, 3), unit="GB/s", cores=threads, kind="port", parity=par,
                one_thread_value=round(nbytes / sec1 / 1e9, 3), nproc=info["nproc"],
                cores_available=info["cores_available"], cpu_model=info["cpu_model"],
                sample=f"{n} full GEMVs of the restated fused SIMD path on {threads} row-shard threads "
                       f"({sec * 1e3:.3f} ms/call) and {n1} on one thread ({sec1 * 1e3:.3f} ms/call); "
                       f"Ensure*SIMDCache projection built once in {cache_s:.2f} s, not timed")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--workload", default="q4k_4096x14336",
                    choices=sorted(WORKLOADS) + sorted(PREFILL) + sorted(MATVECT) + sorted(DECODE) + sorted(PROMPT) + sorted(PROBE))
    ap.add_argument("--cpu-budget-s", type=float, default=10.0)
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-decode", action="store_true",
                    help="leave out the decode_32l tokens/s run the headline workload's line carries")
    ap.add_argument("--decode-steps", type=int, default=40)
    ap.add_argument("--traffic-kib", type=float, nargs=2, metavar=("FETCH_KIB", "WRITE_KIB"),
                    help="override the per-dispatch FETCH_SIZE and WRITE_SIZE (KiB) of the GEMV kernel "
                         "(rocprofv3 --pmc of this command) used for roofline.traffic")
    ap.add_argument("--launch", choices=("stream", "graph"), default="stream",
                    help="timed region: K stream launches from the host behind a queue primed with the warmup "
                         "launches (default), or one HIP graph holding the K launches (measured slower per "
                         "launch on MI355X: 12.5 against 9.0 us at the headline shape)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="also run plain device-to-device copies of MIB MiB (torch copy_) for counter calibration")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU (every box here has one MI355X); "
              "the multi-GPU sharding plan is design-only, not run. Use --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    import welvet_amd as wv

    if args.workload in PROBE:
        return probe_main(args, torch)
    if args.workload in PREFILL:
        return prefill_main(args, torch, wv)
    if args.workload in MATVECT:
        return matvect_main(args, torch, wv)
    if args.workload in DECODE:
        print(json.dumps(decode_run(args, wv, args.workload, args.steps, args.warmup, not args.no_cpu)), flush=True)
        return
    if args.workload in PROMPT:
        print(json.dumps(prompt_run(args, wv, args.workload)), flush=True)
        return
    fmt, rows, cols, desc = WORKLOADS[args.workload]
    ternary = fmt in wv.NATIVE
    print(f"[bench] {desc}: packing", file=sys.stderr, flush=True)
    w, rng = make_weights(fmt, rows, cols)
    packed = wv.pack(fmt, w, rows, cols)
    del w
    x = rng.standard_normal(cols, dtype=np.float32)
    nbytes = algorithmic_bytes(packed, rows, cols, ternary)

    wv.init(0)
    copies = max(8, math.ceil(1.25 * MALL_BYTES / packed.nbytes))
    print(f"[bench] uploading {copies} copies ({copies * packed.nbytes / 1e6:.0f} MB)", file=sys.stderr, flush=True)
    blobs = [wv.upload(packed) for _ in range(copies)]
    dev_bytes = blobs[0].info()["device_bytes"]
    stream = torch.cuda.Stream()
    sh = stream.cuda_stream
    tx = torch.from_numpy(x).cuda()
    ty = torch.empty(rows, device="cuda")
    torch.cuda.synchronize()

    # correctness gate on the benchmarked blob (full parity is in tests/)
    blobs[0].matvec_dev(tx.data_ptr(), ty.data_ptr(), 1, sh)
    stream.synchronize()
    assert torch.isfinite(ty).all().item(), "non-finite output"
    y_gate = ty.cpu().numpy().copy()

    # The launch loop calls the C entry point directly (arguments converted
    # once) so that host-side dispatch stays shorter than one kernel.
    launch = wv.lib().wv_matvec_dev
    handles = [b.handle for b in blobs]
    xp, yp = tx.data_ptr(), ty.data_ptr()

    def run(n, first=0):
        rc = 0
        for i in range(n):
            rc |= launch(handles[(first + i) % copies], xp, yp, 1, sh)
        wv.check(rc)

    def timed_stream():
        # The warmup launches are enqueued and e0 is recorded behind them with
        # no synchronisation, so the GPU is busy when the timed region starts
        # and the host stays ahead of it (a launch costs less host time than
        # the kernel takes).
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        stream.synchronize()
        with torch.cuda.stream(stream):
            run(args.warmup)
            e0.record(stream)
            run(args.steps, args.warmup)
            e1.record(stream)
        e1.synchronize()
        return e0.elapsed_time(e1) / args.steps

    def timed_graph():
        # One graph holds exactly the K timed launches (weight copies in
        # rotation); it is replayed once untimed (upload), then the warmup runs
        # as stream launches and the timed replay follows on the primed queue.
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            run(args.steps, args.warmup)
        g.replay()
        stream.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            run(args.warmup)
            e0.record(stream)
            g.replay()
            e1.record(stream)
        e1.synchronize()
        return e0.elapsed_time(e1) / args.steps

    ms_stream = timed_stream()
    ms_graph = timed_graph() if args.launch == "graph" else None
    ms_per_step = ms_graph if ms_graph is not None else ms_stream
    torch.cuda.synchronize()
    value = nbytes / (ms_per_step * 1e-3) / 1e9

    # The timed region is K back-to-back launches of one kernel on one
    # stream; the events bracket them on that stream, so the region's average
    # is the kernel's average duration plus the dispatcher's gap between
    # consecutive launches. profiles/ holds the rocprofv3 --kernel-trace
    # --stats summary of this same command.
    event_us = ms_per_step * 1e3
    traffic = None
    pmc = tuple(args.traffic_kib) if args.traffic_kib else PMC_KIB.get(args.workload)
    if pmc:
        traffic = int(pmc[0] * 1024 * COPY_FETCH_SCALE + pmc[1] * 1024 * COPY_WRITE_SCALE)

    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int32" if ternary else "f32",
        "data": "synthetic: W ~ N(0,0.02) packed by the library's quant.Pack restatement, x ~ N(0,1)",
        "config": {
            "workload": desc, "format": fmt, "in": cols, "out": rows, "batch": 1,
            "weight_copies_rotated": copies, "packed_bytes": int(packed.nbytes),
            "launch": "one HIP graph of the K launches" if ms_graph is not None else "K stream launches",
            "device_bytes": int(dev_bytes), "algorithmic_bytes_per_step": int(nbytes),
        },
        "pct_of_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        "roofline": {
            "bound": "hbm", "achieved": round(value, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(value / HBM_PEAK_GBS, 4), "traffic": traffic,
            "event_us_per_launch": round(event_us, 3),
            "event_us_per_launch_graph": None if ms_graph is None else round(ms_graph * 1e3, 3),
            "traffic_source": PMC_SOURCE.get(args.workload) if pmc and not args.traffic_kib else None,
        },
    }
    if not args.no_cpu:
        info = host_info()
        threads = args.cpu_threads or info["threads"]
        print(f"[bench] cpu baseline ({threads} threads, ~{args.cpu_budget_s:.0f} s)", file=sys.stderr, flush=True)
        result["cpu_baseline"] = cpu_baseline(packed, x, rows, cols, ternary, nbytes, args.cpu_budget_s, threads,
                                              y_gpu=y_gate)
    copy_probe(args, torch, result)
    for b in blobs:
        b.free()
    del blobs
    if args.workload == "q4k_4096x14336" and not args.no_decode:
        # The metric's second half: decode tokens/s of BASELINE config 5.
        d = decode_run(args, wv, "decode_32l", args.decode_steps, 4, with_cpu=not args.no_cpu, prompt_n=512)
        result["decode_tokens_per_s"] = d["value"]
        result["decode_ms_per_token"] = d["ms_per_step"]
        result["decode_roofline"] = d["roofline"]
        result["decode_config"] = d["config"]["workload"]
        if "cpu_baseline" in d:
            result["decode_cpu_baseline"] = d["cpu_baseline"]
        # the device prompt forward of the same model (512 tokens, wv_decoder_prefill)
        if "prompt" in d:
            result["prompt_tokens_per_s"] = d["prompt"]["value"]
            result["prompt_ms"] = d["prompt"]["ms_per_step"]
            result["prompt_roofline"] = d["prompt"]["roofline"]
        elif "prompt_error" in d:
            result["prompt_error"] = d["prompt_error"]
    print(json.dumps(result), flush=True)


def prefill_main(args, torch, wv):
    """One step = Y[M][out] = X[M][in] W^T for the whole token block."""
    fmt, rows, cols, m, desc = PREFILL[args.workload]
    print(f"[bench] {desc}: packing", file=sys.stderr, flush=True)
    w, rng = make_weights(fmt, rows, cols)
    packed = wv.pack(fmt, w, rows, cols)
    del w
    x = rng.standard_normal((m, cols), dtype=np.float32)
    flops = 2.0 * m * rows * cols
    nbytes = packed.nbytes + 4 * m * cols + 4 * m * rows
    wv.init(0)
    copies = max(4, math.ceil(1.25 * MALL_BYTES / packed.nbytes))
    blobs = [wv.upload(packed) for _ in range(copies)]
    stream = torch.cuda.Stream()
    sh = stream.cuda_stream
    tx = torch.from_numpy(x).cuda()
    ty = torch.empty((m, rows), device="cuda")
    torch.cuda.synchronize()
    launch = wv.lib().wv_matmul_dev
    handles = [b.handle for b in blobs]
    xp, yp = tx.data_ptr(), ty.data_ptr()

    def run(n):
        rc = 0
        for i in range(n):
            rc |= launch(handles[i % copies], xp, yp, m, sh)
        wv.check(rc)

    run(1)
    stream.synchronize()
    assert torch.isfinite(ty).all().item(), "non-finite output"
    y_gate = ty.cpu().numpy().copy()
    steps = max(20, min(args.steps, 400))
    warmup = max(5, min(args.warmup, 40))
    # e0 is recorded behind the enqueued warmup launches with no
    # synchronisation, so the GPU is busy when the timed region starts.
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        run(warmup)
        e0.record(stream)
        run(steps)
        e1.record(stream)
    e1.synchronize()
    ms = e0.elapsed_time(e1) / steps
    tflops = flops / (ms * 1e-3) / 1e12
    ai = flops / nbytes
    peak = min(MFMA_F16_PEAK_TFLOPS, ai * HBM_PEAK_GBS / 1e3)
    result = {
        "metric": f"prefill GEMM TFLOP/s, {desc}",
        "value": round(tflops, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(ms, 6), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16 (MFMA, f32 accumulate)",
        "data": "synthetic: W ~ N(0,0.02) packed by the library's quant.Pack restatement, X ~ N(0,1)",
        "config": {"workload": desc, "format": fmt, "in": cols, "out": rows, "M": m,
                   "weight_copies_rotated": copies, "flops_per_step": flops, "algorithmic_bytes_per_step": nbytes},
        "roofline": {"bound": "mfma" if ai * HBM_PEAK_GBS / 1e3 >= MFMA_F16_PEAK_TFLOPS else "hbm",
                     "achieved": round(tflops, 2), "peak": round(peak, 1), "unit": "TFLOP/s",
                     "frac": round(tflops / peak, 4), "traffic": None, "arith_intensity": round(ai, 1),
                     "hbm_gbs": round(nbytes / (ms * 1e-3) / 1e9, 1)},
    }
    if not args.no_cpu:
        import oracle
        info = host_info()
        threads = args.cpu_threads or info["threads"]
        op = oracle.Packed(packed.fmt, rows, cols, packed.raw, packed.scales, packed.meta, packed.block_weights)
        simd = oracle.SimdPath(op)
        simd.matvec(x[0], nthreads=threads)
        n = 0
        ys = []
        t0 = time.perf_counter()
        while n < m and time.perf_counter() - t0 < args.cpu_budget_s:
            ys.append(simd.matvec(x[n], nthreads=threads))
            n += 1
        dt = (time.perf_counter() - t0) / n
        simd.close()
        result["cpu_baseline"] = {
            "value": round(2.0 * rows * cols / dt / 1e12, 5), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "nproc": info["nproc"], "cpu_model": info["cpu_model"],
            "parity": parity_vs(y_gate[:n], np.stack(ys), exact=False),
            "sample": f"{n} of the M row GEMVs the reference runs for this block (restated fused SIMD path, "
                      f"{threads} row-shard threads), {dt * 1e3:.3f} ms per row; parity over those rows"}
    copy_probe(args, torch, result)
    for b in blobs:
        b.free()
    print(json.dumps(result), flush=True)


def probe_main(args, torch):
    """--workload stream_read_*: the read ceiling of one launch of that many
    bytes, timed like the GEMV (HIP events around K back-to-back launches on
    one stream, buffers rotated past the 256 MB Infinity Cache)."""
    import ctypes
    nbytes = PROBE[args.workload]
    lib = ctypes.CDLL(os.path.join(ROOT, "welvet_amd", "libwv_probe.so"))
    lib.wv_probe_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p]
    copies = max(8, math.ceil(1.25 * MALL_BYTES / nbytes))
    bufs = [torch.zeros(nbytes, dtype=torch.uint8, device="cuda") for _ in range(copies)]
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    stream = torch.cuda.Stream()
    sh = stream.cuda_stream
    ptrs = [b.data_ptr() for b in bufs]
    torch.cuda.synchronize()

    def run(n, first=0):
        rc = 0
        for i in range(n):
            rc |= lib.wv_probe_stream_read(ptrs[(first + i) % copies], nbytes, sink.data_ptr(), sh)
        assert rc == 0, "probe launch failed"

    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        run(args.warmup)
        e0.record(stream)
        run(args.steps, args.warmup)
        e1.record(stream)
    e1.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    value = nbytes / (ms * 1e-3) / 1e9
    print(json.dumps({
        "metric": "streaming-read GB/s of one launch (probe)", "value": round(value, 2), "unit": "GB/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 6),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "u8", "data": "zeros",
        "config": {"workload": f"read {nbytes} B per launch, one 16 B non-temporal load per thread, "
                               f"{nbytes // 4096} blocks x 256", "buffers_rotated": copies},
        "roofline": {"bound": "hbm", "achieved": round(value, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(value / HBM_PEAK_GBS, 4), "traffic": None,
                     "event_us_per_launch": round(ms * 1e3, 3)},
    }), flush=True)


def copy_probe(args, torch, result):
    """--copy-probe MIB: plain device-to-device copies of a known size, whose
    FETCH_SIZE / WRITE_SIZE readings scale the kernel's counters to bytes."""
    if not args.copy_probe:
        return
    src = torch.empty(args.copy_probe << 20, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(4):
        dst.copy_(src)
    torch.cuda.synchronize()
    result["copy_probe_bytes"] = args.copy_probe << 20


def matvect_main(args, torch, wv):
    """One step = gx += W^T gy for one weight (the backward GEMV of a Dense layer)."""
    fmt, rows, cols, desc = MATVECT[args.workload]
    print(f"[bench] {desc}: packing", file=sys.stderr, flush=True)
    w, rng = make_weights(fmt, rows, cols)
    packed = wv.pack(fmt, w, rows, cols)
    del w
    gy = rng.standard_normal(rows, dtype=np.float32)
    nbytes = packed.nbytes + 4 * rows + 8 * cols  # weights + gy + gx read and written
    wv.init(0)
    copies = max(8, math.ceil(1.25 * MALL_BYTES / packed.nbytes))
    blobs = [wv.upload(packed) for _ in range(copies)]
    layout = blobs[0].info()["layout"]
    stream = torch.cuda.Stream()
    sh = stream.cuda_stream
    tg = torch.from_numpy(gy).cuda()
    tx = torch.zeros(cols, device="cuda")
    torch.cuda.synchronize()
    launch = wv.lib().wv_matvec_t_dev
    handles = [b.handle for b in blobs]
    gp, xp = tg.data_ptr(), tx.data_ptr()

    def run(n):
        rc = 0
        for i in range(n):
            rc |= launch(handles[i % copies], gp, xp, 1, sh)
        wv.check(rc)

    run(1)
    stream.synchronize()
    assert torch.isfinite(tx).all().item(), "non-finite output"
    gx_gate = tx.cpu().numpy().copy()  # gx after one accumulation into zeros
    steps = max(20, min(args.steps, 1000))
    warmup = max(5, min(args.warmup, 100))
    # e0 is recorded behind the enqueued warmup launches with no
    # synchronisation, so the GPU is busy when the timed region starts.
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        run(warmup)
        e0.record(stream)
        run(steps)
        e1.record(stream)
    e1.synchronize()
    ms = e0.elapsed_time(e1) / steps
    gbs = nbytes / (ms * 1e-3) / 1e9
    result = {
        "metric": f"MatVecT HBM GB/s, {desc}",
        "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(ms, 6), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: W ~ N(0,0.02) packed by the library's quant.Pack restatement, gy ~ N(0,1)",
        "config": {"workload": desc, "format": fmt, "rows": rows, "cols": cols, "layout": layout,
                   "weight_copies_rotated": copies, "algorithmic_bytes_per_step": nbytes},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": MATVECT_TRAFFIC.get(args.workload),
                     "traffic_source": (f"profiles/k_gemvt_rpl_{args.workload}.txt"
                                        if args.workload in MATVECT_TRAFFIC else None),
                     "step_us": round(ms * 1e3, 3)},
    }
    if not args.no_cpu:
        import oracle
        op = oracle.Packed(packed.fmt, rows, cols, packed.raw, packed.scales, packed.meta, packed.block_weights,
                           packed.mins)
        gx_ref = oracle.matvec_t_scalar(op, gy, np.zeros(cols, np.float32))
        gx = np.zeros(cols, np.float32)
        n = 0
        t0 = time.perf_counter()
        while n < 1000 and (n == 0 or time.perf_counter() - t0 < args.cpu_budget_s):
            gx = oracle.matvec_t_scalar(op, gy, gx)
            n += 1
        dt = (time.perf_counter() - t0) / n
        info = host_info()
        result["cpu_baseline"] = {
            "value": round(nbytes / dt / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "nproc": info["nproc"], "cpu_model": info["cpu_model"], "parity": parity_vs(gx_gate, gx_ref, exact=False),
            "sample": f"{n} calls of the restated scalar quant.MatVecT (the reference's only MatVecT path, "
                      f"serial), {dt * 1e3:.3f} ms/call"}
    for b in blobs:
        b.free()
    copy_probe(args, torch, result)
    print(json.dumps(result), flush=True)


def build_decoder(wv, spec, fill_kv):
    """The synthetic 32-layer Q4_K model of BASELINE config 5, resident on the
    device: `distinct_layers` distinct layers of N(0, 0.02) weights cycled over
    the layers, unit norm weights, an N(0, 1) embedding table; with fill_kv,
    KV cache rows 0..kv-2 N(0, 1)."""
    from welvet_amd.decode import Config, Decoder
    kv = spec["kv"]
    cfg = Config(n_layers=spec["n_layers"], hidden=spec["hidden"], n_heads=spec["n_heads"],
                 n_kv_heads=spec["n_kv_heads"], head_dim=spec["head_dim"], ffn=spec["ffn"], vocab=spec["vocab"],
                 max_seq=kv, rope_theta=5e5, rms_eps=1e-5)
    rng = np.random.default_rng(1234)
    shapes = [("q", cfg.q_dim, cfg.hidden), ("k", cfg.kv_dim, cfg.hidden), ("v", cfg.kv_dim, cfg.hidden),
              ("o", cfg.hidden, cfg.q_dim), ("gate", cfg.ffn, cfg.hidden), ("up", cfg.ffn, cfg.hidden),
              ("down", cfg.hidden, cfg.ffn)]
    wv.init(0)
    t0 = time.perf_counter()
    packed_sets = []
    for _ in range(spec["distinct_layers"]):
        ps = []
        for _, r, c in shapes:
            w = (rng.standard_normal(r * c, dtype=np.float32) * np.float32(0.02))
            ps.append(wv.pack("Q4_K", w, r, c))
        packed_sets.append(ps)
        print(f"[bench] packed a layer's weights ({time.perf_counter() - t0:.1f} s)", file=sys.stderr, flush=True)
    wl = rng.standard_normal(cfg.vocab * cfg.hidden, dtype=np.float32) * np.float32(0.02)
    p_lm = wv.pack("Q4_K", wl, cfg.vocab, cfg.hidden)
    del wl
    emb = rng.standard_normal((cfg.vocab, cfg.hidden), dtype=np.float32)
    dec = Decoder(cfg)
    blobs = []
    layer_bytes = sum(p.nbytes for p in packed_sets[0])
    for L in range(cfg.n_layers):
        bl = [wv.upload(p) for p in packed_sets[L % len(packed_sets)]]
        blobs += bl
        dec.set_layer(L, bl, np.ones(cfg.hidden, np.float32), np.ones(cfg.hidden, np.float32))
        if fill_kv:
            k = rng.standard_normal((kv - 1, cfg.kv_dim), dtype=np.float32)
            v = rng.standard_normal((kv - 1, cfg.kv_dim), dtype=np.float32)
            dec.set_kv(L, 0, k, v)
    lm = wv.upload(p_lm)
    dec.set_output(lm, np.ones(cfg.hidden, np.float32), emb)
    print(f"[bench] model resident ({time.perf_counter() - t0:.1f} s)", file=sys.stderr, flush=True)
    return dec, cfg, rng, packed_sets, p_lm, layer_bytes, blobs + [lm]


def decode_run(args, wv, workload, steps, warmup, with_cpu, prompt_n=0):
    """One step = one greedy decode token of the whole 32-layer model at KV
    length 2048. With prompt_n, an n-token prompt forward is timed on the same
    decoder afterwards (its line under "prompt")."""
    spec = DECODE[workload]
    kv = spec["kv"]
    dec, cfg, rng, packed_sets, p_lm, layer_bytes, owned = build_decoder(wv, spec, True)
    dec.use_graph(True)
    pos, tok = kv - 1, 1
    steps = max(8, min(steps, 200))
    warmup = max(2, min(warmup, 10))
    dec.generate(tok, pos, warmup, advance_pos=False)
    t1 = time.perf_counter()
    toks = dec.generate(tok, pos, steps, advance_pos=False)
    dt = time.perf_counter() - t1
    tps = steps / dt
    kv_bytes = cfg.n_layers * 2 * kv * cfg.kv_dim * 4
    step_bytes = cfg.n_layers * layer_bytes + p_lm.nbytes + kv_bytes
    gbs = step_bytes * tps / 1e9
    result = {
        "metric": "decode tokens/s, 32-layer Q4_K decoder (BASELINE config 5)",
        "value": round(tps, 2), "unit": "tokens/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(1e3 / tps, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32 (Q4_K weights, f32 activations and KV cache)",
        "data": (f"synthetic random init: {spec['distinct_layers']} distinct layers of N(0,0.02) Q4_K weights cycled "
                 f"over {cfg.n_layers} resident layer copies, KV cache N(0,1) for {kv - 1} positions, greedy step at "
                 f"position {pos} (KV length {kv}) replayed as one HIP graph per token"),
        "config": {"workload": "32-layer decoder decode step, hidden 4096, 32/8 heads x 128, SwiGLU 14336, "
                               "vocab 32000, RoPE 5e5, RMSNorm eps 1e-5, KV 2048 f32, batch 1",
                   "bytes_per_step": step_bytes, "weight_bytes_per_step": step_bytes - kv_bytes,
                   "kv_bytes_per_step": kv_bytes, "last_tokens": [int(t) for t in toks[-4:]]},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": DECODE_TRAFFIC.get(workload),
                     "traffic_unit": "bytes per token",
                     "traffic_source": DECODE_TRAFFIC_SOURCE if workload in DECODE_TRAFFIC else None},
    }
    if prompt_n:
        try:
            result["prompt"] = time_prompt(dec, cfg, rng, packed_sets, p_lm, prompt_n, 10, 2)
        except Exception as e:  # the decode line stands without it
            result["prompt_error"] = f"{type(e).__name__}: {e}"
    if with_cpu:
        import oracle
        threads = args.cpu_threads or host_info()["threads"]
        per_layer = 0.0
        for p in packed_sets[0]:
            op = oracle.Packed(p.fmt, p.rows, p.cols, p.raw, p.scales, p.meta, p.block_weights)
            simd = oracle.SimdPath(op)
            x = rng.standard_normal(p.cols, dtype=np.float32)
            simd.matvec(x, nthreads=threads)
            n, t2 = 0, time.perf_counter()
            while n < 3:
                simd.matvec(x, nthreads=threads)
                n += 1
            per_layer += (time.perf_counter() - t2) / n
            simd.close()
        from oracle import decode_ref
        kc = rng.standard_normal((kv, cfg.kv_dim))
        vc = rng.standard_normal((kv, cfg.kv_dim))
        q = rng.standard_normal(cfg.q_dim)
        t2 = time.perf_counter()
        decode_ref.attention(q, kc, vc, kv, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim)
        per_layer += time.perf_counter() - t2
        op = oracle.Packed(p_lm.fmt, p_lm.rows, p_lm.cols, p_lm.raw, p_lm.scales, p_lm.meta, p_lm.block_weights)
        simd = oracle.SimdPath(op)
        x = rng.standard_normal(p_lm.cols, dtype=np.float32)
        simd.matvec(x, nthreads=threads)
        t2 = time.perf_counter()
        simd.matvec(x, nthreads=threads)
        lm_t = time.perf_counter() - t2
        simd.close()
        tok_s = cfg.n_layers * per_layer + lm_t
        info = host_info()
        result["cpu_baseline"] = {
            "value": round(1.0 / tok_s, 3), "unit": "tokens/s", "cores": threads, "kind": "port",
            "nproc": info["nproc"], "cpu_model": info["cpu_model"],
            "sample": f"one layer's 7 projections (restated fused SIMD path, {threads} row-shard threads) and its "
                      f"f64 attention over {kv} positions, x{cfg.n_layers} layers, plus the LM head: "
                      f"{tok_s * 1e3:.1f} ms per token"}
    dec.free()
    for b in owned:
        b.free()
    return result


def prompt_run(args, wv, workload):
    """One step = one n-token prompt through the whole 32-layer model on the
    device (wv_decoder_prefill: every layer's projections on the prefill GEMM,
    causal attention over the block, the KV caches written, the last row's
    logits and next token)."""
    spec = PROMPT[workload]
    dec, cfg, rng, packed_sets, p_lm, layer_bytes, owned = build_decoder(wv, spec, False)
    result = time_prompt(dec, cfg, rng, packed_sets, p_lm, spec["prompt"], max(3, min(args.steps, 20)),
                         max(1, min(args.warmup, 3)))
    dec.free()
    for b in owned:
        b.free()
    return result


def time_prompt(dec, cfg, rng, packed_sets, p_lm, n, reps, warmup):
    """Times dec.prefill of one n-token prompt from position 0 (host-timed,
    synchronous calls) and returns its bench line."""
    toks = rng.integers(0, cfg.vocab, n).astype(np.int32)
    for _ in range(warmup):
        dec.prefill(toks, 0)
    t1 = time.perf_counter()
    for _ in range(reps):
        nxt = dec.prefill(toks, 0)
    dt = (time.perf_counter() - t1) / reps
    flops = 2.0 * n * (cfg.n_layers * sum(p.rows * p.cols for p in packed_sets[0]) + p_lm.rows * p_lm.cols / n)
    return {
        "metric": f"prompt forward tokens/s, 32-layer Q4_K decoder, {n}-token prompt",
        "value": round(n / dt, 1), "unit": "tokens/s", "n_gpus": 1, "steps": reps, "warmup": warmup,
        "ms_per_step": round(dt * 1e3, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32 activations, Q4_K weights (fp16 MFMA projections), f32 KV cache",
        "data": "synthetic random init as decode_32l; prompt token ids uniform over the vocabulary",
        "config": {"workload": f"32-layer decoder prompt forward, {n} tokens from position 0, hidden 4096, "
                               "32/8 heads x 128, SwiGLU 14336, vocab 32000", "prompt": n,
                   "next_token": int(nxt)},
        "roofline": {"bound": "mfma", "achieved": round(flops / dt / 1e12, 1), "peak": 2500.0, "unit": "TFLOP/s",
                     "frac": round(flops / dt / 1e12 / 2500.0, 4), "traffic": None,
                     "note": "projection FLOPs only (the LM head for the last row); host-timed, synchronous calls"},
    }


if __name__ == "__main__":
    main()
