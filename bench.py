"""Benchmark: effective TFLOP/s of block-sparse SpMM on one MI355X.

Workload of the headline (`value`): the skewed SpMM, the largest single-GPU
configuration: C = A*B with A 16384x16384 in 32x32 bf16 blocks, Zipf(1.2)
blocks per block row capped at 512 and rescaled to 2% mean density (5243
blocks), B 16384x1024 bf16, fp32 accumulation and fp32 output.  It is
HBM-bound (99 FLOP per algorithmic byte), so its roofline is the HBM one.
The same run measures every benchmark configuration as a section:
  c1         A 1024x1024, 10%, N=256 (the reference's CPU-golden case)
  sweep      A 4096x4096, densities 1/5/25/50%, N=512, fp32 and bf16 C
  sddmm      mask 4096x4096 10%, X 4096x256, Y 256x4096
  skewed     the headline workload
  attention  seq 8192, d 128: SDDMM then SpMM, and the fused pair
  spgemm     8192x8192 x 8192x8192, 32x32 blocks, 5% x 5%
  large      the reference's 8192^3 configuration (256x256 blocks, 25%) and
             the same shape with 128x128 and 64x64 blocks
  patterns   the reference's pattern families (Row, Col, Multi-diag, Random,
             tril, triu) at 8192^3 with 256x256 blocks
  host       the blocking host-buffer entry point (PCIe included; never `value`)
  ablation   load balancing on and off (the reference's `_no_lb` operators) and
             the per-workgroup timeline of the instrumented library (only when
             asked for with --only ablation)
The last stdout line is one compact JSON object: the headline fields, its
roofline and CPU baseline, and a `summary` row per configuration.  The full
per-section records are written to --sections-out.

A step is one launch over the whole workload.  Inputs are resident in HBM:
the timed launches cycle through enough copies of the operands and outputs
(> 512 MB) that no launch finds them in the 256 MB Infinity Cache.
Effective TFLOP/s counts only nonzero-block FLOPs, 2*nnzb*R*C*N (the
reference's formula, GEMM_profiling/read_spmm_profiler.py:73).

Timing, per section, all on the stream the kernels run on:
  - us_per_launch: the K timed launches captured once into a HIP graph and
    replayed between two HIP events; replay time / K is the steady-state time
    per launch (the fixed cost of a launch included).  `value` and the
    headline roofline use it.
  - kernel_us: the same launches issued one by one and traced (torch's
    profiler, the HIP runtime's activity records): the median kernel duration,
    as rocprofv3 --kernel-trace reports it.
The CPU baseline is the oracle (the C restatement of the reference's golden,
oracle/bsp_oracle.c) on this host, per section: one thread (how the
reference's golden runs: its OpenMP pragma does not compile) on a named
sample of block rows, and all cores (OpenMP over block rows) on the whole
workload; median of 3 runs after one warm-up.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--only a,b]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import re
import sys
import time
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA (AMD Instinct MI355X datasheet)
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E
ROTATE_BYTES = 600 << 20   # > 2 x the 256 MB Infinity Cache
SECTIONS = ("c1", "sweep", "sddmm", "skewed", "attention", "spgemm", "large", "patterns", "host", "ablation")


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--no-kernel-time", action="store_true", help="skip the traced kernel durations")
    p.add_argument("--copy-calibration", action="store_true",
                   help="first run a 256 MiB device copy and a 256 MiB elementwise multiply (kernels of known traffic, "
                        "for scaling FETCH_SIZE / WRITE_SIZE counters)")
    p.add_argument("--only", default="", help="comma list of sections (head = the skewed headline workload only): "
                   + ", ".join(("head",) + SECTIONS))
    p.add_argument("--sections-out", default=str(REPO / "gpurun_out" / "bench_sections.json"),
                   help="file for the full per-section records (the last stdout line carries the summary)")
    return p.parse_args()


# ---------------------------------------------------------------------------
# Timing
class Timer:
    """Graph replay of K launches between two HIP events (us_per_launch), and
    the same launches one by one under the tracer (kernel durations)."""

    def __init__(self, torch, steps, trace=True):
        self.torch = torch
        self.steps = steps
        self.trace = trace

    def run(self, launch, warmup, kernel_filter=("bsp::",)):
        torch = self.torch
        steps = self.steps
        cur = torch.cuda.current_stream()
        for i in range(warmup):
            launch(i, cur.cuda_stream)
        torch.cuda.synchronize()
        kernels = {}
        if self.trace:
            from torch.profiler import ProfilerActivity, profile
            with profile(activities=[ProfilerActivity.CUDA]) as prof:
                for i in range(steps):
                    launch(warmup + i, cur.cuda_stream)
                    cur.synchronize()  # one launch at a time: each kernel starts on an idle GPU
            per = {}
            for e in prof.events():
                if e.device_time > 0 and any(k in e.name for k in kernel_filter):
                    per.setdefault(e.name, []).append(e.device_time)
            kernels = {name: {"median_us": round(float(np.median(v)), 3), "mean_us": round(float(np.mean(v)), 3),
                              "launches": len(v)} for name, v in per.items()}
        graph = torch.cuda.CUDAGraph()
        cap = torch.cuda.Stream()
        cap.wait_stream(cur)
        with torch.cuda.graph(graph, stream=cap):
            for i in range(steps):
                launch(warmup + i, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        graph.replay()  # one untimed replay
        torch.cuda.synchronize()
        g0, g1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        g0.record()
        graph.replay()
        g1.record()
        torch.cuda.synchronize()
        graph_ms = g0.elapsed_time(g1)
        del graph
        # kernel time per launch: the sum over the launch's kernels (a split
        # plan adds its reduce kernel) of their median traced durations
        k_us = sum(v["median_us"] * v["launches"] / steps for v in kernels.values()) if kernels else None
        return {"graph_ms": graph_ms, "launch_ms": graph_ms / steps, "kernel_us": k_us, "kernels": kernels}


def dev_u16(torch, arr):
    arr = np.ascontiguousarray(arr, dtype=np.uint16)
    if arr.size == 0:
        return torch.zeros(8, dtype=torch.int16, device="cuda")
    return torch.from_numpy(arr.view(np.int16)).to("cuda")


def summarize(t, flops, nbytes):
    """Per-launch figures from the graph replay and from the traced kernel
    durations: us, TFLOP/s, GB/s (algorithmic bytes) and fractions of peak."""
    k_s = t["launch_ms"] * 1e-3
    out = {
        "us_per_launch": round(t["launch_ms"] * 1e3, 3),
        "tflops": round(flops / k_s / 1e12, 3),
        "frac_mfma_peak": round(flops / k_s / 1e12 / PEAK_BF16_TFLOPS, 4),
        "gbs": round(nbytes / k_s / 1e9, 1),
        "frac_hbm_peak": round(nbytes / k_s / 1e9 / PEAK_HBM_GBS, 4),
        "flops": flops,
        "bytes": nbytes,
    }
    if t.get("kernel_us"):
        ks = t["kernel_us"] * 1e-6
        out.update({"kernel_us": round(t["kernel_us"], 3),
                    "kernel_tflops": round(flops / ks / 1e12, 3),
                    "kernel_gbs": round(nbytes / ks / 1e9, 1),
                    "kernel_frac_hbm_peak": round(nbytes / ks / 1e9 / PEAK_HBM_GBS, 4),
                    "kernel_frac_mfma_peak": round(flops / ks / 1e12 / PEAK_BF16_TFLOPS, 4),
                    "kernels": t["kernels"]})
    return out


def plan_summary(info):
    keys = ("tile_n", "stages", "group", "grid", "waves", "persistent", "a_stages", "step_entries", "n_split_rows",
            "n_entries", "n_items")
    return {k: info[k] for k in keys if k in info}


# ---------------------------------------------------------------------------
# Measured HBM-side traffic from the committed counter summaries
# (profiles/*_traffic.md: FETCH_SIZE and WRITE_SIZE per dispatch, scaled by
# kernels of known traffic).
def committed_traffic() -> dict:
    """{workload key: measured bytes per launch} from the `traffic_record:`
    lines (one JSON object each) of profiles/*_traffic.md."""
    out = {}
    for f in sorted((REPO / "profiles").glob("*_traffic.md")):
        for line in f.read_text().splitlines():
            if line.startswith("traffic_record: "):
                r = json.loads(line[len("traffic_record: "):])
                out[r["workload"]] = {"file": f.name, "kernel": r.get("kernel"), "bytes": int(r["bytes_per_launch"])}
    return out


TRAFFIC = committed_traffic()


def attach_traffic(rec, key):
    tr = TRAFFIC.get(key)
    if tr:
        rec["traffic"] = {"bytes_per_launch": tr["bytes"], "ratio_to_algorithmic": round(tr["bytes"] / rec["bytes"], 3),
                          "source": "profiles/" + tr["file"], "kernel": tr["kernel"]}
    rec["traffic_key"] = key


# ---------------------------------------------------------------------------
# Sections
def bench_spmm(torch, capi, W, a, b, out_dtype, timer, warmup, rotate=True, lib=None):
    """Times SpMM on (a, b) (through `lib`, default libbsparse.so); returns
    (timings, flops, bytes, plan info, copies)."""
    M, N = a.H, b.shape[1]
    plan = capi.SpmmPlan(capi.Bsr(a.H, a.W, a.R, a.C, a.indptr, a.indices), N, out_dtype, lib=lib)
    out_bytes = 4 if out_dtype == "f32" else 2
    per_copy = a.data.nbytes + b.nbytes + M * N * out_bytes
    ncopy = max(1, -(-ROTATE_BYTES // per_copy)) if rotate else 1
    da0, db0 = dev_u16(torch, a.data), dev_u16(torch, b)
    copies = []
    for _ in range(ncopy):
        dc = torch.empty((M, N), dtype=torch.float32 if out_dtype == "f32" else torch.int16, device="cuda")
        copies.append((da0.clone(), db0.clone(), dc))

    def launch(i, stream):
        da, db, dc = copies[i % ncopy]
        plan.run(da, db, dc, stream=stream)

    t = timer.run(launch, warmup)
    info = plan.info()
    plan.close()
    del copies
    return t, W.spmm_flops(a.nblocks, a.R, a.C, N), W.spmm_bytes(a, N, out_bytes), info, ncopy


def bench_sddmm(torch, capi, W, mask, x, y, y_layout, out_dtype, timer, warmup, lib=None):
    K = x.shape[1]
    plan = capi.SddmmPlan(capi.Bsr(mask.H, mask.W, mask.R, mask.C, mask.indptr, mask.indices), K,
                          y_layout, out_dtype, lib=lib)
    nv = mask.nblocks * mask.R * mask.C
    out_bytes = 4 if out_dtype == "f32" else 2
    per_copy = mask.data.nbytes + x.nbytes + y.nbytes + nv * out_bytes
    ncopy = max(1, -(-ROTATE_BYTES // per_copy))
    dm0, dx0, dy0 = dev_u16(torch, mask.data), dev_u16(torch, x), dev_u16(torch, y)
    copies = []
    for _ in range(ncopy):
        do = torch.empty(nv, dtype=torch.float32 if out_dtype == "f32" else torch.int16, device="cuda")
        copies.append((dm0.clone(), dx0.clone(), dy0.clone(), do))
    ldy = mask.W if y_layout == capi.ROW_MAJOR else K

    def launch(i, stream):
        dm, dx, dy, do = copies[i % ncopy]
        plan.run(dm, dx, dy, do, ldy=ldy, stream=stream)

    t = timer.run(launch, warmup)
    info = plan.info()
    plan.close()
    del copies
    return t, W.sddmm_flops(mask.nblocks, mask.R, mask.C, K), W.sddmm_bytes(mask, K, out_bytes), info


def bench_attention(torch, capi, W, w, out_dtype, timer, warmup):
    """The fused pair (bsp_attention); bytes are Q, K, V, the mask values, the
    index arrays and O (S never leaves the chip)."""
    m, q, k, v, d = w["mask"], w["q"], w["k"], w["v"], w["d"]
    plan = capi.AttentionPlan(capi.Bsr(m.H, m.W, m.R, m.C, m.indptr, m.indices), d, out_dtype)
    out_bytes = 4 if out_dtype == "f32" else 2
    per_copy = m.data.nbytes + q.nbytes + k.nbytes + v.nbytes + m.H * d * out_bytes
    ncopy = max(1, -(-ROTATE_BYTES // per_copy))
    base = [dev_u16(torch, x) for x in (m.data, q, k, v)]
    copies = []
    for _ in range(ncopy):
        do = torch.empty((m.H, d), dtype=torch.float32 if out_dtype == "f32" else torch.int16, device="cuda")
        copies.append([x.clone() for x in base] + [do])

    def launch(i, stream):
        dm, dq, dk, dv, do = copies[i % ncopy]
        plan.run(dm, dq, dk, dv, do, stream=stream)

    t = timer.run(launch, warmup)
    info = plan.info()
    plan.close()
    del copies
    flops = W.sddmm_flops(m.nblocks, m.R, m.C, d) + W.spmm_flops(m.nblocks, m.R, m.C, d)
    nbytes = (float(m.data.nbytes + q.nbytes + k.nbytes + v.nbytes) + 4.0 * (m.nblocks + m.nbrows + 1)
              + float(m.H) * d * out_bytes)
    return t, flops, nbytes, info


def bench_spgemm(torch, capi, W, a, b, out_dtype, timer, warmup):
    """The SpGEMM numeric phase on (a, b); FLOPs are 2*R*C*BC per (A block,
    B block) pair, bytes are A's and B's values and index arrays plus C's."""
    plan = capi.SpgemmPlan(capi.Bsr(a.H, a.W, a.R, a.C, a.indptr, a.indices),
                           capi.Bsr(b.H, b.W, b.R, b.C, b.indptr, b.indices), out_dtype)
    out_bytes = 4 if out_dtype == "f32" else 2
    nv = plan.out_values
    per_copy = a.data.nbytes + b.data.nbytes + nv * out_bytes
    ncopy = max(1, -(-ROTATE_BYTES // per_copy))
    da0, db0 = dev_u16(torch, a.data), dev_u16(torch, b.data)
    copies = []
    for _ in range(ncopy):
        do = torch.empty(max(nv, 1), dtype=torch.float32 if out_dtype == "f32" else torch.int16, device="cuda")
        copies.append((da0.clone(), db0.clone(), do))

    def launch(i, stream):
        da, db, do = copies[i % ncopy]
        plan.run(da, db, do, stream=stream)

    t = timer.run(launch, warmup)
    info = plan.info()
    nblocks = plan.structure.nblocks
    plan.close()
    del copies
    pa = np.zeros((a.nbrows, a.W // a.C), np.int64)
    np.add.at(pa, (np.repeat(np.arange(a.nbrows), np.diff(a.indptr)), a.indices), 1)
    pb = np.zeros((b.nbrows, b.W // b.C), np.int64)
    np.add.at(pb, (np.repeat(np.arange(b.nbrows), np.diff(b.indptr)), b.indices), 1)
    pairs = int((pa @ pb).sum())
    flops = 2.0 * pairs * a.R * a.C * b.C
    nbytes = (float(a.data.nbytes + b.data.nbytes) + 4.0 * (a.nblocks + a.nbrows + 1 + b.nblocks + b.nbrows + 1)
              + float(nv) * out_bytes)
    return t, flops, nbytes, info, {"pairs": pairs, "out_blocks": nblocks}


def traffic_key_spmm(a, N, out_dtype):
    return f"spmm {a.H}x{a.W} r{a.R}c{a.C} nnzb{a.nblocks} N{N} {out_dtype}"


# ---------------------------------------------------------------------------
# CPU baseline (the oracle on this host)
def host_cores():
    cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    return max(1, min(cores, int(os.environ.get("OMP_NUM_THREADS", cores))))


def _median_time(fn, reps=3):
    fn()  # warm-up
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts))


def _row_prefix(indptr, flops_per_block, budget):
    """Block rows 0..r-1 whose blocks cost at most `budget` FLOPs (at least one row)."""
    cum = np.cumsum(np.diff(indptr).astype(np.float64) * flops_per_block)
    return max(1, int(np.searchsorted(cum, budget, side="right")))


SINGLE_BUDGET = 4e8   # FLOPs of the one-thread sample (about half a second)
ALL_BUDGET = 1.6e10   # the all-core leg times the whole workload up to this


def cpu_spmm(orc, W, a, b, cores, gpu_tflops, single_budget=SINGLE_BUDGET):
    N = b.shape[1]
    fpb = 2.0 * a.R * a.C * N
    rec = {}
    for leg, threads, budget in (("single", 1, single_budget), ("all", cores, ALL_BUDGET)):
        r = _row_prefix(a.indptr, fpb, budget)
        r = min(r, a.nbrows)
        nb = int(a.indptr[r])
        ip = np.ascontiguousarray(a.indptr[: r + 1])
        t = _median_time(lambda: orc.spmm(ip, a.indices[:nb], a.data[: nb * a.R * a.C], r * a.R, a.W, a.R, a.C, b,
                                          threads=threads))
        tf = W.spmm_flops(nb, a.R, a.C, N) / t / 1e12
        rec[leg] = {"tflops": round(tf, 6), "cores": threads, "seconds": round(t, 4),
                    "sample": "whole workload" if r == a.nbrows else
                    f"block rows 0..{r - 1} ({nb} of {a.nblocks} blocks)",
                    "gpu_speedup": round(gpu_tflops / tf, 1) if gpu_tflops and tf > 0 else None}
    rec["kind"] = "port"
    return rec


def cpu_sddmm(orc, W, m, x, y, cores, gpu_tflops, y_colmajor=False):
    K = x.shape[1]
    fpb = 2.0 * m.R * m.C * K + m.R * m.C
    rec = {}
    for leg, threads, budget in (("single", 1, SINGLE_BUDGET), ("all", cores, ALL_BUDGET)):
        r = min(_row_prefix(m.indptr, fpb, budget), m.nbrows)
        nb = int(m.indptr[r])
        ip = np.ascontiguousarray(m.indptr[: r + 1])
        xs = np.ascontiguousarray(x[: r * m.R])
        t = _median_time(lambda: orc.sddmm(ip, m.indices[:nb], m.data[: nb * m.R * m.C], r * m.R, m.W, m.R, m.C, xs,
                                           y, y_colmajor=y_colmajor, threads=threads))
        tf = W.sddmm_flops(nb, m.R, m.C, K) / t / 1e12
        rec[leg] = {"tflops": round(tf, 6), "cores": threads, "seconds": round(t, 4),
                    "sample": "whole workload" if r == m.nbrows else
                    f"block rows 0..{r - 1} ({nb} of {m.nblocks} blocks)",
                    "gpu_speedup": round(gpu_tflops / tf, 1) if gpu_tflops and tf > 0 else None}
    rec["kind"] = "port"
    return rec


def cpu_pair(orc, W, w, cores, gpu_tflops):
    """The attention pair on the oracle: SDDMM (K as column-major Y) then SpMM."""
    m, d = w["mask"], w["d"]
    fpb = 2.0 * m.R * m.C * d * 2 + m.R * m.C
    rec = {}
    for leg, threads, budget in (("single", 1, SINGLE_BUDGET), ("all", cores, ALL_BUDGET)):
        r = min(_row_prefix(m.indptr, fpb, budget), m.nbrows)
        nb = int(m.indptr[r])
        ip = np.ascontiguousarray(m.indptr[: r + 1])
        qs = np.ascontiguousarray(w["q"][: r * m.R])

        def pair():
            orc.sddmm(ip, m.indices[:nb], m.data[: nb * 1024], r * m.R, m.W, m.R, m.C, qs, w["k"], y_colmajor=True,
                      threads=threads)
            orc.spmm(ip, m.indices[:nb], m.data[: nb * 1024], r * m.R, m.W, m.R, m.C, w["v"], threads=threads)
        t = _median_time(pair)
        tf = (W.sddmm_flops(nb, m.R, m.C, d) + W.spmm_flops(nb, m.R, m.C, d)) / t / 1e12
        rec[leg] = {"tflops": round(tf, 6), "cores": threads, "seconds": round(t, 4),
                    "sample": "whole pair (SDDMM then SpMM)" if r == m.nbrows else
                    f"block rows 0..{r - 1} ({nb} of {m.nblocks} blocks), SDDMM then SpMM",
                    "gpu_speedup": round(gpu_tflops / tf, 1) if gpu_tflops and tf > 0 else None}
    rec["kind"] = "port"
    return rec


def cpu_spgemm(orc, W, a, b, gpu_tflops):
    """The SpGEMM golden (single-threaded, as the reference's bsr_matrix::spgemm)."""
    rows = 32
    nb = int(a.indptr[rows])
    bcount = np.diff(b.indptr).astype(np.int64)
    pairs = int(bcount[a.indices[:nb]].sum())
    t = _median_time(lambda: orc.spgemm(a.indptr[: rows + 1], a.indices[:nb], a.data[: nb * a.R * a.C], rows * a.R,
                                        a.R, a.C, b.indptr, b.indices, b.data, b.W, b.C))
    tf = 2.0 * pairs * a.R * a.C * b.C / t / 1e12
    single = {"tflops": round(tf, 6), "cores": 1, "seconds": round(t, 4),
              "sample": f"block rows 0..{rows - 1} of A ({nb} blocks, {pairs} block products)",
              "gpu_speedup": round(gpu_tflops / tf, 1) if gpu_tflops else None}
    return {"single": single, "all": dict(single, note="the SpGEMM golden has no threaded form"), "kind": "port"}


def cpu_large(orc, W, a, b, cores, gpu_tflops):
    """256x256 blocks: per-block work is large; the sample is the first
    block rows (one per thread) against the first 64 columns of B."""
    ncols = 64
    bs = np.ascontiguousarray(b[:, :ncols])
    rec = {}
    for leg, threads in (("single", 1), ("all", cores)):
        rows = min(a.nbrows, threads)
        nb = int(a.indptr[rows])
        t = _median_time(lambda: orc.spmm(a.indptr[: rows + 1], a.indices[:nb], a.data[: nb * a.R * a.C], rows * a.R,
                                          a.W, a.R, a.C, bs, threads=threads))
        tf = W.spmm_flops(nb, a.R, a.C, ncols) / t / 1e12
        rec[leg] = {"tflops": round(tf, 6), "cores": threads, "seconds": round(t, 4),
                    "sample": f"block rows 0..{rows - 1} ({nb} of {a.nblocks} blocks) times the first {ncols} "
                              "columns of B",
                    "gpu_speedup": round(gpu_tflops / tf, 1) if gpu_tflops and tf > 0 else None}
    rec["kind"] = "port"
    return rec


# ---------------------------------------------------------------------------
# On-chip roof of the 32x32 SpMM: the kernel's L2 -> LDS volume at the
# measured rate of an L2-resident DMA stream, plus the fixed cost of a launch.
def probe_lib():
    lib = ctypes.CDLL(str(REPO / "tenstorrent-wh-blockspmm_amd" / "libbsp_probe.so"))
    lib.bsp_probe_dma_stream.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                         ctypes.c_void_p]
    lib.bsp_probe_empty.argtypes = [ctypes.c_int, ctypes.c_void_p]
    return lib


def measure_roofs(torch, steps=50):
    """TB/s of an L2-resident DMA stream (2 MB region, 512 workgroups x 8
    waves, two per compute unit as in the SpMM kernel, 16 loads of 1 KB in
    flight per wave) and an HBM one (1 GB), and the graph-replay time of an
    empty 512-workgroup kernel.  Each stream launch moves 4 GB, so the fixed
    cost of its launch stays below 2% of its time (the floor adds that cost
    once, as the empty launch)."""
    lib = probe_lib()
    buf = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
    buf.fill_(1)
    st = torch.cuda.current_stream()
    grid, waves, iters = 512, 8, 1024

    def graph_us(fn, steps=steps):
        for _ in range(3):
            fn(st.cuda_stream)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        cap = torch.cuda.Stream()
        cap.wait_stream(st)
        with torch.cuda.graph(g, stream=cap):
            for _ in range(steps):
                fn(torch.cuda.current_stream().cuda_stream)
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / steps

    out = {}
    for name, region in (("l2_stream_tbs", 2 << 20), ("hbm_stream_tbs", 1 << 30)):
        us = graph_us(lambda s: lib.bsp_probe_dma_stream(buf.data_ptr(), region, grid, waves, iters, s), steps=5)
        out[name] = round(grid * waves * iters * 1024 / (us * 1e-6) / 1e12, 2)
    out["empty_launch_us"] = round(graph_us(lambda s: lib.bsp_probe_empty(512, s)), 3)
    del buf
    return out


def on_chip_roof(info, us, roofs):
    """L2 -> LDS bytes of a 32x32 SpMM launch (every entry brings its 2 KB A
    sub-block and the 32 x tile slice of B into LDS) against the measured
    L2-resident stream rate, plus the launch's fixed cost."""
    vol = float(info["n_entries"]) * (2048 + 64 * info["tile_n"])
    stream_us = vol / (roofs["l2_stream_tbs"] * 1e12) * 1e6
    floor = stream_us + roofs["empty_launch_us"]
    return {"l2_to_lds_bytes": vol, "l2_stream_tbs": roofs["l2_stream_tbs"],
            "empty_launch_us": roofs["empty_launch_us"], "floor_us": round(floor, 3),
            "frac": round(floor / us, 4),
            "note": "floor = L2->LDS volume at the L2-resident DMA rate + an empty launch; frac = floor / us_per_launch"}


# Dense reference: the vendor library's bf16 GEMM (torch.matmul, which runs
# hipBLASLt) on the dense equivalent of a workload, operands resident.  It
# says what the block-sparse kernel saves against ignoring the sparsity, and
# at 8192^3 what MFMA rate a tuned dense kernel reaches on this GPU (the
# clock drops under sustained MFMA load, so no kernel reaches the nominal
# peak).
_DENSE = {}


def dense_gemm(torch, M, K, N, iters=20):
    key = (M, K, N)
    if key not in _DENSE:
        a = torch.randn(M, K, device="cuda", dtype=torch.bfloat16)
        b = torch.randn(K, N, device="cuda", dtype=torch.bfloat16)
        c = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
        for _ in range(3):
            torch.matmul(a, b, out=c)
        torch.cuda.synchronize()
        # timed like the sparse kernels: graph replay of `iters` launches
        graph = torch.cuda.CUDAGraph()
        cap = torch.cuda.Stream()
        cap.wait_stream(torch.cuda.current_stream())
        with torch.cuda.graph(graph, stream=cap):
            for _ in range(iters):
                torch.matmul(a, b, out=c)
        graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        graph.replay()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / iters
        del graph, a, b, c
        _DENSE[key] = {"shape": [M, K, N], "us": round(us, 3),
                       "tflops": round(2.0 * M * K * N / (us * 1e-6) / 1e12, 1)}
    return dict(_DENSE[key])


def dense_record(torch, M, K, N, us):
    """The dense-equivalent GEMM's time and this kernel's speedup over it."""
    d = dense_gemm(torch, M, K, N)
    d["speedup"] = round(d["us"] / us, 2)
    d["note"] = "torch.matmul bf16 (hipBLASLt) on the dense M x K by K x N product, graph replay, operands resident"
    return d


# ---------------------------------------------------------------------------
def roofline(flops, nbytes, us, traffic_bytes, kernel):
    """The bound is the lower roof for the kernel's algorithmic intensity:
    MFMA when FLOP/byte >= peak FLOP/s / peak bytes/s (312.5), else HBM."""
    k_s = us * 1e-6
    ai = flops / nbytes
    ridge = PEAK_BF16_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9)
    tflops = flops / k_s / 1e12
    gbs = nbytes / k_s / 1e9
    r = {"kernel": kernel, "us_per_launch": round(us, 3), "algorithmic_flop_per_launch": flops,
         "algorithmic_bytes_per_launch": nbytes, "intensity_flop_per_byte": round(ai, 1), "traffic": traffic_bytes,
         "mfma_tflops": round(tflops, 3), "mfma_frac": round(tflops / PEAK_BF16_TFLOPS, 4),
         "hbm_gbs": round(gbs, 1), "hbm_frac": round(gbs / PEAK_HBM_GBS, 4)}
    if ai >= ridge:
        r.update({"bound": "mfma", "achieved": round(tflops, 3), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                  "frac": round(tflops / PEAK_BF16_TFLOPS, 4)})
    else:
        r.update({"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                  "frac": round(gbs / PEAK_HBM_GBS, 4)})
    return r


PATTERNS = ("row", "col", "multi_diag", "random")


def pattern_workload(W, pattern, density):
    """A of 8192^2 in 256x256 blocks in one of the reference's pattern
    families (block_spmm/inc/profiling_suite.hpp:3513-3574): the first
    round(density * 1024) positions of FILL_ROW / FILL_COL / FILL_MULTI_DIAG,
    or uniform-random ones; tril and triu are the full triangles.  Values
    U[-1, 1] bf16."""
    n, R = 8192, 256
    nbr = n // R
    rng = W.Rng(W.SEED_BASE + 7)
    if pattern in ("tril", "triu"):
        a = (W.fill_tril if pattern == "tril" else W.fill_triu)(n, n, R, R)
    elif pattern == "random":
        a = W.random_positions(n, n, R, R, int(round(density * nbr * nbr)), rng)
    else:
        fill = {"row": W.fill_row, "col": W.fill_col, "multi_diag": W.fill_multi_diag}[pattern]
        a = fill(n, n, R, R, int(round(density * nbr * nbr)))
    a.data = W.bf16_from_f32(W.uniform_f32(rng, a.nblocks * R * R))
    return a


def pattern_b(W):
    """B of the pattern sweep: 8192 x 8192 bf16 U[-1, 1]."""
    return W.bf16_from_f32(W.uniform_f32(W.Rng(W.SEED_BASE + 8), (8192, 8192)))


def main():
    args = parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only; run with --gpus 1 "
                                   "(the multi-GPU sharding is a design note, not built)"}))
        sys.exit(2)
    import torch
    import __graft_entry__ as entry

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(1)
    pkg = entry.load_package()
    capi, W = pkg.capi, pkg.workloads
    capi.load()
    only = set(filter(None, args.only.split(",")))

    def run(section):
        if only and section not in only:
            return False
        if not only and section == "ablation":  # its own run: bench.py --only ablation
            return False
        print(f"[bench] {section}", file=sys.stderr, flush=True)  # progress, one line per section
        return True
    steps, warmup = args.steps, args.warmup
    timer = Timer(torch, steps, trace=not args.no_kernel_time)
    orc = None if args.no_cpu else entry._load_oracle()
    cores = host_cores()
    if args.copy_calibration:
        # Two kernels that each read 256 MiB and write 256 MiB: the runtime's
        # device-to-device copy and an elementwise multiply.
        src = torch.ones(64 << 20, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.mul(src, 2.0, out=dst)
        torch.cuda.synchronize()
        del src, dst

    out = {}

    def spmm_section(w, od, label, rotate=True, cpu=True):
        t, fl, nb, info, ncopy = bench_spmm(torch, capi, W, w["a"], w["b"], od, timer, warmup, rotate=rotate)
        rec = {"workload": label, "out": od, "nnzb": w["a"].nblocks, **summarize(t, fl, nb),
               "plan": plan_summary(info), "copies": ncopy}
        attach_traffic(rec, traffic_key_spmm(w["a"], w["b"].shape[1], od))
        rec["dense_gemm"] = dense_record(torch, w["a"].H, w["a"].W, w["b"].shape[1], rec["us_per_launch"])
        if cpu and orc is not None:
            rec["cpu"] = cpu_spmm(orc, W, w["a"], w["b"], cores, rec["tflops"])
        return rec, t, fl, nb, info

    if run("c1"):
        w = W.workload_spmm_small()
        rec, *_ = spmm_section(w, "f32", "SpMM A 1024x1024, 32x32 blocks, 10% (102 blocks), B 1024x256, fp32 C")
        rec["input_sha256"] = W.workload_digest(w)
        out["c1"] = rec

    if run("sweep"):
        sweep = []
        for d in W.SPMM_SWEEP_DENSITIES:
            w = W.workload_spmm_sweep(d)
            digest = W.workload_digest(w)
            cpu_rec = None
            for od in ("f32", "bf16"):
                rec, t, fl, nb, info = spmm_section(
                    w, od, f"SpMM A 4096x4096, 32x32 blocks, {int(d * 100)}%, B 4096x512, {od} C",
                    cpu=cpu_rec is None)
                if cpu_rec is None:
                    cpu_rec = rec.get("cpu")
                elif cpu_rec is not None:
                    # the oracle's rate does not depend on the GPU's output type
                    rec["cpu"] = {k: (dict(v, gpu_speedup=round(rec["tflops"] / v["tflops"], 1))
                                      if isinstance(v, dict) else v) for k, v in cpu_rec.items()}
                rec.update({"density": d, "input_sha256": digest})
                sweep.append(rec)
            # warm (cache-resident) figure for the same launch, for reference
            t, fl, nb, info, _ = bench_spmm(torch, capi, W, w["a"], w["b"], "f32", timer, warmup, rotate=False)
            sweep.append({"density": d, "out": "f32", "warm_cache": True, **summarize(t, fl, nb)})
        out["sweep"] = sweep

    if run("sddmm"):
        s = W.workload_sddmm()
        m = s["mask"]
        t, fl, nb, info = bench_sddmm(torch, capi, W, m, s["x"], s["y"], capi.ROW_MAJOR, "f32", timer, warmup)
        rec = {"workload": "SDDMM mask 4096x4096 32x32 blocks d=10%, X 4096x256, Y 256x4096, fp32 out",
               "nnzb": m.nblocks, **summarize(t, fl, nb), "plan": {"grid": info["grid"], "one_shot": info["stages"]},
               "input_sha256": W.workload_digest(s)}
        attach_traffic(rec, f"sddmm {m.H}x{m.W} r{m.R}c{m.C} nnzb{m.nblocks} K{s['K']} f32")
        if orc is not None:
            rec["cpu"] = cpu_sddmm(orc, W, m, s["x"], s["y"], cores, rec["tflops"])
        out["sddmm"] = rec

    if run("skewed") or run("head"):
        w = W.workload_spmm_skewed()
        rec, *_ = spmm_section(w, "f32", "SpMM A 16384x16384 Zipf(1.2) rows, 2% mean density, B 16384x1024, fp32 C")
        rec["input_sha256"] = W.workload_digest(w)
        rec["max_row_blocks"] = int(np.diff(w["a"].indptr).max())
        out["skewed"] = rec

    if run("attention"):
        w = W.workload_attention()
        m = w["mask"]
        t1, f1, b1, _ = bench_sddmm(torch, capi, W, m, w["q"], w["k"], capi.COL_MAJOR, "bf16", timer, warmup)
        a = W.BsrArrays(m.H, m.W, 32, 32, m.indptr, m.indices, m.data)
        t2, f2, b2, info2, _ = bench_spmm(torch, capi, W, a, w["v"], "f32", timer, warmup)
        t3, f3, b3, _ = bench_attention(torch, capi, W, w, "f32", timer, warmup)
        fused = summarize(t3, f3, b3)
        attach_traffic(fused, f"attention seq{m.H} d{w['d']} nnzb{m.nblocks} f32")
        s_rec, o_rec = summarize(t1, f1, b1), summarize(t2, f2, b2)
        o_rec["dense_gemm"] = dense_record(torch, m.H, m.W, w["d"], o_rec["us_per_launch"])
        attach_traffic(s_rec, f"sddmm {m.H}x{m.W} r{m.R}c{m.C} nnzb{m.nblocks} K{w['d']} bf16 colmajor")
        attach_traffic(o_rec, traffic_key_spmm(a, w["d"], "f32"))
        rec = {"workload": "seq 8192, d 128, 8 causal block bands + 1% global; S=mask(.)QK^T (bf16) then "
                           "O=S*V (fp32)",
               "nnzb": m.nblocks, "input_sha256": W.workload_digest(w), "sddmm": s_rec,
               "spmm": {**o_rec, "plan": plan_summary(info2)},
               "pair_tflops": round((f1 + f2) / ((t1["launch_ms"] + t2["launch_ms"]) * 1e-3) / 1e12, 3),
               "fused": fused}
        if orc is not None:
            rec["cpu"] = cpu_pair(orc, W, w, cores, fused["tflops"])
        out["attention"] = rec

    if run("spgemm"):
        w = W.workload_spgemm()
        rows = []
        for od in ("f32", "bf16"):
            t, fl, nb, info, extra = bench_spgemm(torch, capi, W, w["a"], w["b"], od, timer, warmup)
            r = {"out": od, **summarize(t, fl, nb), "grid": info["grid"], "sub_blocks": info["n_items"],
                 "products": info["n_entries"], **extra}
            attach_traffic(r, f"spgemm {w['a'].H}x{w['b'].W} r{w['a'].R}c{w['a'].C} nnzb{w['a'].nblocks}x{w['b'].nblocks} {od}")
            rows.append(r)
        rec = {"workload": "SpGEMM C=A*B, A and B 8192x8192, 32x32 blocks, 5% each (3277 blocks)",
               "nnzb": w["a"].nblocks, "input_sha256": W.workload_digest(w), "runs": rows}
        if orc is not None:
            rec["cpu"] = cpu_spgemm(orc, W, w["a"], w["b"], rows[0]["tflops"])
        out["spgemm"] = rec
        del w

    if run("large"):
        # The reference's own published configuration: M = N = K = 8192 with
        # 256 x 256 blocks at 25% (its best: 50.6 TFLOP/s on a Wormhole N150,
        # block_spmm/scripts/experiments_dram_reads_table.tex:27-30).
        w = W.workload_spmm_large_blocks(0.25)
        lt = Timer(torch, max(10, steps // 10), trace=timer.trace)
        rows = []
        for od in ("bf16", "f32"):
            t, fl, nb, info, _ = bench_spmm(torch, capi, W, w["a"], w["b"], od, lt, max(5, warmup // 2))
            r = {"out": od, **summarize(t, fl, nb), "plan": plan_summary(info)}
            attach_traffic(r, traffic_key_spmm(w["a"], 8192, od))
            r["dense_gemm"] = dense_record(torch, 8192, 8192, 8192, r["us_per_launch"])
            rows.append(r)
        rec = {"workload": "SpMM 8192^3, 256x256 blocks, 25% (256 blocks)", "nnzb": w["a"].nblocks,
               "input_sha256": W.workload_digest(w), "runs": rows}
        if orc is not None:
            rec["cpu"] = cpu_large(orc, W, w["a"], w["b"], cores, rows[-1]["tflops"])
        out["large_blocks"] = rec
        del w
        rows = []
        for R in (128, 64):
            w = W.workload_spmm_large_blocks(0.25, R=R)
            t, fl, nb, info, _ = bench_spmm(torch, capi, W, w["a"], w["b"], "f32", lt, max(5, warmup // 2))
            r = {"R": R, "C": R, "nnzb": w["a"].nblocks, "out": "f32", **summarize(t, fl, nb),
                 "plan": plan_summary(info)}
            attach_traffic(r, traffic_key_spmm(w["a"], 8192, "f32"))
            rows.append(r)
            del w
        out["block_sizes"] = {"workload": "SpMM 8192^3, R x R blocks, 25%, fp32 C", "runs": rows}

    if run("patterns"):
        # The reference's pattern sweep (Row, Col, Multi-diag, Random at 5% and
        # 50%; full tril and triu) at 8192^3 with 256x256 blocks, bf16 C (its
        # output type); its published DDA figures are in the records.
        published = {("row", 0.05): 11.5, ("random", 0.05): 28.0, ("multi_diag", 0.05): 25.0, ("col", 0.05): 25.7,
                     ("row", 0.5): 49.2, ("random", 0.5): 48.0, ("multi_diag", 0.5): 47.6, ("col", 0.5): 47.0,
                     ("tril", 1.0): 43.3, ("triu", 1.0): 29.6}
        lt = Timer(torch, max(10, steps // 10), trace=timer.trace)
        rows = []
        b = pattern_b(W)
        for pat, d in [(p, d) for d in (0.05, 0.5) for p in PATTERNS] + [("tril", 1.0), ("triu", 1.0)]:
            a = pattern_workload(W, pat, d)
            t, fl, nb, info, _ = bench_spmm(torch, capi, W, a, b, "bf16", lt, max(5, warmup // 2))
            r = {"pattern": pat, "density": d if pat not in ("tril", "triu") else round(a.nblocks / 1024, 4),
                 "nnzb": a.nblocks, "out": "bf16", **summarize(t, fl, nb), "plan": plan_summary(info),
                 "reference_dda_tflops_n150": published.get((pat, d))}
            attach_traffic(r, traffic_key_spmm(a, 8192, "bf16") + f" {pat}")
            r["dense_gemm"] = dense_record(torch, 8192, 8192, 8192, r["us_per_launch"])
            rows.append(r)
            del a
        del b
        out["patterns"] = {"workload": "SpMM 8192^3, 256x256 blocks, the reference's pattern families, bf16 C",
                           "runs": rows}

    if run("host"):
        # The blocking host-buffer entry point (the reference operator's shape):
        # plan, device allocation, PCIe upload of A and B, launch, download of
        # C, synchronise, free.  Reported beside `value`, never as it.
        w = W.workload_spmm_sweep(0.25)
        a = w["a"]
        bsr = capi.Bsr(a.H, a.W, a.R, a.C, a.indptr, a.indices)
        capi.host_spmm(bsr, a.data, w["b"], "f32")
        ts = []
        for _ in range(5):
            t0 = time.perf_counter()
            capi.host_spmm(bsr, a.data, w["b"], "f32")
            ts.append(time.perf_counter() - t0)
        t_host = float(np.median(ts))
        fl = W.spmm_flops(a.nblocks, 32, 32, 512)
        out["host_entry"] = {"workload": "25% SpMM through bsp_host_spmm (host buffers, blocking)",
                             "ms_per_call": round(t_host * 1e3, 3), "tflops": round(fl / t_host / 1e12, 4)}

    if run("ablation"):
        out["ablation"] = ablation(torch, capi, W, timer, warmup)

    roofs = measure_roofs(torch)
    big = dense_gemm(torch, 8192, 8192, 8192)
    sections_path = Path(args.sections_out)
    sections_path.parent.mkdir(parents=True, exist_ok=True)
    sections_path.write_text(json.dumps({"roofs": roofs, "dense_gemm_8192": big, **out}, indent=1))
    if "skewed" not in out:
        print(json.dumps({"sections": os.path.relpath(sections_path, REPO), "summary": summary_rows(out, roofs)}))
        return
    shown = os.path.relpath(sections_path, REPO) if sections_path.is_absolute() else str(sections_path)
    line = build_headline(out, roofs, big, steps, warmup, shown)
    print(json.dumps(line, separators=(",", ":")))


# ---------------------------------------------------------------------------
# Ablation: the cost decomposition, load balancing on and off, and the
# per-workgroup timeline.
#
# The reference prices its kernels' parts with profiling variants of its
# operators (block_spmm/inc/host_code.hpp:86-161, registered in
# HostCodeRegistryProfiling, :195-222; block_sddmm/inc/host_code.hpp:71-153;
# block_sddmm/PROFILING_PLAN.md).  Its comparisons are rebuilt here on
# committed code, all through libbsparse_timeline.so (the same sources as
# libbsparse.so, plus the switches and stamps of include/bsparse_timeline.h):
#   - the decomposition: each workload timed whole and with one part left
#     out (its _no_a_read, _no_b_read, _no_compute and _no_write variants;
#     SDDMM's _no_b/c/d_read), and with everything left out (the launch and
#     the schedule's own walk);
#   - load balancing on and off (its `_no_lb` operators; the published table
#     block_spmm/scripts/figures/load_imbalance_table.csv): plans built with
#     BSP_SPMM_BALANCE=0 keep rows whole and place work in natural order, in
#     contiguous ranges;
#   - where a launch's time goes: each workgroup's start, first landing,
#     progress and end.
class plan_env:
    """Environment variables set while plans are created (the library reads
    its schedule overrides at plan creation)."""

    def __init__(self, env):
        self.env = dict(env or {})

    def __enter__(self):
        self.saved = {k: os.environ.get(k) for k in self.env}
        os.environ.update({k: str(v) for k, v in self.env.items()})

    def __exit__(self, *exc):
        for k, v in self.saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


def timeline_stats(stamps, khz, kind):
    """Per-workgroup phases from a (grid x 64) stamp array: start offset from
    the first workgroup's start, first landing after its own start, work end
    after the first start, and (persistent SpMM) the time per unit."""
    s = stamps.astype(np.int64)
    ok = s[:, 0] > 0
    s = s[ok]
    if not len(s):
        return {"workgroups": 0}
    t0 = s[:, 0].min()
    to_us = 1000.0 / khz
    q = lambda v: {"p10": round(float(np.percentile(v, 10)), 3), "p50": round(float(np.median(v)), 3),
                   "p90": round(float(np.percentile(v, 90)), 3), "max": round(float(np.max(v)), 3)}
    start = (s[:, 0] - t0) * to_us
    end = (s[:, 63] - t0) * to_us
    landed = s[:, 1] > 0
    rec = {"workgroups": int(len(s)), "clock_khz": khz,
           "start_offset_us": q(start),
           "first_landing_us": q((s[landed, 1] - s[landed, 0]) * to_us) if landed.any() else None,
           "end_us": q(end), "span_us": round(float(end.max()), 3),
           "busy_us": q(end - start)}
    if kind == "persistent":
        # unit ends in slots 2.. (each unit with entries); the time between
        # consecutive ends, and the first unit's end after the first landing
        per = []
        for row in s:
            u = row[2:63]
            u = u[u > 0]
            if len(u) > 1:
                per.extend(np.diff(u) * to_us)
        rec["unit_us"] = q(np.array(per)) if per else None
    if kind == "sweep":
        # progress stamps every 8 entries: time per 8 entries after the first landing
        per = []
        for row in s:
            u = row[2:63]
            u = u[u > 0]
            if len(u) > 1:
                per.extend(np.diff(u) * to_us)
        rec["per_8_entries_us"] = q(np.array(per)) if per else None
    if kind == "sddmm":
        done = s[:, 2] > 0
        rec["products_us"] = q((s[done, 2] - s[done, 1]) * to_us) if done.any() else None
    return rec


def _timeline_run(torch, capi, tl, launch, grid, reps=3):
    """Launches through the timeline library `reps` times (cold operands:
    each launch takes the next copy) and returns the last launch's stamps and
    the stamp clock in kHz."""
    stamps = torch.zeros((grid, capi.TIMELINE_SLOTS), dtype=torch.int64, device="cuda")
    st = torch.cuda.current_stream()
    capi.check(tl.bsp_timeline_attach(stamps.data_ptr(), grid, 0), tl)
    try:
        for i in range(reps):
            stamps.zero_()
            launch(i, st.cuda_stream)
        torch.cuda.synchronize()
    finally:
        tl.bsp_timeline_attach(None, 0, 0)
    khz = ctypes.c_int(0)
    capi.check(tl.bsp_timeline_clock_khz(0, ctypes.byref(khz)), tl)
    return stamps.cpu().numpy(), khz.value


def timeline_spmm(torch, capi, W, a, b, out_dtype, env, kind):
    tl = capi.load_timeline()
    M, N = a.H, b.shape[1]
    with plan_env(env):
        plan = capi.SpmmPlan(capi.Bsr(a.H, a.W, a.R, a.C, a.indptr, a.indices), N, out_dtype, lib=tl)
    info = plan.info()
    out_bytes = 4 if out_dtype == "f32" else 2
    per_copy = a.data.nbytes + b.nbytes + M * N * out_bytes
    ncopy = max(1, -(-ROTATE_BYTES // per_copy))
    da0, db0 = dev_u16(torch, a.data), dev_u16(torch, b)
    copies = [(da0.clone(), db0.clone(),
               torch.empty((M, N), dtype=torch.float32 if out_dtype == "f32" else torch.int16, device="cuda"))
              for _ in range(ncopy)]

    def launch(i, stream):
        da, db, dc = copies[i % ncopy]
        plan.run(da, db, dc, stream=stream)
    stamps, khz = _timeline_run(torch, capi, tl, launch, info["grid"])
    plan.close()
    rec = timeline_stats(stamps, khz, kind)
    rec["plan"] = plan_summary(info)
    return rec


def timeline_sddmm(torch, capi, W, m, x, y, out_dtype):
    tl = capi.load_timeline()
    K = x.shape[1]
    plan = capi.SddmmPlan(capi.Bsr(m.H, m.W, m.R, m.C, m.indptr, m.indices), K, capi.ROW_MAJOR, out_dtype, lib=tl)
    info = plan.info()
    nv = m.nblocks * m.R * m.C
    base = [dev_u16(torch, v) for v in (m.data, x, y)]
    per_copy = m.data.nbytes + x.nbytes + y.nbytes + nv * 4
    ncopy = max(1, -(-ROTATE_BYTES // per_copy))
    copies = [[v.clone() for v in base] + [torch.empty(nv, dtype=torch.float32, device="cuda")]
              for _ in range(ncopy)]

    def launch(i, stream):
        dm, dx, dy, do = copies[i % ncopy]
        plan.run(dm, dx, dy, do, ldy=m.W, stream=stream)
    stamps, khz = _timeline_run(torch, capi, tl, launch, info["grid"])
    plan.close()
    rec = timeline_stats(stamps, khz, "sddmm")
    rec["plan"] = {"grid": info["grid"], "one_shot": info["stages"]}
    return rec


SPMM_PARTS = (("full", 0), ("no_a_read", 1), ("no_b_read", 2), ("no_reads", 1 | 2), ("no_compute", 8),
              ("no_write", 16), ("nothing", 1 | 2 | 8 | 16))
SDDMM_PARTS = (("full", 0), ("no_mask_read", 1), ("no_x_read", 2), ("no_y_read", 4), ("no_compute", 8),
               ("no_write", 16), ("nothing", 1 | 2 | 4 | 8 | 16))


def decompose(torch, capi, tl, parts, time_one):
    """Times one workload with each set of parts left out (graph replay,
    cold operands); returns {part: us} and the time each part adds (full
    minus the time without it)."""
    rec = {}
    try:
        for name, flags in parts:
            capi.check(tl.bsp_timeline_skip(flags), tl)
            rec[name] = time_one()
    finally:
        tl.bsp_timeline_skip(0)
    rec["saved_us"] = {name: round(rec["full"] - rec[name], 3) for name, _ in parts if name != "full"}
    return rec


def decomposition(torch, capi, W, warmup):
    """The cost decomposition of the headline kernels: 4096^2 25% and 50%
    (fp32 C), the skewed 16384^2, the reference's own 8192^3 configuration
    (256x256 blocks, random 50%, bf16 C), and the 10% SDDMM."""
    tl = capi.load_timeline()
    timer = Timer(torch, 50, trace=False)
    out = {}

    def spmm(label, a, b, od, env=None):
        plan_kind = {}

        def one():
            with plan_env(env):
                t, fl, nb, info, _ = bench_spmm(torch, capi, W, a, b, od, timer, warmup, lib=tl)
            plan_kind.update(plan_summary(info))
            return round(t["launch_ms"] * 1e3, 3)
        r = decompose(torch, capi, tl, SPMM_PARTS, one)
        r["plan"] = plan_kind
        with plan_env(env):  # the same launch through libbsparse.so, for the instrumented build's overhead
            t, *_ = bench_spmm(torch, capi, W, a, b, od, timer, warmup)
        r["plain_us"] = round(t["launch_ms"] * 1e3, 3)
        out[label] = r
        print(f"[bench] ablation {label}: " + json.dumps(dict({k: r[k] for k, _ in SPMM_PARTS}, plain=r["plain_us"])), file=sys.stderr,
              flush=True)

    for d in (0.25, 0.5):
        w = W.workload_spmm_sweep(d)
        spmm(f"c2_{int(d * 100)}_f32", w["a"], w["b"], "f32")
    w = W.workload_spmm_skewed()
    spmm("c4", w["a"], w["b"], "f32")
    spmm("c4_sweep_kernel", w["a"], w["b"], "f32", {"BSP_SPMM_SWEEP": "2"})
    del w
    a, b = pattern_workload(W, "random", 0.5), pattern_b(W)
    spmm("8192c_256_random50_bf16", a, b, "bf16")
    del a, b
    s3 = W.workload_sddmm()

    def one_sddmm():
        t, fl, nb, info = bench_sddmm(torch, capi, W, s3["mask"], s3["x"], s3["y"], capi.ROW_MAJOR, "f32", timer,
                                      warmup, lib=tl)
        return round(t["launch_ms"] * 1e3, 3)
    out["c3_sddmm"] = decompose(torch, capi, tl, SDDMM_PARTS, one_sddmm)
    t, *_ = bench_sddmm(torch, capi, W, s3["mask"], s3["x"], s3["y"], capi.ROW_MAJOR, "f32", timer, warmup)
    out["c3_sddmm"]["plain_us"] = round(t["launch_ms"] * 1e3, 3)
    return out


def ablation(torch, capi, W, timer, warmup):
    """The cost decomposition, load balancing on and off, and the
    per-workgroup timelines."""
    rec = {"balance": [], "timeline": {}}
    rec["decomposition"] = decomposition(torch, capi, W, warmup)
    published = {"tril": (43.31, 29.5), "triu": (29.6, 24.88)}  # N150 DDA with / without LB, 8192, R=C=256
    w = W.workload_spmm_skewed()
    for label, env in (("skewed 16384^2, persistent kernel", {}),
                       ("skewed 16384^2, per-item kernels", {"BSP_SPMM_STREAM": "0"})):
        row = {"workload": label}
        for lb in ("1", "0"):
            with plan_env(dict(env, BSP_SPMM_BALANCE=lb)):
                t, fl, nb, info, _ = bench_spmm(torch, capi, W, w["a"], w["b"], "f32", timer, warmup)
            row["balanced" if lb == "1" else "unbalanced"] = {"us": round(t["launch_ms"] * 1e3, 3),
                                                              "tflops": round(fl / (t["launch_ms"] * 1e-3) / 1e12, 1),
                                                              "kernel_us": t.get("kernel_us") and round(t["kernel_us"], 3),
                                                              "plan": plan_summary(info)}
        row["speedup"] = round(row["unbalanced"]["us"] / row["balanced"]["us"], 3)
        rec["balance"].append(row)
    lt = Timer(torch, max(10, timer.steps // 10), trace=timer.trace)
    b = pattern_b(W)
    for pat in ("tril", "triu"):
        a = pattern_workload(W, pat, 1.0)
        row = {"workload": f"{pat} 8192^3, 256x256 blocks ({a.nblocks} blocks), bf16 C",
               "reference_n150_dda_tflops": {"balanced": published[pat][0], "unbalanced": published[pat][1]}}
        for lb in ("1", "0"):
            with plan_env({"BSP_SPMM_BALANCE": lb}):
                t, fl, nb, info, _ = bench_spmm(torch, capi, W, a, b, "bf16", lt, max(5, warmup // 2))
            row["balanced" if lb == "1" else "unbalanced"] = {"us": round(t["launch_ms"] * 1e3, 3),
                                                              "tflops": round(fl / (t["launch_ms"] * 1e-3) / 1e12, 1),
                                                              "plan": plan_summary(info)}
        row["speedup"] = round(row["unbalanced"]["us"] / row["balanced"]["us"], 3)
        rec["balance"].append(row)
        del a
    del b
    # timelines
    w25 = W.workload_spmm_sweep(0.25)
    rec["timeline"]["c2_25_f32"] = timeline_spmm(torch, capi, W, w25["a"], w25["b"], "f32", {}, "persistent")
    rec["timeline"]["c4_persistent"] = timeline_spmm(torch, capi, W, w["a"], w["b"], "f32", {}, "persistent")
    rec["timeline"]["c4_persistent_unbalanced"] = timeline_spmm(torch, capi, W, w["a"], w["b"], "f32",
                                                                {"BSP_SPMM_BALANCE": "0"}, "persistent")
    rec["timeline"]["c4_sweep"] = timeline_spmm(torch, capi, W, w["a"], w["b"], "f32", {"BSP_SPMM_SWEEP": "2"},
                                                "sweep")
    s3 = W.workload_sddmm()
    rec["timeline"]["c3_sddmm"] = timeline_sddmm(torch, capi, W, s3["mask"], s3["x"], s3["y"], "f32")
    rec["summary"] = {
        "decomposition_us": {k: dict({p: v[p] for p, _ in (SDDMM_PARTS if k.startswith("c3") else SPMM_PARTS)},
                                     plain=v["plain_us"])
                             for k, v in rec["decomposition"].items()},
        "lb_speedup": {r["workload"].split(",")[0].split(" ")[0] + ("_items" if "per-item" in r["workload"] else ""):
                       r["speedup"] for r in rec["balance"]},
        "timeline_p50_us": {k: {"start": v["start_offset_us"]["p50"],
                                "landing": v["first_landing_us"]["p50"] if v.get("first_landing_us") else None,
                                "end": v["end_us"]["p50"], "span": v["span_us"]}
                            for k, v in rec["timeline"].items() if v.get("workgroups")}}
    return rec


# ---------------------------------------------------------------------------
# The result line.  Full per-section records go to a side file; the last
# stdout line carries the headline (the largest single-GPU configuration, the
# skewed 16384^2 SpMM) and one compact row per configuration.
HEADLINE_MAX_BYTES = 8192


def floor_us(flops, nbytes, roofs):
    """Attainable time of one launch: the empty launch (graph replay of an
    empty kernel, same run) plus the longer of the algorithmic bytes at the
    measured HBM stream rate and the FLOPs at the MFMA peak."""
    t_hbm = nbytes / (roofs["hbm_stream_tbs"] * 1e12) * 1e6
    t_mfma = flops / (PEAK_BF16_TFLOPS * 1e12) * 1e6
    return round(roofs["empty_launch_us"] + max(t_hbm, t_mfma), 3)


def _row(rec, roofs):
    us = rec["us_per_launch"]
    r = {"us": us, "kernel_us": rec.get("kernel_us"), "tflops": round(rec["tflops"], 1),
         "mfma": round(rec["frac_mfma_peak"], 4), "hbm": round(rec["frac_hbm_peak"], 4)}
    if rec.get("kernel_us"):
        r["kernel_hbm"] = round(rec["kernel_frac_hbm_peak"], 4)
    tr = rec.get("traffic")
    if tr:
        r["traffic_x"] = tr["ratio_to_algorithmic"]
    if roofs:
        f = floor_us(rec["flops"], rec["bytes"], roofs)
        r["floor_us"] = f
        r["frac_of_floor"] = round(f / us, 3)
    cpu = rec.get("cpu")
    if cpu and "single" in cpu:
        r["cpu_x"] = [cpu["single"].get("gpu_speedup"), cpu["all"].get("gpu_speedup")]
    return r


def summary_rows(out, roofs):
    """One compact row per configuration: replay us, kernel us, TFLOP/s,
    fractions of the MFMA and HBM peaks, measured traffic over algorithmic
    bytes, the attainable floor and the fraction of it reached, and the GPU
    speedup over the one-thread and all-core CPU oracle."""
    rows = {}
    if "c1" in out:
        rows["c1"] = _row(out["c1"], roofs)
    for rec in out.get("sweep", []):
        if rec.get("warm_cache"):
            continue
        r = _row(rec, roofs)
        if rec["density"] == 0.25 and rec["out"] == "f32" and "plan" in rec and "n_entries" in rec["plan"]:
            r["on_chip_frac"] = on_chip_roof(rec["plan"], rec["us_per_launch"], roofs)["frac"]
        rows[f"c2_{int(round(rec['density'] * 100))}_{rec['out']}"] = r
    if "sddmm" in out:
        rows["c3"] = _row(out["sddmm"], roofs)
    if "skewed" in out:
        rows["c4"] = _row(out["skewed"], roofs)
    if "attention" in out:
        at = out["attention"]
        rows["c5_sddmm"] = _row(at["sddmm"], roofs)
        rows["c5_spmm"] = _row(at["spmm"], roofs)
        rows["c5_fused"] = _row(dict(at["fused"], cpu=at.get("cpu")), roofs)
    if "spgemm" in out:
        for r in out["spgemm"]["runs"]:
            rows[f"spgemm_{r['out']}"] = _row(r, roofs)
    if "large_blocks" in out:
        for r in out["large_blocks"]["runs"]:
            rows[f"8192c_256_{r['out']}"] = _row(r, roofs)
    if "block_sizes" in out:
        for r in out["block_sizes"]["runs"]:
            rows[f"8192c_{r['R']}_f32"] = _row(r, roofs)
    if "patterns" in out:
        for r in out["patterns"]["runs"]:
            key = f"pat_{r['pattern']}" + ("" if r["pattern"] in ("tril", "triu") else f"_{int(round(r['density'] * 100))}")
            rows[key] = {"tflops": round(r["tflops"], 1), "mfma": round(r["frac_mfma_peak"], 4),
                         "n150_dda_tflops": r.get("reference_dda_tflops_n150")}
    if "ablation" in out:
        rows["ablation"] = out["ablation"].get("summary")
    if "host_entry" in out:
        rows["host_ms"] = out["host_entry"]["ms_per_call"]
    return rows


def build_headline(out, roofs, big, steps, warmup, sections_path):
    """The result line: the skewed 16384^2 SpMM (the largest single-GPU
    configuration) as `value`, its HBM roofline (it is HBM-bound: 99 FLOP per
    algorithmic byte) and CPU baseline, and the per-configuration summary."""
    rec = out["skewed"]
    us = rec["us_per_launch"]
    kname = next(iter(rec.get("kernels") or {}), None)
    tr = rec.get("traffic", {}).get("bytes_per_launch")
    rl = roofline(rec["flops"], rec["bytes"], us, tr, kname)
    for k in ("algorithmic_flop_per_launch", "algorithmic_bytes_per_launch"):
        rl.pop(k, None)
    rl.update({"bytes_per_launch": rec["bytes"], "flop_per_launch": rec["flops"],
               "traffic_source": rec.get("traffic", {}).get("source"),
               "floor_us": floor_us(rec["flops"], rec["bytes"], roofs),
               "hbm_stream_tbs": roofs["hbm_stream_tbs"], "empty_launch_us": roofs["empty_launch_us"],
               "mfma_attainable_tflops": big["tflops"]})
    rl["frac_of_floor"] = round(rl["floor_us"] / us, 4)
    if rec.get("kernel_us"):
        rl["kernel_us"] = rec["kernel_us"]
        rl["kernel_frac"] = round(rec["bytes"] / (rec["kernel_us"] * 1e-6) / 1e9 / PEAK_HBM_GBS, 4)
    cpu = None
    if "cpu" in rec:
        c = rec["cpu"]
        cpu = {"value": c["all"]["tflops"], "unit": "TFLOP/s", "cores": c["all"]["cores"], "kind": "port",
               "sample": f"{c['all']['sample']} of the skewed workload, OpenMP over block rows; median of 3 runs "
                         f"after 1 warm-up: {c['all']['seconds']} s",
               "single_core": {"value": c["single"]["tflops"], "cores": 1,
                               "sample": f"{c['single']['sample']}: {c['single']['seconds']} s"},
               "gpu_speedup": [c["single"]["gpu_speedup"], c["all"]["gpu_speedup"]]}
    return {
        "metric": "effective TFLOP/s on nonzero blocks (SpMM, SDDMM); % bf16 MFMA peak / % HBM BW",
        "value": round(rec["tflops"], 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(us * 1e-3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded xoshiro256**: Zipf(1.2) row counts, uniform block columns, U[-1,1] bf16 values)",
        "config": {"workload": "skewed BSR SpMM C=A*B: A 16384x16384, 32x32 blocks, Zipf(1.2) blocks per block row "
                               "capped at 512, 2% mean density (5243 blocks), B 16384x1024 bf16, fp32 accumulate, "
                               "fp32 C",
                   "M": 16384, "K": 16384, "N": 1024, "block": [32, 32], "nnzb": rec["nnzb"],
                   "max_row_blocks": rec.get("max_row_blocks"), "input_sha256": rec.get("input_sha256"),
                   "timing": "graph replay of `steps` launches between two HIP events on the launch stream; "
                             "inputs rotated over > 512 MB of copies",
                   "peaks": {"bf16_mfma_tflops": PEAK_BF16_TFLOPS, "hbm_gbs": PEAK_HBM_GBS,
                             "source": "AMD Instinct MI355X published dense figures"}},
        "roofline": rl,
        "cpu_baseline": cpu,
        "summary": summary_rows(out, roofs),
        "sections": sections_path,
    }


if __name__ == "__main__":
    main()
