"""Times the vendor's FP32 GEMM on the BASELINE shapes, for comparison.

    python vendor_gemm.py [--workloads cfg3,cfg2,cfg4,cfg5] [--steps 100] [--json out.json]

PyTorch-ROCm's ``torch.mm`` on float32 reaches rocBLAS (``preferred_blas_library
("cublas")``) or hipBLASLt (``"cublaslt"``).  The product is laid out as this
package's kernel computes it: column-major A (m x k), B (k x n) and D (m x n) are
the row-major tensors A^T (k x m), B^T (n x k) and D^T (n x m), and
D^T = B^T A^T is one ``torch.mm`` with no transposed operand.  TF32-style
reduced precision is switched off (``allow_tf32 = False``, precision
"highest"), and each result is checked against the float64 product of the same
inputs on sampled columns (max|D - D64| / max|D64|, next to the 1e-5 sqrt(K)
bar the package's kernels meet).

Per workload and library: at least 10 and at least 0.25 s of untimed launches
(the engine clock leaves its idle state), then ``--steps`` back-to-back
launches between two events (the mean) and 50 single launches each between
their own events (the median).  This is the protocol ``bench.py`` uses for its
ramped figures, so the two are comparable when run on the same box.  One JSON
object per line on stdout.

``--interleaved ROUNDS`` instead times this package's instance
(``catalog.select``, with its edge kernels and default split-K / stream-K) and
both libraries on the same inputs (U[-1,1) or N(0,1), seed 3, from
``sgemm_fill``) in one process: after 0.5 s of warm-up launches of each, ROUNDS
rounds of two untimed and then ``--burst-ms`` (default 2) of back-to-back
launches per entry, the order reversed every other round (the first timing
after another entry can be off by 1-3% either way), and the median per entry.
The first launches after a switch of kernel run slower for every entry, so
short bursts measure that transition and long ones the steady state.
"""
from __future__ import annotations

import argparse
import json
import math
import statistics
import sys
import time

import torch

FP32_MFMA_PEAK_TFLOPS = 157.3

WORKLOADS = {
    # name: (m, n, k, normal-distributed inputs)
    "cfg2": (1024, 1024, 1024, False),
    "cfg3": (4096, 4096, 4096, False),
    "cfg4": (8192, 8192, 256, True),
    "cfg5": (16384, 128, 4096, False),
}
LIBRARIES = (("rocblas", "cublas"), ("hipblaslt", "cublaslt"))


def _inputs(m, n, k, normal, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    if normal:
        at = torch.randn((k, m), generator=g, device="cuda", dtype=torch.float32)
        bt = torch.randn((n, k), generator=g, device="cuda", dtype=torch.float32)
    else:
        at = torch.rand((k, m), generator=g, device="cuda", dtype=torch.float32) * 2 - 1
        bt = torch.rand((n, k), generator=g, device="cuda", dtype=torch.float32) * 2 - 1
    return at, bt


def _error_vs_f64(at, bt, dt, cols=64):
    """Normwise error of sampled columns of D against the float64 product."""
    n = bt.shape[0]
    idx = torch.linspace(0, n - 1, min(cols, n), device="cuda").round().long().unique()
    ref = (bt[idx].double() @ at.double())          # rows of D^T = columns of D
    got = dt[idx].double()
    return float((got - ref).abs().max() / ref.abs().max())


def time_library(m, n, k, normal, steps, seed=0):
    at, bt = _inputs(m, n, k, normal, seed)
    dt = torch.empty((n, m), device="cuda", dtype=torch.float32)
    flops = 2.0 * m * n * k

    def launch():
        torch.mm(bt, at, out=dt)

    launch()
    torch.cuda.synchronize()
    err = _error_vs_f64(at, bt, dt)
    warm, t0 = 0, time.perf_counter()
    while warm < 10 or time.perf_counter() - t0 < 0.25:
        launch()
        warm += 1
        if warm % 10 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        launch()
    e1.record()
    torch.cuda.synchronize()
    mean_ms = e0.elapsed_time(e1) / steps
    singles = []
    for _ in range(50):
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s0.record()
        launch()
        s1.record()
        s1.synchronize()
        singles.append(s0.elapsed_time(s1))
    med_ms = statistics.median(singles)
    return {
        "warmup_launches": warm,
        "ms_mean": mean_ms,
        "tflops_mean": flops / (mean_ms * 1e-3) / 1e12,
        "ms_median_single": med_ms,
        "tflops_median_single": flops / (med_ms * 1e-3) / 1e12,
        "frac_of_peak": flops / (mean_ms * 1e-3) / 1e12 / FP32_MFMA_PEAK_TFLOPS,
        "error_vs_f64": err,
        "tolerance": 1e-5 * math.sqrt(k),
    }


def interleaved(workloads, rounds, out=None, burst_ms=2.0):
    """Interleaved timing of this package and both vendor libraries."""
    import os
    import numpy as np
    here = os.path.dirname(os.path.abspath(__file__))
    sys.path.insert(0, os.path.dirname(here))
    from generator import catalog
    from shim import sgemm_shim as S
    for wl in workloads:
        m, n, k, normal = WORKLOADS[wl]
        dist = S.SGEMM_DIST_NORMAL if normal else S.SGEMM_DIST_UNIFORM
        A, B = S.fill_matrix(m, k, 3, 0, dist), S.fill_matrix(k, n, 3, 1, dist)
        dA, dB, dD = S.DeviceBuffer.from_array(A), S.DeviceBuffer.from_array(B), S.DeviceBuffer(4 * m * n)
        # column-major A (m x k) is the row-major tensor A^T (k x m); D^T = B^T A^T
        at = torch.from_numpy(np.ascontiguousarray(A.T)).cuda()
        bt = torch.from_numpy(np.ascontiguousarray(B.T)).cuda()
        dt = torch.empty((n, m), device="cuda", dtype=torch.float32)
        name = catalog.select(m, n, k)
        kern = S.Kernel(*catalog.paths(name))
        edges = [S.Kernel(*catalog.paths(e)) for e in catalog.EDGE_KERNEL.get(name, ())]
        if edges:
            kern.set_edge_kernels(*edges)
        flops = 2.0 * m * n * k
        reps = max(5, int(burst_ms * 1e-3 / (flops / 140e12)))

        def ours(r):
            return kern.time(dA, dB, None, dD, m, n, k, warmup=0, runs=r) / r

        def vendor(backend):
            def run(r):
                torch.backends.cuda.preferred_blas_library(backend)
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(r):
                    torch.mm(bt, at, out=dt)
                e1.record()
                torch.cuda.synchronize()
                return e0.elapsed_time(e1) / r
            return run

        entries = [(f"this build ({name})", ours)] + [(label, vendor(b)) for label, b in LIBRARIES]
        for _, fn in entries:
            t0 = time.perf_counter()
            while time.perf_counter() - t0 < 0.5:
                fn(10)
        times = {label: [] for label, _ in entries}
        for r in range(rounds):
            for label, fn in (entries if r % 2 == 0 else entries[::-1]):
                fn(2)
                times[label].append(fn(reps))
        cols = sorted({0, n // 2, n - 1})
        ref = np.asarray(A, np.float64) @ np.asarray(B, np.float64)[:, cols]
        errs = {}
        kern.launch(dA, dB, None, dD, m, n, k)
        kern.synchronize()
        got = dD.download().reshape(n, m).T[:, cols]
        errs[entries[0][0]] = float(np.abs(got - ref).max() / np.abs(ref).max())
        for label, backend in LIBRARIES:
            torch.backends.cuda.preferred_blas_library(backend)
            torch.mm(bt, at, out=dt)
            torch.cuda.synchronize()
            got = dt.cpu().numpy().T[:, cols]
            errs[label] = float(np.abs(got - ref).max() / np.abs(ref).max())
        for label, _ in entries:
            ms = statistics.median(times[label])
            rec = {"mode": "interleaved", "workload": wl, "m": m, "n": n, "k": k, "entry": label,
                   "rounds": rounds, "launches_per_timing": reps, "ms_median": ms,
                   "tflops_median": flops / (ms * 1e-3) / 1e12,
                   "tflops_min": flops / (max(times[label]) * 1e-3) / 1e12,
                   "tflops_max": flops / (min(times[label]) * 1e-3) / 1e12,
                   "error_vs_f64": errs[label], "tolerance": 1e-5 * math.sqrt(k),
                   "device": torch.cuda.get_device_name(0), "torch": torch.__version__}
            line = json.dumps(rec)
            print(line, flush=True)
            if out:
                out.write(line + "\n")
                out.flush()
        for x in [kern] + edges:
            x.close()
        for x in (dA, dB, dD):
            x.close()


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--workloads", default="cfg3,cfg2,cfg4,cfg5")
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--json", default=None, help="also append the lines to this file")
    ap.add_argument("--interleaved", type=int, default=0, metavar="ROUNDS",
                    help="time this package's instance and both libraries round-robin instead")
    ap.add_argument("--burst-ms", type=float, default=2.0, help="length of each interleaved timing")
    args = ap.parse_args()
    if not torch.cuda.is_available():
        print("vendor_gemm: no GPU visible", file=sys.stderr)
        return 1
    torch.backends.cuda.matmul.allow_tf32 = False
    torch.set_float32_matmul_precision("highest")
    out = open(args.json, "a") if args.json else None
    if args.interleaved:
        interleaved(args.workloads.split(","), args.interleaved, out, args.burst_ms)
        if out:
            out.close()
        return 0
    for wl in args.workloads.split(","):
        m, n, k, normal = WORKLOADS[wl]
        for label, backend in LIBRARIES:
            torch.backends.cuda.preferred_blas_library(backend)
            print(f"[vendor_gemm] {wl} {m}x{n}x{k} {label}", file=sys.stderr, flush=True)
            rec = {"workload": wl, "m": m, "n": n, "k": k, "library": label,
                   "device": torch.cuda.get_device_name(0), "torch": torch.__version__}
            rec.update(time_library(m, n, k, normal, args.steps))
            line = json.dumps(rec)
            print(line, flush=True)
            if out:
                out.write(line + "\n")
                out.flush()
    if out:
        out.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
