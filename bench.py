"""Headline benchmark: FP32 column-major NN SGEMM at 4096^3 on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload cfg3] [--layout nn]

A step is one launch of the tuned gfx950 kernel on the BASELINE.json config
(M = N = K = 4096, A and B uniform[-1, 1) from seed 2, C = 0, alpha = 1,
beta = 0) with A, B and D resident in HBM.  W untimed launches, then K timed
launches bracketed by device synchronisation; the host clock gives
ms_per_step and `value` (TFLOP/s), HIP events on the kernel's stream give the
per-launch kernel time used for the roofline fraction.  W defaults to at least
10 launches and at least 0.25 s of them: the engine clock ramps up over
milliseconds of load, which is all of a short workload's 10 launches.

The CPU baseline is the reference's own cpuGemm (compiled from its source into
oracle/_ref) -- or this project's C restatement of it when that was not built --
timed single-threaded on a column slice D[:, :s] of the same workload (the
slice is itself a cpuGemm call with n = s, so per-output work and memory
pattern are unchanged); s is calibrated to about 15 s of CPU time.  The slice
is also compared with the GPU result (normwise error, 1e-5 * sqrt(K) bar), and
both float32 results with the float64 product of the same inputs.  A second,
separately labelled CPU figure (cpu_baseline.parallel) runs the same loop over
columns on up to 16 host threads (about 5 s).

--layout tn / nt / tt stores A (k x m) and/or B (n x k) transposed and runs
the instance catalog.select picks for that layout (op(A) = A^T, op(B) = B^T);
the CPU baseline multiplies the transposed-back operands.

Prints one JSON line on stdout; progress goes to stderr.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "amdgpu-arch-gemm_amd"))

import numpy as np  # noqa: E402

from generator import catalog  # noqa: E402
from shim import sgemm_shim as S  # noqa: E402

FP32_MFMA_PEAK_TFLOPS = 157.3  # MI355X dense FP32 matrix peak (256 CU x 256 FLOP/clk x 2.4 GHz)
HBM_PEAK_GBS = 8000.0

WORKLOADS = {
    # name: (m, n, k, seed, dist)
    "cfg3": (4096, 4096, 4096, 2, S.SGEMM_DIST_UNIFORM),
    "cfg2": (1024, 1024, 1024, 1, S.SGEMM_DIST_UNIFORM),
    "cfg4": (8192, 8192, 256, 3, S.SGEMM_DIST_NORMAL),
    "cfg5": (16384, 128, 4096, 4, S.SGEMM_DIST_UNIFORM),
    # not a BASELINE.json config: few output tiles and a deep K, the case the
    # split-K kernel exists for (64 tiles of 64 x 64, 4 K ranges each, on 256
    # compute units)
    "deepk": (512, 512, 16384, 5, S.SGEMM_DIST_UNIFORM),
    # not a BASELINE.json config: one past the headline in every dimension, so
    # a fixed tile grid leaves one-row and one-column sliver tiles (edge
    # strips) and a partial last round
    "q4097": (4097, 4097, 4097, 6, S.SGEMM_DIST_UNIFORM),
}
# BASELINE.json's metric, verbatim
HEADLINE_METRIC = "FP32 SGEMM TFLOP/s at 4096\u00b3 NN; % of MI355X FP32 MFMA peak"


def log(msg: str):
    print(msg, file=sys.stderr, flush=True)


def read_traffic(kernel: str, workload: str):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary, if any."""
    path = os.path.join(ROOT, "profiles", f"{kernel}_{workload}_traffic.txt")
    if not os.path.exists(path):
        return None
    vals = {}
    with open(path) as f:
        for line in f:
            if ":" in line and not line.startswith("#"):
                key, val = line.split(":", 1)
                vals[key.strip()] = val.strip()
    try:
        return float(vals["hbm_bytes_per_launch"])
    except (KeyError, ValueError):
        return None


def host_cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), or the platform's processor string."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def cpu_baseline(A, B, D_gpu, m, n, k, target_s: float):
    """Times the reference cpuGemm (or the oracle port) on a column slice."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle

    use_ref = oracle.ref_lib() is not None
    gemm = oracle.ref_cpu_gemm if use_ref else oracle.cpu_gemm
    kind = "reference" if use_ref else "port"

    def timed(cols):
        Bs = np.asfortranarray(B[:, :cols])
        t0 = time.perf_counter()
        D = gemm(A, Bs, None, 1.0, 0.0)
        return time.perf_counter() - t0, D

    probe = 4
    t_probe, _ = timed(probe)
    cols = int(max(probe, min(n, round(target_s / max(t_probe / probe, 1e-9)))))
    log(f"cpu baseline ({kind}): {probe} columns took {t_probe:.2f} s; timing {cols} columns")
    t, D = timed(cols)
    tflops = 2.0 * m * cols * k / t / 1e12
    err = oracle.normwise_error(D_gpu[:, :cols], D)
    # both float32 results against the float64 product of the same inputs
    D64 = A.astype(np.float64) @ B[:, :cols].astype(np.float64)
    # labelled separately: the same loop over columns on the host's cores (the
    # box's share: at most 16), each output keeping its summation order, so
    # the result is bitwise the single-thread one
    threads = max(1, min(16, os.cpu_count() or 1))
    cols_mt = int(min(n, max(threads, round(cols * threads * 5.0 / max(t, 1e-9)))))
    Bm = np.asfortranarray(B[:, :cols_mt])
    t0 = time.perf_counter()
    D_mt = oracle.cpu_gemm_mt(A, Bm, None, 1.0, 0.0, threads=threads)
    t_mt = time.perf_counter() - t0
    overlap = min(cols, cols_mt)
    parallel = {
        "value": 2.0 * m * cols_mt * k / t_mt / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
        "sample": f"D[:, :{cols_mt}] of the same workload, columns over {threads} threads, {t_mt:.1f} s",
        "bitwise_equal_to_single_thread": bool(np.array_equal(D_mt[:, :overlap], D[:, :overlap])),
    }
    return {
        "value": tflops,
        "unit": "TFLOP/s",
        "cores": 1,
        "host_cpu": host_cpu_model(),
        "host_cores": os.cpu_count(),
        "kind": kind,
        "sample": f"D[:, :{cols}] of the {m}x{n}x{k} workload (n={cols} columns), single thread, {t:.1f} s",
        "seconds": t,
        "parallel": parallel,
    }, {"normwise_error": err, "tolerance": oracle.tolerance(k), "columns_checked": cols,
        "gpu_vs_f64": oracle.normwise_error(D_gpu[:, :cols], D64), "cpu_vs_f64": oracle.normwise_error(D, D64),
        "pass": bool(err <= oracle.tolerance(k))}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=None,
                    help="untimed launches before the timed ones (default: at least 10 and at least "
                         "0.25 s of launches, so the engine clock has left its idle state)")
    ap.add_argument("--workload", default="cfg3", choices=sorted(WORKLOADS))
    ap.add_argument("--kernel", default=None, help="catalog instance (default: catalog.select)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--split-k", type=int, default=None,
                    help="K ranges per output tile (0 = per problem; default: the instance's own setting)")
    ap.add_argument("--stream-k", type=int, default=None,
                    help="stream-K mode (0 off, 1 auto, 2 forced; default: the instance's own setting)")
    ap.add_argument("--no-edge", action="store_true", help="do not attach the catalog's edge kernel")
    ap.add_argument("--layout", default="nn", choices=["nn", "tn", "nt", "tt"],
                    help="operand layout: t stores A (k x m) or B (n x k) transposed")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build's SGEMM runs on a single MI355X "
              f"(--gpus {args.gpus} requested). Use --gpus 1.", file=sys.stderr)
        sys.exit(2)

    m, n, k, seed, dist = WORKLOADS[args.workload]
    ta, tb = args.layout[0] == "t", args.layout[1] == "t"
    name = args.kernel or catalog.select(m, n, k, ta, tb)
    co, toml = catalog.paths(name)
    info = S.device_info()
    log(f"device: {info}")
    log(f"workload {args.workload} {args.layout}: {m}x{n}x{k} seed {seed} dist {dist}; kernel {name}")

    A = S.fill_matrix(*((k, m) if ta else (m, k)), seed, 0, dist)
    B = S.fill_matrix(*((n, k) if tb else (k, n)), seed, 1, dist)
    kern = S.Kernel(co, toml)
    if (bool(kern.info.trans_a), bool(kern.info.trans_b)) != (ta, tb):
        kern.close()
        print(f"{name} is not a {args.layout} kernel", file=sys.stderr)
        sys.exit(2)
    edges = []
    if name in catalog.EDGE_KERNEL and not args.no_edge:
        edges = [S.Kernel(*catalog.paths(e)) for e in catalog.EDGE_KERNEL[name]]
        kern.set_edge_kernels(*edges)
    interior = kern.edge_interior(m, n, k)
    if interior != (m, n):
        log(f"edge strips: interior {interior[0]}x{interior[1]} on {name}, strips on {catalog.EDGE_KERNEL[name]}")
    if args.split_k is not None:
        kern.set_split_k(args.split_k)
    if args.stream_k is not None:
        kern.set_stream_k(args.stream_k)
    splits = kern.launch_splits(m, n, k)
    sk_tiles = kern.stream_k_tiles(m, n, k) if kern.info.stream_k_groups else 0
    log(f"K ranges per output tile: {splits}; stream-K tiles: {sk_tiles}")
    dA, dB = S.DeviceBuffer.from_array(A), S.DeviceBuffer.from_array(B)
    dD = S.DeviceBuffer(m * n * 4)
    dD.zero()

    if args.warmup is not None:
        warmup = args.warmup
        for _ in range(warmup):
            kern.launch(dA, dB, None, dD, m, n, k, 1.0, 0.0)
        kern.synchronize()
    else:
        # the engine clock ramps up over milliseconds of load: keep launching
        # until 0.25 s have passed (and at least 10 launches)
        warmup, t_w = 0, time.perf_counter()
        while warmup < 10 or time.perf_counter() - t_w < 0.25:
            for _ in range(10):
                kern.launch(dA, dB, None, dD, m, n, k, 1.0, 0.0)
            warmup += 10
            kern.synchronize()
    log(f"warmup: {warmup} launches")

    # timed region: exactly `steps` launches, device idle on both sides
    t0 = time.perf_counter()
    event_ms = kern.time(dA, dB, None, dD, m, n, k, 1.0, 0.0, warmup=0, runs=args.steps)
    kern.synchronize()
    wall_s = time.perf_counter() - t0

    flops = 2.0 * m * n * k
    ms_per_step = wall_s * 1e3 / args.steps
    value = flops / (wall_s / args.steps) / 1e12
    kernel_ms = event_ms / args.steps
    achieved = flops / (kernel_ms * 1e-3) / 1e12
    per_launch = kern.time_each(dA, dB, None, dD, m, n, k, 1.0, 0.0, runs=20)
    median_ms = float(np.median(per_launch))
    log(f"wall {ms_per_step:.4f} ms/step = {value:.2f} TFLOP/s; events {kernel_ms:.4f} ms/launch = "
        f"{achieved:.2f} TFLOP/s; per-launch median {median_ms:.4f} ms")

    D = dD.download().reshape(n, m).T
    # A, B read once and D written once; a split launch also writes and
    # reads its partials (4 bytes per output per K range), not counted here
    alg_bytes = 4.0 * (m * k + k * n + m * n)
    traffic = read_traffic(name, args.workload)
    line = {
        "metric": (HEADLINE_METRIC if (args.workload, args.layout) == ("cfg3", "nn")
                   else f"FP32 SGEMM TFLOP/s at {m}x{n}x{k} {args.layout.upper()}"),
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": f"sgemm_{args.layout}_colmajor_{m}x{n}x{k}",
            "m": m, "n": n, "k": k, "seed": seed,
            "dist": "uniform[-1,1)" if dist == S.SGEMM_DIST_UNIFORM else "normal(0,1)",
            "alpha": 1.0, "beta": 0.0,
            "kernel": name,
            "split_k": splits,
            "stream_k_tiles": sk_tiles,
            "edge_kernels": list(catalog.EDGE_KERNEL[name]) if interior != (m, n) else None,
            "pct_of_fp32_mfma_peak": round(100.0 * value / FP32_MFMA_PEAK_TFLOPS, 2),
            "device": info["name"],
            "peak_sclk_mhz": info["clock_khz"] / 1000.0,
        },
        "roofline": {
            "bound": "mfma",
            "achieved": round(achieved, 3),
            "peak": FP32_MFMA_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / FP32_MFMA_PEAK_TFLOPS, 4),
            "traffic": traffic,
            "kernel_ms_mean": round(kernel_ms, 5),
            "kernel_ms_median": round(median_ms, 5),
            "algorithmic_bytes": alg_bytes,
            "algorithmic_gbs": round(alg_bytes / (kernel_ms * 1e-3) / 1e9, 1),
        },
    }
    if not args.no_cpu_baseline and args.gpus == 1:
        opA = np.asfortranarray(A.T) if ta else A
        opB = np.asfortranarray(B.T) if tb else B
        cpu, parity = cpu_baseline(opA, opB, D, m, n, k, args.cpu_seconds)
        line["cpu_baseline"] = cpu
        line["parity"] = parity
    else:
        line["cpu_baseline"] = None
    kern.close()
    for e in edges:
        e.close()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
