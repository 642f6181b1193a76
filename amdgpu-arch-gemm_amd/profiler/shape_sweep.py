"""TFLOP/s of the default selection path over a list of shapes.

For each m x n x k the instance is ``catalog.select(m, n, k)`` with the
catalog's edge-strip kernels attached and the handle's default split-K and
stream-K settings -- what a caller of the library gets without tuning.  Inputs
are U[-1,1) (seed 3), alpha = 1, beta = 0, resident on the device.  The clock
is warmed with 0.5 s of launches first; then ``--rounds`` interleaved rounds
over the shapes, each timing at least ~3 ms of back-to-back launches, and the
median per shape is reported, with its K ranges and stream-K tiles.

    python amdgpu-arch-gemm_amd/profiler/shape_sweep.py --shapes 2048x2048x2048,3000x3000x3000 \\
        --summary out/default_path_shapes.md
"""
import argparse
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
from generator import catalog  # noqa: E402
from shim import sgemm_shim as S  # noqa: E402

PEAK = 157.3  # TFLOP/s, MI355X dense FP32 MFMA


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--shapes", required=True, help="comma-separated MxNxK")
    ap.add_argument("--rounds", type=int, default=5)
    ap.add_argument("--summary", default=None, help="markdown summary path")
    args = ap.parse_args(argv)
    shapes = [tuple(int(x) for x in s.lower().split("x")) for s in args.shapes.split(",") if s.strip()]
    kerns, edges = {}, []

    def kernel(name):
        if name not in kerns:
            k = S.Kernel(*catalog.paths(name))
            if name in catalog.EDGE_KERNEL:
                e = [S.Kernel(*catalog.paths(x)) for x in catalog.EDGE_KERNEL[name]]
                edges.extend(e)  # they must stay open while attached
                k.set_edge_kernels(*e)
            kerns[name] = k
        return kerns[name]

    bufs = {}
    for (m, n, k) in shapes:
        bufs[(m, n, k)] = (S.DeviceBuffer.from_array(S.fill_matrix(m, k, 3, 0)),
                           S.DeviceBuffer.from_array(S.fill_matrix(k, n, 3, 1)), S.DeviceBuffer(m * n * 4))
    first = shapes[0]
    kk = kernel(catalog.select(*first))
    t0 = time.time()
    while time.time() - t0 < 0.5:
        kk.time(*bufs[first][:2], None, bufs[first][2], *first, warmup=0, runs=5)
    times = {sh: [] for sh in shapes}
    for r in range(args.rounds):
        for sh in shapes:
            kk = kernel(catalog.select(*sh))
            dA, dB, dD = bufs[sh]
            reps = max(5, int(3e-3 / (2.0 * sh[0] * sh[1] * sh[2] / 140e12)))
            kk.time(dA, dB, None, dD, *sh, warmup=2, runs=1)
            times[sh].append(kk.time(dA, dB, None, dD, *sh, warmup=0, runs=reps) / reps)
        print(f"round {r} done", flush=True)
    rows = []
    for sh in shapes:
        m, n, k = sh
        name = catalog.select(*sh)
        kk = kernel(name)
        med = float(np.median(times[sh]))
        tf = 2.0 * m * n * k / med / 1e9
        sk = kk.stream_k_tiles(m, n, k) if kk.info.stream_k_groups else 0
        interior = kk.edge_interior(m, n, k)
        rows.append((f"{m}x{n}x{k}", name, kk.launch_splits(m, n, k), sk,
                     "" if interior == (m, n) else f"{interior[0]}x{interior[1]}", med * 1e3, tf))
        print(f"{m}x{n}x{k}: {tf:7.2f} TFLOP/s ({med * 1e3:.1f} us) {name}", flush=True)
    if args.summary:
        os.makedirs(os.path.dirname(os.path.abspath(args.summary)), exist_ok=True)
        with open(args.summary, "w") as f:
            f.write("# Default selection path over shapes\n\nCommand (from the repository root on the GPU box):\n\n")
            f.write("    python amdgpu-arch-gemm_amd/profiler/shape_sweep.py --shapes " + args.shapes
                    + f" --rounds {args.rounds} --summary {args.summary}\n\n")
            f.write("`catalog.select(m, n, k)` with the catalog's edge kernels and the default split-K / stream-K "
                    "settings; U[-1,1) seed 3, alpha 1, beta 0; 0.5 s of warm-up launches, then "
                    f"{args.rounds} interleaved rounds; median per shape.\n\n")
            f.write("| shape | instance | K ranges | stream-K tiles | edge-strip interior | us | TFLOP/s | % of 157.3 |\n")
            f.write("|---|---|---|---|---|---|---|---|\n")
            for shape, name, splits, sk, interior, us, tf in rows:
                f.write(f"| {shape} | `{name}` | {splits} | {sk} | {interior or '-'} | {us:.1f} | {tf:.2f} | "
                        f"{100.0 * tf / PEAK:.1f} |\n")
    for k in list(kerns.values()) + edges:
        k.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
