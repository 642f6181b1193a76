"""Times the catalog's time-model candidates on many shapes (GPU).

    python select_sweep.py --name fit --shapes 1024x1024x1024,4096x4096x256,... [--rounds 3]
                           [--extra inst1,inst2] --out sweep.json

Every shape is timed over all candidates (``catalog.CANDIDATES`` plus
``--extra``) round-robin, ``--rounds`` times, the order reversed every other
round, and the median launch time is kept, so that the clock state is shared
by the instances compared on a shape and none always runs first (the first
timing after another shape's launches can be off by 1-3% either way).
Each instance launches with its own split-K / stream-K setting (split-K per
problem where the code object carries the kernel) and without edge kernels:
what ``predicted_launch_seconds`` models.  Inputs are U[-1, 1), alpha = 1,
beta = 0.  The output appends one sweep ``{"name", "shapes": [{"shape",
"tflops": {instance: TFLOP/s}}]}`` to ``--out`` (created if absent), the format
of tests/golden/select_measured.json, which ``tuner/fit_time_model.py`` fits.
"""
from __future__ import annotations

import argparse
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))

import numpy as np  # noqa: E402

from generator import catalog  # noqa: E402
from shim import sgemm_shim as S  # noqa: E402


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--name", required=True)
    ap.add_argument("--shapes", required=True, help="comma-separated MxNxK")
    ap.add_argument("--rounds", type=int, default=3)
    ap.add_argument("--extra", default="", help="more catalog instances to time")
    ap.add_argument("--out", required=True)
    args = ap.parse_args()
    cands = list(catalog.CANDIDATES) + [e for e in args.extra.split(",") if e and e not in catalog.CANDIDATES]
    shapes = [tuple(int(x) for x in s.split("x")) for s in args.shapes.split(",")]
    kerns = {}
    for c in cands:
        kern = S.Kernel(*catalog.paths(c))
        if kern.info.split_k_max > 1:
            kern.set_split_k(0)
        kerns[c] = kern
    doc = json.load(open(args.out)) if os.path.exists(args.out) else {"sweeps": []}
    sweep = {"name": args.name, "shapes": []}
    doc["sweeps"].append(sweep)
    for (m, n, k) in shapes:
        A, B = S.fill_matrix(m, k, 3, 0), S.fill_matrix(k, n, 3, 1)
        dA, dB, dD = S.DeviceBuffer.from_array(A), S.DeviceBuffer.from_array(B), S.DeviceBuffer(m * n * 4)
        del A, B
        flops = 2.0 * m * n * k
        runs = max(3, min(40, int(1.2e14 / flops)))   # about 1 ms of launches per timing
        times = {c: [] for c in cands}
        for r in range(args.rounds):
            for c in (cands if r % 2 == 0 else cands[::-1]):
                kerns[c].time(dA, dB, None, dD, m, n, k, warmup=2, runs=1)
                times[c].append(kerns[c].time(dA, dB, None, dD, m, n, k, warmup=0, runs=runs) / runs)
        tf = {c: round(flops / (float(np.median(times[c])) * 1e-3) / 1e12, 1) for c in cands}
        sweep["shapes"].append({"shape": [m, n, k], "tflops": tf})
        best = max(tf, key=tf.get)
        print(f"{m}x{n}x{k}: best {best} {tf[best]:.1f}; select() {catalog.select(m, n, k)}", flush=True)
        for b in (dA, dB, dD):
            b.close()
        with open(args.out, "w") as f:
            json.dump(doc, f, indent=1)
    for kern in kerns.values():
        kern.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
