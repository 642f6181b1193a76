"""Fits the time model's per-instance constants to measured TFLOP/s.

    python fit_time_model.py [tests/golden/select_measured.json] [--sweep fit]

For every instance of ``catalog.CANDIDATES`` the measured launch times of one
sweep (``profiler/select_sweep.py`` output) are split by whether the grid gives
each CU more than one work-group.  On the fuller grids (efficiency, fixed
seconds per tile) minimise the squared log error of
``predicted_launch_seconds`` over a grid of values (0.800-1.000 in steps of
0.005, 0-6 us in steps of 0.25 us); on the one-work-group grids the third
constant, that case's efficiency, does the same with the fixed cost kept.
Prints the ``CANDIDATES`` table.  ``fit()`` is what a test re-runs to show the
committed constants come from the committed measurements.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
from typing import Dict, List, Tuple

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))

from generator import catalog  # noqa: E402

EFFS = [round(0.800 + 0.005 * i, 3) for i in range(41)]
ALONE_EFFS = [round(0.700 + 0.005 * i, 3) for i in range(61)]
FIXED = [0.25e-6 * j for j in range(25)]


def _one_per_cu(name: str, m: int, n: int, k: int, compute_units: int) -> bool:
    cfg, _ = catalog.SOLUTIONS[name]
    t0, t1 = cfg.tile_size
    tiles = -(-m // t0) * -(-n // t1)
    return tiles * catalog.auto_split(name, m, n, k, compute_units) <= compute_units


def fit(shapes: List[dict], compute_units: int = catalog.GFX950_COMPUTE_UNITS) -> Dict[str, Tuple[float, float, float]]:
    """(eff, fixed seconds, eff with one work-group per CU) per candidate."""
    saved = dict(catalog.CANDIDATES)
    out = {}
    try:
        for name in saved:
            pts = [(tuple(s["shape"]), 2.0 * s["shape"][0] * s["shape"][1] * s["shape"][2] / (s["tflops"][name] * 1e12))
                   for s in shapes if name in s["tflops"]]
            full = [p for p in pts if not _one_per_cu(name, *p[0], compute_units)]
            alone = [p for p in pts if _one_per_cu(name, *p[0], compute_units)]

            def loss(points, consts):
                catalog.CANDIDATES[name] = consts
                return sum(math.log(catalog.predicted_launch_seconds(name, *shape, compute_units) / t) ** 2
                           for shape, t in points)

            _, eff, fixed = min((loss(full, (e, f, e)), e, f) for e in EFFS for f in FIXED)
            eff_alone = min((loss(alone, (eff, fixed, a)), a) for a in ALONE_EFFS)[1] if alone else eff
            out[name] = (eff, fixed, eff_alone)
            catalog.CANDIDATES[name] = saved[name]
    finally:
        catalog.CANDIDATES.clear()
        catalog.CANDIDATES.update(saved)
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("data", nargs="?", default=os.path.join(os.path.dirname(os.path.dirname(HERE)), "tests",
                                                            "golden", "select_measured.json"))
    ap.add_argument("--sweep", default="fit", help="the sweep (by name) to fit")
    args = ap.parse_args()
    doc = json.load(open(args.data))
    shapes = next(s["shapes"] for s in doc["sweeps"] if s["name"] == args.sweep)
    for name, (eff, fixed, alone) in fit(shapes).items():
        print(f'    "{name}": ({eff:.3f}, {fixed * 1e6:.2f}e-6, {alone:.3f}),')
    return 0


if __name__ == "__main__":
    sys.exit(main())
