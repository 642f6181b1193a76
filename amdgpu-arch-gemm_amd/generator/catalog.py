"""Named kernel instances shipped with the package, and shape-keyed selection.

Each entry is one (GemmSolutionConfig, GemmOptimizations) pair that
``build_all`` compiles into ``kernels/<name>.co`` + ``kernels/<name>.toml``.
``select(m, n, k)`` returns the name to use for a problem: the instance the
gfx950 tuner chose for a BASELINE shape (``PREFERRED``), else the member of
``CANDIDATES`` with the least ``predicted_seconds`` -- a time model of wave
quantisation over the compute units, per-tile fixed cost, epilogue stores and
split-K partials.  The reference has no catalog: its tuner prints the best
point and keeps nothing (sgemm_tuner.py:116-128).
"""
from __future__ import annotations

import copy
import os
from concurrent.futures import ThreadPoolExecutor
from typing import Dict, List, Optional, Tuple

from .generator import (MAX_LDS_NUM_BYTES, MAX_SPLIT_K, DataType, GemmOptimizations, GemmSolutionConfig,
                        MFMA_16x16x4, MFMA_32x32x2, build_kernel)

PACKAGE_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
KERNEL_DIR = os.path.join(PACKAGE_ROOT, "kernels")

F = DataType.FP32
# compute units of an MI355X (gfx950); the host library reads the real count
GFX950_COMPUTE_UNITS = 256


def _cfg(mfma, wg, wt, dk, stages=1, ta=False, tb=False):
    return GemmSolutionConfig(F, F, F, F, mfma, wg, wt, dk, ta, tb, vmem_stage=stages)


def _opt(wgm=1, plr=1, gw=1, mapk=0, xcd=0, pd=1, occ=0, sk=1, stk=0, stk_rounds=0, ws=0, ws_pd=2, ksplit=0):
    return GemmOptimizations(1, wgm=wgm, plr=plr, gw=gw, map_k_idx=mapk, xcd=xcd, pd=pd, occ=occ, split_k=sk,
                             stream_k=stk, stream_k_rounds=stk_rounds, ws=ws, ws_pd=ws_pd, ksplit=ksplit)


# name -> (config, optimizations)
SOLUTIONS: Dict[str, Tuple[GemmSolutionConfig, GemmOptimizations]] = {
    # tuner winners on gfx950 (interleaved early refill, three LDS buffers);
    # sk=0: the code object also holds the split-K kernel, used when a
    # problem's tiles cannot fill the GPU (not for 256 x 256 tiles, whose
    # 256 accumulators per lane leave no registers for the split epilogue)
    "mt256x256_a32_wg2x2_dk16_s3": (_cfg(MFMA_32x32x2, (2, 2), (4, 4), 16, stages=2), _opt(wgm=4, plr=3, xcd=8)),
    # a 24-deep K tile: three 53 KB LDS buffers (159,744 B of the 160 KiB) and a
    # third fewer barriers per launch than depth 16; 4096 = 170 * 24 + 16, so
    # the first K tile is the partial one (shifted K origin)
    "mt256x256_a32_wg2x2_dk24_s3": (_cfg(MFMA_32x32x2, (2, 2), (4, 4), 24, stages=2), _opt(wgm=4, plr=3, xcd=8)),
    "mt64x64_a16_wg2x2_dk32_s3": (_cfg(MFMA_16x16x4, (2, 2), (2, 2), 32, stages=2), _opt(wgm=4, plr=3, xcd=8, sk=0)),
    "mt128x64_a16_wg2x2_dk16_s3": (_cfg(MFMA_16x16x4, (2, 2), (4, 2), 16, stages=2), _opt(wgm=4, plr=1, xcd=8)),
    "mt128x64_a16_wg2x2_dk32_s3": (_cfg(MFMA_16x16x4, (2, 2), (4, 2), 32, stages=2), _opt(wgm=4, plr=3, xcd=8, sk=0)),
    # winners of the wide sweep (all wave groups, 32..256 tiles)
    "mt256x256_a32_wg4x2_dk16_s3": (_cfg(MFMA_32x32x2, (4, 2), (2, 4), 16, stages=2), _opt(wgm=8, plr=3, xcd=8)),
    # stream-K only up to two rounds of tiles: interleaved runs at 4096 deep
    # gained 4-13% at 1280^2..2304^2 (1.0-1.7 rounds) and lost 3-13% on longer
    # grids (3000^3, 3840^2, 4864^2)
    "mt64x64_a16_wg1x4_dk32_s3": (_cfg(MFMA_16x16x4, (1, 4), (4, 1), 32, stages=2),
                                  _opt(wgm=8, plr=3, xcd=8, sk=0, stk=1, stk_rounds=2)),
    "mt128x64_a16_wg2x2_dk16_s2": (_cfg(MFMA_16x16x4, (2, 2), (4, 2), 16, stages=1), _opt(wgm=1, plr=3, xcd=0, sk=0)),
    # two work-groups per CU (registers capped for 2 waves per SIMD)
    "mt128x64_a16_wg2x2_dk32_s3_occ2": (_cfg(MFMA_16x16x4, (2, 2), (4, 2), 32, stages=2),
                                        _opt(wgm=4, plr=3, xcd=8, occ=2, sk=0, stk=1)),
    "mt256x128_a32_wg2x2_dk16_s3_occ2": (_cfg(MFMA_32x32x2, (2, 2), (4, 2), 16, stages=2),
                                         _opt(wgm=4, plr=3, xcd=8, occ=2)),
    # the same with the refill's memory instructions not interleaved one by one
    # (plr=2): ahead at K = 256 (135.4 / 135.3 TFLOP/s against 132.0 / 132.9 at
    # 8192 x 8192 x 256), behind at K = 512 and at 4096^3
    "mt256x128_a32_wg2x2_dk16_s3_occ2_plr2": (_cfg(MFMA_32x32x2, (2, 2), (4, 2), 16, stages=2),
                                              _opt(wgm=4, plr=2, xcd=8, occ=2)),
    # the same tile with eight waves of 64 x 64 (4 x 2), registers capped for
    # four waves per SIMD: two work-groups, 16 waves per CU
    "mt256x128_a32_wg4x2_dk16_s3_occ4_plr2": (_cfg(MFMA_32x32x2, (4, 2), (2, 2), 16, stages=2),
                                              _opt(wgm=4, plr=2, xcd=8, occ=4)),
    # eight waves (2 x 4 of 64 x 16) and a 64-deep K tile: two waves per SIMD
    # take turns at its MFMAs, one 96 KiB work-group per CU.  At 16384 x 128 x
    # 4096 (one tile per CU) 146.4 / 146.7 TFLOP/s in interleaved runs against
    # 142.5 / 143.4 for the four-wave 128 x 64 instance; with the work-group
    # remap and XCD mapping (wgm=4, xcd=8) it ran 144.2 / 143.8.  Only grids
    # of exactly two rounds with N = 128 favour a remap (wgm=2, xcd=8:
    # 131.8 against 121.0 at 32768 x 128 x 4096, the tiles sharing an A panel
    # then run in one round); stream-K grids favour the plain order (20000 x
    # 128 x 4096: 122.5 against 111.0)
    "mt128x64_a16_wg2x4_dk64": (_cfg(MFMA_16x16x4, (2, 4), (4, 1), 64), _opt(plr=3, sk=0, stk=1)),
    "mt64x128_a32_wg1x4_dk16_s3": (_cfg(MFMA_32x32x2, (1, 4), (2, 1), 16, stages=2), _opt(wgm=4, plr=3, xcd=8)),
    # wave specialisation of the 1024^3 geometry: four computing waves, four
    # loading waves, four LDS buffers ordered by LDS counters (no barrier per
    # K tile).  Measured 2-3% behind the barrier-synchronised instance at
    # 1024^3 and at 1024 x 1024 x 4096, so select() never picks it.
    "mt64x64_a16_wg1x4_dk32_s4_ws": (_cfg(MFMA_16x16x4, (1, 4), (4, 1), 32, stages=3),
                                     _opt(wgm=8, plr=3, xcd=8, ws=1, ws_pd=2)),
    # in-group K split of the 1024^3 geometry: two groups of four waves each
    # multiply half of the tile's K tiles in an LDS ring of their own and add
    # their sums through LDS.  Measured 2.3% behind the one-group instance at
    # 1024^3 (114.8 against 117.5 TFLOP/s) and 1.5% at 1024 x 1024 x 4096, so
    # select() never picks it.
    "mt64x64_a16_wg1x4_dk32_s3_ks": (_cfg(MFMA_16x16x4, (1, 4), (4, 1), 32, stages=2),
                                     _opt(wgm=8, plr=3, xcd=8, ksplit=1)),
    # prefetch depth 2: global loads issued two K tiles ahead of their LDS writes
    "mt128x64_a16_wg2x2_dk32_s3_pd2": (_cfg(MFMA_16x16x4, (2, 2), (4, 2), 32, stages=2),
                                       _opt(wgm=4, plr=3, xcd=8, pd=2)),
    "mt128x64_a16_wg2x2_dk16_s2_pd2": (_cfg(MFMA_16x16x4, (2, 2), (4, 2), 16, stages=1),
                                       _opt(wgm=1, plr=3, xcd=0, pd=2)),
    "mt64x64_a16_wg1x4_dk32_s3_pd2": (_cfg(MFMA_16x16x4, (1, 4), (4, 1), 32, stages=2),
                                      _opt(wgm=8, plr=3, xcd=8, pd=2)),
    "mt256x256_a32_wg2x2_dk16_s3_pd2": (_cfg(MFMA_32x32x2, (2, 2), (4, 4), 16, stages=2),
                                        _opt(wgm=4, plr=3, xcd=8, pd=2)),
    "mt16x16_a16_wg1x1_dk16_s3_pd2": (_cfg(MFMA_16x16x4, (1, 1), (1, 1), 16, stages=2), _opt(plr=3, mapk=4, pd=2)),
    "mt32x32_a32_wg1x1_dk16_s2_pd2": (_cfg(MFMA_32x32x2, (1, 1), (1, 1), 16, stages=1), _opt(plr=2, pd=2)),
    # the first-generation schedule (refill after the last block), kept as a baseline
    "mt256x256_a32_wg2x2_dk16": (_cfg(MFMA_32x32x2, (2, 2), (4, 4), 16), _opt(wgm=4, xcd=8)),
    "mt256x256_a32_wg2x2_dk16_plr2": (_cfg(MFMA_32x32x2, (2, 2), (4, 4), 16), _opt(wgm=4, plr=2, xcd=8)),
    "mt256x128_a32_wg2x2_dk16": (_cfg(MFMA_32x32x2, (2, 2), (4, 2), 16), _opt(wgm=4, xcd=8)),
    "mt128x128_a32_wg2x2_dk16": (_cfg(MFMA_32x32x2, (2, 2), (2, 2), 16), _opt(wgm=4, xcd=8)),
    "mt128x128_a32_wg2x2_dk32": (_cfg(MFMA_32x32x2, (2, 2), (2, 2), 32), _opt(wgm=4, xcd=8)),
    "mt64x64_a32_wg2x2_dk16": (_cfg(MFMA_32x32x2, (2, 2), (1, 1), 16), _opt(wgm=4, xcd=8)),
    # the direct-store epilogue (gw=0): accumulators straight to D, no LDS staging
    "mt64x64_a32_wg2x2_dk16_gw0": (_cfg(MFMA_32x32x2, (2, 2), (1, 1), 16), _opt(wgm=4, xcd=8, gw=0)),
    "mt128x64_a16_wg2x2_dk32_s3_gw0": (_cfg(MFMA_16x16x4, (2, 2), (4, 2), 32, stages=2),
                                       _opt(wgm=4, plr=3, xcd=8, gw=0, sk=0)),
    "mt128x64_a16_wg4x1_dk32": (_cfg(MFMA_16x16x4, (4, 1), (2, 4), 32), _opt(wgm=4, xcd=8)),
    "mt64x128_a32_wg2x2_dk16": (_cfg(MFMA_32x32x2, (2, 2), (1, 2), 16), _opt(xcd=8)),
    # variants that exercise every knob in the parity tests
    "mt128x128_a16_wg2x2_dk16": (_cfg(MFMA_16x16x4, (2, 2), (4, 4), 16), _opt(wgm=2)),
    "mt64x64_a16_wg2x2_dk8": (_cfg(MFMA_16x16x4, (2, 2), (2, 2), 8), _opt(plr=0)),
    "mt128x64_a32_wg4x1_dk8_s3": (_cfg(MFMA_32x32x2, (4, 1), (1, 2), 8, stages=2), _opt(mapk=4, plr=3)),
    "mt64x64_a32_wg1x1_dk16": (_cfg(MFMA_32x32x2, (1, 1), (2, 2), 16), _opt(wgm=8, mapk=8, xcd=8, plr=2)),
    "mt16x16_a16_wg1x1_dk16_s3_plr3": (_cfg(MFMA_16x16x4, (1, 1), (1, 1), 16, stages=2), _opt(plr=3, mapk=4)),
    # stream-K on one-wave tiles (plain and transposed) for the VM and GPU stream-K tests
    "mt32x32_a32_wg1x1_dk16_s3_stk": (_cfg(MFMA_32x32x2, (1, 1), (1, 1), 16, stages=2), _opt(plr=3, stk=1)),
    "mt32x32_a16_wg2x2_dk16_stk_tn": (_cfg(MFMA_16x16x4, (2, 2), (1, 1), 16, ta=True), _opt(stk=1)),
    # split-K (default split count 4) on a one-wave tile, plain and transposed
    "mt32x32_a32_wg1x1_dk16_s3_sk4": (_cfg(MFMA_32x32x2, (1, 1), (1, 1), 16, stages=2), _opt(plr=3, sk=4)),
    "mt32x32_a32_wg1x1_dk16_sk4_tt": (_cfg(MFMA_32x32x2, (1, 1), (1, 1), 16, ta=True, tb=True), _opt(sk=4)),
    # transposed layouts (TN, NT, TT): op(A) = A^T and/or op(B) = B^T
    "mt256x256_a32_wg2x2_dk16_s3_tn": (_cfg(MFMA_32x32x2, (2, 2), (4, 4), 16, stages=2, ta=True),
                                       _opt(wgm=4, plr=3, xcd=8)),
    "mt256x256_a32_wg2x2_dk16_s3_nt": (_cfg(MFMA_32x32x2, (2, 2), (4, 4), 16, stages=2, tb=True),
                                       _opt(wgm=4, plr=3, xcd=8)),
    "mt256x256_a32_wg2x2_dk16_s3_tt": (_cfg(MFMA_32x32x2, (2, 2), (4, 4), 16, stages=2, ta=True, tb=True),
                                       _opt(wgm=4, plr=3, xcd=8)),
    "mt64x64_a16_wg2x2_dk32_s3_tn": (_cfg(MFMA_16x16x4, (2, 2), (2, 2), 32, stages=2, ta=True),
                                     _opt(wgm=4, plr=3, xcd=8)),
    "mt32x32_a32_wg1x1_dk16_tt": (_cfg(MFMA_32x32x2, (1, 1), (1, 1), 16, ta=True, tb=True), _opt()),
    "mt16x16_a16_wg1x1_dk16_nt": (_cfg(MFMA_16x16x4, (1, 1), (1, 1), 16, tb=True), _opt(plr=3)),
    # edge-strip kernels (sgemm_set_edge_kernels): 16 rows or 16 columns wide,
    # split-K over the strip's few tiles.  A strip one element wide is a
    # memory-bound pass over B (bottom) or A (right): at 4097^3, 67 MB each,
    # 16.0 and 15.3 us with these (4.2 / 4.4 TB/s); 16 x 128 and 128 x 16 at
    # depth 32 took 16.5 and 17.0, 16 x 256 and 256 x 16 21.3 and 20.5
    "mt16x128_a16_wg1x4_dk64_s2": (_cfg(MFMA_16x16x4, (1, 4), (1, 2), 64, stages=1), _opt(plr=3, xcd=8, sk=0)),
    "mt64x16_a16_wg4x1_dk64_s3": (_cfg(MFMA_16x16x4, (4, 1), (1, 1), 64, stages=2), _opt(plr=3, xcd=8, sk=0)),
    # the reference's one-wave VM configurations (test_vm.py:447-627)
    "mt32x32_a32_wg1x1_dk16": (_cfg(MFMA_32x32x2, (1, 1), (1, 1), 16), _opt()),
    "mt16x16_a16_wg1x1_dk16": (_cfg(MFMA_16x16x4, (1, 1), (1, 1), 16), _opt()),
    "mt16x16_a16_wg1x1_dk16_wgm4": (_cfg(MFMA_16x16x4, (1, 1), (1, 1), 16), _opt(wgm=4)),
    "mt16x16_a16_wg1x1_dk16_mapk4": (_cfg(MFMA_16x16x4, (1, 1), (1, 1), 16), _opt(mapk=4)),
    "mt16x16_a16_wg1x1_dk16_s3": (_cfg(MFMA_16x16x4, (1, 1), (1, 1), 16, stages=2), _opt()),
}

# shape class -> preferred instance (filled from tuner results; see select())
PREFERRED: List[Tuple[Tuple[int, int, int], str]] = [
    # one 256 x 256 work-group of eight waves per CU (two per SIMD hide each
    # other's waits): as fast as two four-wave 256 x 128 work-groups per CU
    # (151.47 against 151.55 TFLOP/s over 30 rounds in alternating order;
    # 139.7 against 138.7 as three fresh processes each under bench.py's
    # 5-launch warm-up) with 22% less HBM traffic: each A and B panel is read
    # by half as many tiles (470 MB per launch, 2.33x the algorithmic bytes,
    # against 605 MB)
    ((4096, 4096, 4096), "mt256x256_a32_wg4x2_dk16_s3"),
    ((1024, 1024, 1024), "mt64x64_a16_wg1x4_dk32_s3"),
    # eight 64 x 64 waves, two work-groups per CU: 135.9 / 136.0 TFLOP/s in
    # bench.py against 134.3 / 134.4 for the four-wave 256 x 128 plr=2 instance
    ((8192, 8192, 256), "mt256x128_a32_wg4x2_dk16_s3_occ4_plr2"),
    # 144.2 / 144.2 TFLOP/s in bench.py against 141.2 / 141.2 for the
    # four-wave 128 x 64 occ=2 instance
    ((16384, 128, 4096), "mt128x64_a16_wg2x4_dk64"),
    # few output tiles and a deep K (bench.py --workload deepk): the split-K kernel
    ((512, 512, 16384), "mt64x64_a16_wg1x4_dk32_s3"),
]
# Instances select() chooses among for other shapes: (fraction of the FP32
# MFMA peak the K loop reaches when the grid gives a CU more than one
# work-group, fixed seconds per tile, the fraction when each CU holds one
# work-group), fitted per instance by least squares on log time to 41 shapes
# from 1024^3 to 16384^2 x 256 timed interleaved on MI355X (rms error 1-7%
# per instance).  One work-group per CU is the four-wave instances' weak spot
# (0.77-0.83 for 128 x 64 and 64 x 64 against 0.93-0.95 on fuller grids), not
# the eight-wave ones', whose two waves per SIMD hide each other's waits: at
# 8192 x 256 x 4096 the eight-wave 128 x 64 runs 145 TFLOP/s against 132 for
# the four-wave occ=2 one.  The plr=2 twin of the 256 x 128 instance pays a
# smaller fixed cost for a slower loop: it wins at short K.  The 64 x 64 one
# also carries the split-K kernel: against mt128x64_a16_wg2x2_dk16_s2 it
# measured 125.6 / 127.5 / 114.8 TFLOP/s at 512^2 x 16384, 1024 x 512 x 8192
# and 256^2 x 65536 (host-chosen split counts), against 109.0 / 110.5 / 59.0.
CANDIDATES: Dict[str, Tuple[float, float, float]] = {
    "mt256x256_a32_wg2x2_dk24_s3": (0.980, 5.00e-6, 0.985),
    "mt256x128_a32_wg2x2_dk16_s3_occ2": (0.990, 2.50e-6, 0.980),
    "mt256x128_a32_wg2x2_dk16_s3_occ2_plr2": (0.945, 0.25e-6, 0.880),
    "mt256x128_a32_wg4x2_dk16_s3_occ4_plr2": (0.965, 0.50e-6, 0.930),
    "mt128x64_a16_wg2x2_dk32_s3": (0.945, 0.25e-6, 0.805),
    "mt128x64_a16_wg2x2_dk32_s3_occ2": (0.950, 0.75e-6, 0.830),
    "mt128x64_a16_wg2x4_dk64": (0.935, 1.00e-6, 0.910),
    "mt64x64_a16_wg1x4_dk32_s3": (0.925, 0.00e-6, 0.770),
}
# instances attached (sgemm_set_edge_kernels) to the large-tile ones for thin
# edge strips: (rows, cols) = a 16-row tile for the strip of rows past the last
# tile row and a 16-column tile for the strip of columns past the last tile
# column, both with split-K for the strips' few tiles
EDGE_PAIR = ("mt16x128_a16_wg1x4_dk64_s2", "mt64x16_a16_wg4x1_dk64_s3")
EDGE_KERNEL: Dict[str, Tuple[str, str]] = {
    "mt256x128_a32_wg2x2_dk16_s3_occ2": EDGE_PAIR,
    "mt256x128_a32_wg2x2_dk16_s3_occ2_plr2": EDGE_PAIR,
    "mt256x256_a32_wg2x2_dk24_s3": EDGE_PAIR,
    "mt128x64_a16_wg2x2_dk32_s3_occ2": EDGE_PAIR,
    "mt128x64_a16_wg2x4_dk64": EDGE_PAIR,
    "mt256x128_a32_wg4x2_dk16_s3_occ4_plr2": EDGE_PAIR,
}


# work-groups of generated_gemm resident per CU for the instances with edge
# kernels and the time model's candidates (the compiler's occupancy; the host
# library queries it): an occ=N instance holds N four-wave work-groups or
# N / 2 eight-wave ones
RESIDENT_PER_CU: Dict[str, int] = {
    "mt256x128_a32_wg2x2_dk16_s3_occ2": 2,
    "mt256x128_a32_wg2x2_dk16_s3_occ2_plr2": 2,
    "mt256x256_a32_wg2x2_dk24_s3": 1,
    "mt128x64_a16_wg2x2_dk32_s3_occ2": 2,
    "mt128x64_a16_wg2x4_dk64": 1,
    "mt256x128_a32_wg4x2_dk16_s3_occ4_plr2": 2,
}


def edge_interior(name: str, m: int, n: int, k: int,
                  compute_units: int = GFX950_COMPUTE_UNITS) -> Tuple[int, int]:
    """(m, n) of the interior the host library gives the instance itself when
    its EDGE_KERNEL pair is attached (the rule of sgemm_set_edge_kernels): a
    strip of at most a quarter of a tile next to a non-empty interior goes to
    an edge kernel when that takes a round of work-groups off the instance's
    grid, and only the strips needed for that.  At 2500^3 in 128 x 64 tiles
    the 4-column strip would not (800 and 780 tiles are both two rounds of
    512): attached, it measured 253.0 us against 246.6 us without."""
    if name not in EDGE_KERNEL or k == 0:
        return m, n
    cfg, _ = SOLUTIONS[name]
    t0, t1 = cfg.tile_size
    me, ne = m % t0, n % t1
    if not (me and me * 4 <= t0 and m > me):
        me = 0
    if not (ne and ne * 4 <= t1 and n > ne):
        ne = 0
    if not me and not ne:
        return m, n
    res = RESIDENT_PER_CU[name] * compute_units

    def rounds(rm, rn):
        return -(-(-(-rm // t0) * -(-rn // t1)) // res)

    both = rounds(m - me, n - ne)
    if rounds(m, n) <= both:
        return m, n
    if me and ne:
        if rounds(m - me, n) <= both:
            ne = 0
        elif rounds(m, n - ne) <= both:
            me = 0
    return m - me, n - ne


# resident stream-K work-groups per CU of the stream-K instances (the
# compiler's occupancy of generated_gemm_streamk; the host library queries it)
STREAM_K_GROUPS_PER_CU: Dict[str, int] = {
    "mt64x64_a16_wg1x4_dk32_s3": 3,
    "mt128x64_a16_wg2x2_dk32_s3_occ2": 2,
    "mt128x64_a16_wg2x4_dk64": 1,
}

# Transposed twins of the time model's candidates and of the BASELINE
# shapes' preferred instances: the same geometry and
# knobs with trans_a / trans_b, named <candidate>_tn / _nt / _tt, for
# select(..., trans_a, trans_b).  The transposed tiles keep each operand's
# contiguous dimension and run at the NN speed (4096^3 on 256 x 256: NN, TN,
# NT, TT 151.3 / 151.3 / 151.2 / 151.1 TFLOP/s), so a twin is ranked with its
# candidate's constants -- where its LDS tile keeps as many work-groups per CU
# as the candidate holds (the generator swizzles A^T's rows in place of a pad
# to keep them); twins that would lose one are not built.  The edge pair has
# twins of every layout too (<edge>_tn / _nt / _tt), and a twin carries the
# pair of its own layout wherever its candidate carries EDGE_PAIR (attached
# edge kernels must share the main kernel's layout).
LAYOUT_SUFFIX: Dict[Tuple[bool, bool], str] = {(True, False): "_tn", (False, True): "_nt", (True, True): "_tt"}
TWINS: Dict[Tuple[str, bool, bool], str] = {}
# twins that are not built: the eight-wave 256 x 128 instance has 128 VGPRs
# per lane (four waves per SIMD), and its A^T tile's row swizzle (one address
# per atom row) spills two of them
NO_TWIN = {("mt256x128_a32_wg4x2_dk16_s3_occ4_plr2", True, False)}


def _add_twins() -> None:
    for name in EDGE_PAIR:
        cfg, opt = SOLUTIONS[name]
        for (ta, tb), suffix in LAYOUT_SUFFIX.items():
            SOLUTIONS[name + suffix] = (_cfg(cfg.mfma, cfg.wave_group, cfg.wave_tiling, cfg.depth_k,
                                             stages=cfg.vmem_stage, ta=ta, tb=tb), copy.copy(opt))
    for name in list(CANDIDATES) + [nm for _, nm in PREFERRED if nm not in CANDIDATES]:
        cfg, opt = SOLUTIONS[name]
        resident = min(MAX_LDS_NUM_BYTES // cfg.lds_usage_bytes, RESIDENT_PER_CU.get(name, MAX_LDS_NUM_BYTES))
        for (ta, tb), suffix in LAYOUT_SUFFIX.items():
            if (name, ta, tb) in NO_TWIN:
                continue
            try:
                twin_cfg = _cfg(cfg.mfma, cfg.wave_group, cfg.wave_tiling, cfg.depth_k, stages=cfg.vmem_stage,
                                ta=ta, tb=tb)
            except RuntimeError:
                continue
            if MAX_LDS_NUM_BYTES // twin_cfg.lds_usage_bytes < resident:
                continue
            twin = name + suffix
            SOLUTIONS[twin] = (twin_cfg, copy.copy(opt))
            TWINS[(name, ta, tb)] = twin
            if name in RESIDENT_PER_CU:
                RESIDENT_PER_CU[twin] = RESIDENT_PER_CU[name]
            if name in STREAM_K_GROUPS_PER_CU:
                STREAM_K_GROUPS_PER_CU[twin] = STREAM_K_GROUPS_PER_CU[name]
            if EDGE_KERNEL.get(name) == EDGE_PAIR:
                EDGE_KERNEL[twin] = tuple(e + suffix for e in EDGE_PAIR)


_add_twins()
# rate of the streamed tiles relative to whole tiles: interleaved runs at
# 1792^2..4864^2 x 4096 and 3000^3 measured 0.89-0.92 of the model's whole-tile
# rate when every tile is streamed, approaching 1 as the streamed share falls
_STREAM_K_RATE = 0.91
# the gap between two dependent launches on one stream
_LAUNCH_SECONDS = 4e-6
# peak FP32 MFMA rate of one CU (157.3 TFLOP/s / 256) and the share of HBM
# write bandwidth one CU's epilogue gets when all store at once (fitted)
_CU_FLOPS = 157.3e12 / GFX950_COMPUTE_UNITS
_CU_WRITE_BYTES_PER_S = 24.8e9


def paths(name: str, kernel_dir: str = KERNEL_DIR) -> Tuple[str, str]:
    return os.path.join(kernel_dir, f"{name}.co"), os.path.join(kernel_dir, f"{name}.toml")


def build_one(name: str, kernel_dir: str = KERNEL_DIR) -> Tuple[str, str]:
    cfg, opt = SOLUTIONS[name]
    cfg.name = name
    return build_kernel(kernel_dir, cfg, opt, kern_name=name)


def build_all(kernel_dir: str = KERNEL_DIR, names: Optional[List[str]] = None, jobs: int = 8) -> List[str]:
    names = list(SOLUTIONS) if names is None else names
    os.makedirs(kernel_dir, exist_ok=True)
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        list(ex.map(lambda n: build_one(n, kernel_dir), names))
    return names


def vector_k(name: str, k: int) -> bool:
    """True when every K tile of a k-deep problem takes the vector path: whole
    K tiles, or a remainder with at least two K tiles on an instance without a
    K rotation (the kernel then shifts the K origin so the first tile is the
    partial one)."""
    cfg, opt = SOLUTIONS[name]
    dk = cfg.depth_k
    return k % dk == 0 or (k > dk and opt.map_k_idx <= 1)


def divides(name: str, m: int, n: int, k: int) -> bool:
    """Whole tiles in M and N and a K the vector path covers."""
    cfg, _ = SOLUTIONS[name]
    t0, t1 = cfg.tile_size
    return m % t0 == 0 and n % t1 == 0 and vector_k(name, k)


SPLIT_RANGE_OVERHEAD = 4  # K tiles


def auto_split(name: str, m: int, n: int, k: int, compute_units: int = GFX950_COMPUTE_UNITS) -> int:
    """K ranges the host library uses for an instance built with split_k = 0
    (the rule of sgemm_set_split_k): none when the tiles fill the compute
    units, else the s <= min(MAX_SPLIT_K, K tiles / 4) with the least
    ceil(tiles * s / CUs) * (ceil(K tiles / s) + SPLIT_RANGE_OVERHEAD): rounds
    of work-groups times a range's K tiles plus its fixed cost (smallest s
    among ties); an instance built with a fixed split count uses that count.
    Either way at most one range per K tile.  The fixed cost, 4 K tiles, is
    the pipeline fill, partial store and fix-up of a range: it makes a thin
    strip of 33 tiles (1 x 4097 x 4097 in 16 x 128 tiles) take 7 ranges,
    17.7 us, where the rounds alone give 15 ranges, 19.2 us."""
    cfg, opt = SOLUTIONS[name]
    t0, t1 = cfg.tile_size
    tiles = -(-m // t0) * -(-n // t1)
    ktiles = -(-k // cfg.depth_k)
    if opt.split_k == 1:
        return 1
    if opt.split_k > 1:
        s = opt.split_k
    elif tiles >= compute_units or tiles == 0:
        s = 1
    else:
        s, best = 1, ktiles + SPLIT_RANGE_OVERHEAD
        for c in range(2, min(MAX_SPLIT_K, ktiles // 4) + 1):
            cost = -(-tiles * c // compute_units) * (-(-ktiles // c) + SPLIT_RANGE_OVERHEAD)
            if cost < best:
                s, best = c, cost
    return max(1, min(s, ktiles))


def stream_k_tiles(tiles: int, groups: int, k: int, mode: int = 1, depth_k: int = 1, max_rounds: int = 0) -> int:
    """Tiles of the stream-K phase the host library gives an unsplit launch of
    ``tiles`` tiles over ``groups`` resident stream-K work-groups (the rule of
    sgemm_set_stream_k; 0 = no stream-K): with T > G, the last partial round
    plus one whole round, T % G + G tiles, when ceil(T / G) rounds cost at
    least 3% over T / G and take at most ``max_rounds`` (0: any; mode 1) or
    always (mode 2, G tiles when T % G == 0), as long as those tiles' K tiles
    (``depth_k`` deep) times G stay below 2^32."""
    if mode == 0 or groups <= 0 or k == 0 or tiles <= groups:
        return 0
    rem = tiles % groups
    if mode == 1:
        rounds = -(-tiles // groups)
        if rem == 0 or rounds * groups * 100 < tiles * 103 or (max_rounds and rounds > max_rounds):
            return 0
    sk = rem + groups if rem else groups
    # the kernel's iteration arithmetic is 32-bit
    if sk * -(-k // depth_k) * groups >= 1 << 32:
        return 0
    return sk


def predicted_seconds(name: str, m: int, n: int, k: int, compute_units: int = GFX950_COMPUTE_UNITS) -> float:
    """predicted_launch_seconds of the parts a launch of ``name`` runs: with
    its EDGE_KERNEL attached, the interior plus the thin edge strips the edge
    kernel takes, one after another."""
    mi, ni = edge_interior(name, m, n, k)
    if (mi, ni) == (m, n):
        return predicted_launch_seconds(name, m, n, k, compute_units)
    rows, cols = EDGE_KERNEL[name]
    t = predicted_launch_seconds(name, mi, ni, k, compute_units)
    if mi < m:
        t += predicted_launch_seconds(rows, m - mi, n, k, compute_units) + _LAUNCH_SECONDS
    if ni < n:
        t += predicted_launch_seconds(cols, mi, n - ni, k, compute_units) + _LAUNCH_SECONDS
    return t


def _loop_efficiency(name: str, work_groups: int, compute_units: int) -> float:
    """The K loop's fraction of the MFMA peak: the full rate once the grid
    gives each CU more than one work-group, the lower one-work-group rate
    otherwise (nothing beside it hides its waits)."""
    eff, _, eff_alone = CANDIDATES.get(name, (0.9, 0.0, 0.9))
    return eff_alone if work_groups <= compute_units else eff


def predicted_launch_seconds(name: str, m: int, n: int, k: int, compute_units: int = GFX950_COMPUTE_UNITS) -> float:
    """Time model behind select(): the CU with the most work-groups sets the
    time (rounds of tiles x K splits over the CUs, each work-group a K loop at
    the instance's MFMA efficiency (_loop_efficiency) plus its fixed cost and
    its epilogue's stores), and a split
    launch adds its partials' writes and the last work-group's reads.  Two
    work-groups per CU (RESIDENT_PER_CU) hide half of each epilogue behind the other's
    K loop.  Wave quantisation is the point: 3000^3 in 256 x 128 tiles is 288
    work-groups, two rounds on 32 CUs, at half the speed of 64 x 64 tiles.  An
    instance with a stream-K kernel that the host would use on this grid
    (stream_k_tiles) has no partial round: its tiles are spread evenly over the
    CUs, the streamed ones at _STREAM_K_RATE."""
    cfg, opt = SOLUTIONS[name]
    t0, t1 = cfg.tile_size
    dk = cfg.depth_k
    tiles = -(-m // t0) * -(-n // t1)
    splits = auto_split(name, m, n, k, compute_units)
    ktiles = -(-max(k, 1) // dk)
    k_range = -(-ktiles // splits) * dk
    rounds = -(-(tiles * splits) // compute_units)
    occ = RESIDENT_PER_CU.get(name, max(opt.occ, 1))  # work-groups per CU
    tile_bytes = t0 * t1 * 4
    eff = _loop_efficiency(name, tiles * splits, compute_units)
    fixed = CANDIDATES.get(name, (0.9, 0.0, 0.9))[1]
    loop = 2.0 * t0 * t1 * k_range / (_CU_FLOPS * eff) + fixed
    epilogue = tile_bytes / _CU_WRITE_BYTES_PER_S
    reduce = 2.0 * splits * tile_bytes / _CU_WRITE_BYTES_PER_S if splits > 1 else 0.0
    sk = 0
    if splits == 1 and opt.stream_k:
        groups = compute_units * STREAM_K_GROUPS_PER_CU.get(name, occ)
        sk = stream_k_tiles(tiles, groups, k, 1, dk, opt.stream_k_rounds)
    if sk:
        # stream-K: no partial last round; the streamed tiles run at a lower
        # rate (their cuts, partials and the fix-up)
        per_cu = ((tiles - sk) * (loop + epilogue / occ) + sk * (loop / _STREAM_K_RATE + epilogue / occ))
        return per_cu / compute_units + epilogue * (1.0 - 1.0 / occ)
    return rounds * (loop + epilogue / occ) + epilogue * (1.0 - 1.0 / occ) + reduce


def select(m: int, n: int, k: int, trans_a: bool = False, trans_b: bool = False) -> str:
    """Instance for an (m, n, k) problem: the tuner's choice for a BASELINE
    shape, else the candidate with the least predicted time
    (predicted_seconds; the larger tile among near ties).  With trans_a /
    trans_b (op(A) = A^T, op(B) = B^T) the same choice among the candidates
    that have a twin of that layout (TWINS) returns the twin."""
    if m <= 0 or n <= 0:
        raise RuntimeError(f"empty problem {m}x{n}x{k}")
    trans = trans_a or trans_b
    pick = next((nm for shape, nm in PREFERRED if shape == (m, n, k)), None)
    if pick is None or (trans and (pick, trans_a, trans_b) not in TWINS):
        names = [nm for nm in CANDIDATES if not trans or (nm, trans_a, trans_b) in TWINS]
        pick = min(names, key=lambda nm: (predicted_seconds(nm, m, n, k),
                                          -SOLUTIONS[nm][0].tile_size[0] * SOLUTIONS[nm][0].tile_size[1]))
    return TWINS[(pick, trans_a, trans_b)] if trans else pick
