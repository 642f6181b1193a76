"""Grid-search tuner for the gfx950 SGEMM kernel family.

Same command line as the reference tuner (tuner/sgemm_tuner.py:25-36):

    python tuner/sgemm_tuner.py --m M --n N --k K --bench ./runner/GeneratorRunner --output-folder ./out

and the same loop (sgemm_tuner.py:41-128): enumerate knob combinations, skip
the ones the generator rejects (RuntimeError) or whose tile does not divide the
problem, compile each survivor, benchmark it with the runner
(``<bench> <co> <toml> M N K 5 50 0``, Gflops parsed from the third-to-last
stdout line) and print the best.  Additions:

* ``--space gfx950`` (default): macro-tile {64,128,256}^2 x wave-group
  {2x2, 4x1} x MFMA atom {32x32x2, 16x16x4} (stage 1), then the code-shape
  knobs depth_k {16,24,32} x vmem_stage {1,2} x wgm {1,4,8} x xcd {0,8} x plr {1,2,3}
  x prefetch depth {1,2}
  on the best ``--refine`` geometries (stage 2), optionally crossed with
  ``--split-k`` (split-K kernel; 0 = split count chosen per problem);
  ``--occ`` (waves per SIMD the registers are capped for, default 0 and 2)
  applies to both stages, and stage 1 tries depth_k 16 and 32.  ``--space
  reference`` is the reference's own 9-knob product.
* every result is appended to ``<out>/results.jsonl`` and a rerun skips
  points already there (resume);
* each point runs in isolation: compile failures, runner failures and
  ``--timeout`` expiries are recorded and the sweep continues (the reference
  aborts on the first failing point, sgemm_tuner.py:121-123);
* the winner is re-emitted as ``<out>/generated_gemm.co`` + ``.toml`` (the
  reference overwrites one artifact per point and keeps none, :67, :107);
* ``--compile-only`` builds every candidate without a GPU; ``--no-compile``
  benchmarks candidates built earlier; ``--in-process`` times them through the
  ctypes shim instead of one runner process per point.
"""
from __future__ import annotations

import argparse
import hashlib
import json
import os
import shutil
import subprocess
import sys
import time
from concurrent.futures import ThreadPoolExecutor, as_completed
from itertools import product
from typing import Dict, Iterable, List, Optional, Sequence, Tuple

_PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if _PKG not in sys.path:
    sys.path.insert(0, _PKG)

from generator.generator import (  # noqa: E402
    DataType,
    FunctionArgument,
    GemmOptimizations,
    GemmSolutionConfig,
    compile,
    default_arguments,
    gemm,
    read_toml,
)

# reference knob lists (sgemm_tuner.py:13-21)
SUPPORTED_WAVE_GROUPS = [(1, 1), (1, 2), (2, 1), (2, 2), (4, 2), (2, 4)]
SUPPORTED_WAVE_TILINGS = [(i, j) for i in range(1, 9) for j in range(1, 9)]
SUPPORTED_MFMAS = [(16, 16, 1, 4), (32, 32, 1, 2)]
SUPPORTED_DEPTH_K = [8, 16, 32, 64]
SUPPORTED_WGM = [1, 2, 4, 8]
SUPPORTED_PLR = [0, 1, 2]
SUPPORTED_GW = [0, 1]
SUPPORTED_MAP_K_IDX = [0, 4, 8]
SUPPORTED_VMEM_STAGES = [1, 2]

# gfx950 space
GFX950_MACRO_TILES = [(a, b) for a in (64, 128, 256) for b in (64, 128, 256)]
GFX950_WAVE_GROUPS = [(2, 2), (4, 1)]
# --space gfx950-wide: also 32-wide tiles and every wave group of the reference
GFX950_WIDE_MACRO_TILES = [(a, b) for a in (32, 64, 128, 256) for b in (32, 64, 128, 256)]
GFX950_WIDE_WAVE_GROUPS = SUPPORTED_WAVE_GROUPS + [(4, 1), (1, 4)]
GFX950_DEPTH_K = [16, 24, 32]
GFX950_VMEM_STAGES = [1, 2]
GFX950_WGM = [1, 4, 8]
GFX950_XCD = [0, 8]
GFX950_PLR = [1, 2, 3]
GFX950_PD = [1, 2]
DEFAULT_KNOBS = dict(depth_k=16, vmem_stage=2, wgm=4, xcd=8, plr=3, gw=0, map_k_idx=0)
# K depths every geometry is tried at in stage 1
STAGE1_DEPTHS = (16, 32)
ARCH = "gfx950"
VERBOSE = False

F = DataType.FP32
Point = Tuple[GemmSolutionConfig, GemmOptimizations]


def point_key(cfg: GemmSolutionConfig, opt: GemmOptimizations) -> str:
    return (f"a{cfg.mfma[0]}_wg{cfg.wave_group[0]}x{cfg.wave_group[1]}_wt{cfg.wave_tiling[0]}x{cfg.wave_tiling[1]}"
            f"_dk{cfg.depth_k}_s{cfg.vmem_stage}_wgm{opt.wgm}_plr{opt.plr}_gw{opt.gw}_mk{opt.map_k_idx}_x{opt.xcd}"
            + (f"_pd{opt.pd}" if opt.pd != 1 else "") + (f"_occ{opt.occ}" if opt.occ else "")
            + (f"_sk{opt.split_k}" if opt.split_k != 1 else ""))


def make_point(mfma, wg, wt, depth_k, vmem_stage, wgm, plr, gw, map_k_idx, xcd, pd=1, occ=0,
               split_k=1) -> Optional[Point]:
    try:
        cfg = GemmSolutionConfig(F, F, F, F, mfma, wg, wt, depth_k, False, False, vmem_stage=vmem_stage)
        opt = GemmOptimizations(1, wgm=wgm, plr=plr, gw=gw, map_k_idx=map_k_idx, xcd=xcd, pd=pd, occ=occ,
                                split_k=split_k)
    except RuntimeError as e:
        if VERBOSE:
            print(e)
        return None
    return cfg, opt


def fits(cfg: GemmSolutionConfig, m: int, n: int, k: int) -> bool:
    """The reference skips tiles that do not divide the problem (sgemm_tuner.py:97-100)
    because its kernel cannot mask edges; this kernel can, so only tiles larger
    than the problem are skipped, plus the reference's vector-load filter
    (:102-105): every work-item moves at least one 16-byte chunk of A and of B."""
    t0, t1 = cfg.tile_size
    if t0 > max(m, 1) or t1 > max(n, 1):
        return False
    return cfg.num_bytes_per_buffer_load == (16, 16)


def geometry_points(knobs: Dict, wide: bool = False, occs: Sequence[int] = (0,),
                    depths: Sequence[int] = (16,)) -> Iterable[Point]:
    """Stage-1 candidates: every macro-tile x wave-group x atom geometry at the
    default code-shape knobs, once per occupancy target in ``occs`` and K
    depth in ``depths``: a geometry that only pays with two work-groups per
    CU (the 4096^3 winner, 256 x 128) or with a deeper K tile (16x16x4 atoms:
    128 x 64 runs 30% faster at depth 32 than at 16) must reach stage 2 at
    that setting."""
    tiles = GFX950_WIDE_MACRO_TILES if wide else GFX950_MACRO_TILES
    groups = GFX950_WIDE_WAVE_GROUPS if wide else GFX950_WAVE_GROUPS
    for (mt0, mt1), wg, mfma, occ, dk in product(tiles, groups, SUPPORTED_MFMAS, occs, depths):
        if mt0 % (mfma[0] * wg[0]) or mt1 % (mfma[1] * wg[1]):
            continue
        wt = (mt0 // (mfma[0] * wg[0]), mt1 // (mfma[1] * wg[1]))
        p = make_point(mfma, wg, wt, dk, knobs["vmem_stage"], knobs["wgm"], knobs["plr"], knobs["gw"],
                       knobs["map_k_idx"], knobs["xcd"], occ=occ)
        if p:
            yield p


def knob_points(cfg: GemmSolutionConfig, split_ks: Sequence[int] = (1,), occs: Sequence[int] = (0,)) -> Iterable[Point]:
    """Stage-2 candidates of one geometry; ``split_ks`` and ``occs`` add the
    gfx950-only split-K (0 = chosen per problem) and occupancy knobs."""
    for dk, st, wgm, xcd, plr, pd, sk, occ in product(GFX950_DEPTH_K, GFX950_VMEM_STAGES, GFX950_WGM, GFX950_XCD,
                                                      GFX950_PLR, GFX950_PD, split_ks, occs):
        if pd == 2 and plr < 2:
            continue
        p = make_point(cfg.mfma, cfg.wave_group, cfg.wave_tiling, dk, st, wgm, plr, 0, 0, xcd, pd, occ, sk)
        if p:
            yield p


def reference_points() -> Iterable[Point]:
    for wg, wt, mfma, dk, wgm, plr, gw, mk, st in product(
            SUPPORTED_WAVE_GROUPS, SUPPORTED_WAVE_TILINGS, SUPPORTED_MFMAS, SUPPORTED_DEPTH_K, SUPPORTED_WGM,
            SUPPORTED_PLR, SUPPORTED_GW, SUPPORTED_MAP_K_IDX, SUPPORTED_VMEM_STAGES):
        p = make_point(mfma, wg, wt, dk, st, wgm, plr, gw, mk, 0)
        if p:
            yield p


# --------------------------------------------------------------- building
POINTS_DIR: Optional[str] = None


def point_dir(out: str) -> str:
    return POINTS_DIR or os.path.join(out, "points")


def build_point(out: str, p: Point) -> Tuple[str, int]:
    cfg, opt = p
    key = point_key(cfg, opt)
    d = point_dir(out)
    co = os.path.join(d, f"{key}.co")
    if os.path.exists(co) and os.path.exists(os.path.join(d, f"{key}.toml")):
        return key, 0
    cfg.name = key
    src = gemm(None, "generated_gemm", ARCH, cfg, opt, default_arguments())
    rc = compile(key, src, ARCH, d, cfg, opt)
    hip = os.path.join(d, f"{key}.hip")
    if os.path.exists(hip):
        os.remove(hip)
    return key, rc


def build_points(out: str, points: List[Point], jobs: int) -> Dict[str, int]:
    """Compiles the candidates in parallel; prints a progress line every 16."""
    os.makedirs(point_dir(out), exist_ok=True)
    res: Dict[str, int] = {}
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        futures = [ex.submit(build_point, out, p) for p in points]
        for i, f in enumerate(as_completed(futures), 1):
            key, rc = f.result()
            res[key] = rc
            if i % 16 == 0 or i == len(futures):
                print(f"compiled {i}/{len(futures)} candidates", flush=True)
    return res


def spills(out: str, key: str) -> bool:
    t = read_toml(os.path.join(point_dir(out), f"{key}.toml"))
    return int(t.get("scratch_bytes_per_lane", 0)) > 0


# ----------------------------------------------------------- benchmarking
class InProcessBench:
    """Times candidates through the ctypes shim with inputs uploaded once."""

    def __init__(self, m, n, k, warmup, runs):
        from shim import sgemm_shim as S
        self.S = S
        self.m, self.n, self.k, self.warmup, self.runs = m, n, k, warmup, runs
        A = S.fill_matrix(m, k, 1, 0)
        B = S.fill_matrix(k, n, 1, 1)
        self.dA, self.dB = S.DeviceBuffer.from_array(A), S.DeviceBuffer.from_array(B)
        self.dD = S.DeviceBuffer(m * n * 4)

    def __call__(self, co, toml, timeout) -> Tuple[int, float]:
        with self.S.Kernel(co, toml) as kern:
            ms = kern.time(self.dA, self.dB, None, self.dD, self.m, self.n, self.k, 1.0, 0.0,
                           warmup=self.warmup, runs=self.runs) / self.runs
        return 0, 2.0 * self.m * self.n * self.k / ms * 1e-6


class RunnerBench:
    """The reference's way: one runner process per point, Gflops from stdout[-3]."""

    def __init__(self, bench, m, n, k, warmup, runs):
        self.bench, self.m, self.n, self.k, self.warmup, self.runs = bench, m, n, k, warmup, runs

    def __call__(self, co, toml, timeout) -> Tuple[int, float]:
        ret = subprocess.run([self.bench, co, toml, str(self.m), str(self.n), str(self.k), str(self.warmup),
                              str(self.runs), "0"], stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                             timeout=timeout)
        if ret.returncode:
            return ret.returncode, 0.0
        out = ret.stdout.decode()
        return 0, float(out.split("\n")[-3].split(":")[-1])


def load_results(path: str) -> Dict[str, Dict]:
    done = {}
    if os.path.exists(path):
        with open(path) as f:
            for line in f:
                line = line.strip()
                if line:
                    r = json.loads(line)
                    done[r["key"]] = r
    return done


def record(path: str, rec: Dict):
    with open(path, "a") as f:
        f.write(json.dumps(rec) + "\n")


def sweep(points: List[Point], out: str, m: int, n: int, k: int, bench, timeout: float, results_path: str,
          compiled: Dict[str, int]) -> List[Dict]:
    done = load_results(results_path)
    shape = f"{m}x{n}x{k}"
    recs = []
    for cfg, opt in points:
        key = point_key(cfg, opt)
        rkey = f"{shape}:{key}"
        if rkey in done:
            recs.append(done[rkey])
            continue
        rec = {"key": rkey, "point": key, "shape": [m, n, k], "tile": list(cfg.tile_size), "mfma": list(cfg.mfma),
               "wave_group": list(cfg.wave_group), "wave_tiling": list(cfg.wave_tiling), "depth_k": cfg.depth_k,
               "vmem_stage": cfg.vmem_stage, **opt.to_dict(), "gflops": 0.0, "status": "ok"}
        co = os.path.join(point_dir(out), f"{key}.co")
        toml = os.path.join(point_dir(out), f"{key}.toml")
        if compiled.get(key, 0) != 0 or not os.path.exists(co):
            rec["status"] = "compile_error"
        elif spills(out, key):
            rec["status"] = "spills"
        else:
            try:
                rc, gflops = bench(co, toml, timeout)
                rec["gflops"] = gflops
                if rc:
                    rec["status"] = f"runner_rc_{rc}"
            except subprocess.TimeoutExpired:
                rec["status"] = "timeout"
            except Exception as e:  # isolate the point, keep sweeping
                rec["status"] = f"error: {e}"
        record(results_path, rec)
        recs.append(rec)
        print(f"Gflops: {rec['gflops']:.1f}, {key} [{rec['status']}]", flush=True)
    return recs


def emit_best(out: str, best: Dict):
    src = point_dir(out)
    for ext in ("co", "toml"):
        shutil.copyfile(os.path.join(src, f"{best['point']}.{ext}"), os.path.join(out, f"generated_gemm.{ext}"))


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--m", dest="m", type=int, required=True, action="store")
    ap.add_argument("--n", dest="n", type=int, required=True, action="store")
    ap.add_argument("--k", dest="k", type=int, required=True, action="store")
    ap.add_argument("--bench", dest="bench", type=str, required=True, action="store")
    ap.add_argument("--output-folder", dest="output_folder", type=str, required=True, action="store")
    ap.add_argument("--space", choices=["gfx950", "gfx950-wide", "reference"], default="gfx950")
    ap.add_argument("--refine", type=int, default=3, help="geometries refined in stage 2")
    ap.add_argument("--results", default=None, help="JSONL results file (default <out>/results.jsonl)")
    ap.add_argument("--compile-only", action="store_true")
    ap.add_argument("--no-compile", action="store_true")
    ap.add_argument("--in-process", action="store_true")
    ap.add_argument("--timeout", type=float, default=120.0)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--runs", type=int, default=50)
    ap.add_argument("--jobs", type=int, default=min(16, os.cpu_count() or 1))
    ap.add_argument("--points-dir", default=None, help="compiled candidates (default <out>/points)")
    ap.add_argument("--all-shapes", action="store_true",
                    help="with --compile-only: build the stage-2 candidates of every geometry")
    ap.add_argument("--split-k", default="1",
                    help="comma-separated split-K values for stage 2 (0 = chosen per problem; default 1: no split)")
    ap.add_argument("--occ", default="0,2",
                    help="comma-separated occupancy targets for stage 2 (0 = compiler's choice; 2 = two waves per SIMD)")
    args = ap.parse_args(argv)
    m, n, k, out = args.m, args.n, args.k, args.output_folder
    split_ks = [int(x) for x in args.split_k.split(",") if x.strip()]
    occs = [int(x) for x in args.occ.split(",") if x.strip()]
    os.makedirs(out, exist_ok=True)
    global POINTS_DIR
    POINTS_DIR = args.points_dir
    results_path = args.results or os.path.join(out, "results.jsonl")

    if args.space == "reference":
        stage1 = [p for p in reference_points() if fits(p[0], m, n, k)]
    else:
        stage1 = [p for p in geometry_points(DEFAULT_KNOBS, wide=args.space == "gfx950-wide", occs=occs,
                                             depths=STAGE1_DEPTHS) if fits(p[0], m, n, k)]

    if args.compile_only:
        pts = list(stage1)
        if args.all_shapes and args.space != "reference":
            for cfg, _ in stage1:
                pts += [p for p in knob_points(cfg, split_ks, occs) if fits(p[0], m, n, k)]
        res = build_points(out, pts, args.jobs)
        bad = sum(1 for v in res.values() if v)
        print(f"compiled {len(res) - bad} of {len(res)} candidates into {point_dir(out)}")
        return 0

    if args.in_process:
        bench = InProcessBench(m, n, k, args.warmup, args.runs)
    else:
        bench = RunnerBench(args.bench, m, n, k, args.warmup, args.runs)

    def compiled_for(points):
        if args.no_compile:
            return {point_key(*p): 0 for p in points}
        return build_points(out, points, args.jobs)

    recs = sweep(stage1, out, m, n, k, bench, args.timeout, results_path, compiled_for(stage1))
    if args.space != "reference" and args.refine > 0:
        ranked = sorted((r for r in recs if r["status"] == "ok"), key=lambda r: -r["gflops"])[:args.refine]
        by_key = {point_key(*p): p for p in stage1}
        stage2: List[Point] = []
        seen = set(by_key)
        for r in ranked:
            cfg = by_key[r["point"]][0]
            for p in knob_points(cfg, split_ks, occs):
                kk = point_key(*p)
                if kk not in seen and fits(p[0], m, n, k):
                    seen.add(kk)
                    stage2.append(p)
        recs += sweep(stage2, out, m, n, k, bench, args.timeout, results_path, compiled_for(stage2))

    ok = [r for r in recs if r["status"] == "ok" and r["gflops"] > 0]
    if not ok:
        print("No valid configurations found.")
        return 1
    best = max(ok, key=lambda r: r["gflops"])
    emit_best(out, best)
    print(f"Best: {best['gflops']:.1f} Gflops ({best['gflops'] / 1e3 / 157.3 * 100:.1f}% of the FP32 MFMA peak), "
          f"MT: {tuple(best['tile'])}, DK: {best['depth_k']}, MI: {tuple(best['mfma'])}, wg: {tuple(best['wave_group'])}, "
          f"wgm: {best['wgm']}, plr: {best['plr']}, gw: {best['gw']}, map_k_idx: {best['map_k_idx']}, "
          f"vmem_stage: {best['vmem_stage']}, xcd: {best['xcd']}, split_k: {best.get('split_k', 1)}, "
          f"occ: {best.get('occ', 0)} -> {out}/generated_gemm.co")
    return 0


if __name__ == "__main__":
    sys.exit(main())
