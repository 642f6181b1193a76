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
  applies to both stages, and stage 1 tries depth_k 16 and 32 (``--stage1-depths``);
  ``--gw`` adds the epilogue flavour to stage 2 and ``--tiles`` narrows stage
  1's macro-tiles.  ``--space reference`` is the reference's own 9-knob product.
* every result is appended to ``<out>/results.jsonl`` with the point's
  ``source_sha`` (generated source, compiler and flags); a rerun skips points
  already there with the same sha (resume) and rebuilds and re-times the
  others, so an edited kernel is never timed from a stale code object;
* each point runs in isolation: compile failures, runner failures and
  ``--timeout`` expiries are recorded and the sweep continues (the reference
  aborts on the first failing point, sgemm_tuner.py:121-123);
* the fastest point that passes validation (the runner's validation_flag = 1
  on the shape clipped to 1024 per dimension) is re-emitted as
  ``<out>/generated_gemm.co`` + ``.toml`` (the reference overwrites one
  artifact per point and keeps none, :67, :107);
* ``--playoff N`` times the N fastest points again, ``--playoff-rounds``
  times round-robin with the order reversed every other round, and emits by
  their medians: one timing per point ranks points within 1-2% of each other
  by noise and by what ran before them;
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
import statistics
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
    DEFAULT_HIPCC_PATH,
    HIPCC_KERNEL_FLAGS,
    DataType,
    FunctionArgument,
    GemmOptimizations,
    GemmSolutionConfig,
    compile,
    default_arguments,
    launch_geometry,
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
GFX950_DEPTH_K = [16, 24, 32, 64]
GFX950_VMEM_STAGES = [1, 2]
GFX950_WGM = [1, 4, 8]
GFX950_XCD = [0, 8]
GFX950_PLR = [1, 2, 3]
GFX950_PD = [1, 2]
GFX950_GW = [1, 0]
DEFAULT_KNOBS = dict(depth_k=16, vmem_stage=2, wgm=4, xcd=8, plr=3, gw=1, map_k_idx=0)
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
            + (f"_sk{opt.split_k}" if opt.split_k != 1 else "")
            + (f"_ws{opt.ws_pd}" if opt.ws else "") + ("_ks" if opt.ksplit else "")
            + ("_" + ("t" if cfg.trans_a else "n") + ("t" if cfg.trans_b else "n")
               if cfg.trans_a or cfg.trans_b else ""))


def make_point(mfma, wg, wt, depth_k, vmem_stage, wgm, plr, gw, map_k_idx, xcd, pd=1, occ=0,
               split_k=1, trans: Tuple[bool, bool] = (False, False), ws: int = 0, ksplit: int = 0) -> Optional[Point]:
    """One candidate; ``trans`` = (trans_a, trans_b) builds it for op(A) = A^T
    and/or op(B) = B^T (the reference's schema fields, generator.py:1007-1009);
    ``ws`` = 1 adds as many loading waves as the geometry has computing ones,
    ``ksplit`` = 1 a second group of them for half of the K tiles."""
    try:
        cfg = GemmSolutionConfig(F, F, F, F, mfma, wg, wt, depth_k, trans[0], trans[1], vmem_stage=vmem_stage)
        opt = GemmOptimizations(1, wgm=wgm, plr=plr, gw=gw, map_k_idx=map_k_idx, xcd=xcd, pd=pd, occ=occ,
                                split_k=split_k, ws=ws, ksplit=ksplit)
        launch_geometry(cfg, opt)  # raises where the geometry cannot take the second half of waves
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
                    depths: Sequence[int] = (16,), tiles: Optional[Sequence[Tuple[int, int]]] = None,
                    trans: Tuple[bool, bool] = (False, False)) -> Iterable[Point]:
    """Stage-1 candidates: every macro-tile x wave-group x atom geometry at the
    default code-shape knobs, once per occupancy target in ``occs`` and K
    depth in ``depths``: a geometry that only pays with two work-groups per
    CU (the 4096^3 winner, 256 x 128) or with a deeper K tile (16x16x4 atoms:
    128 x 64 runs 30% faster at depth 32 than at 16) must reach stage 2 at
    that setting.  ``tiles`` narrows the macro-tiles to the given list;
    ``trans`` is the operands' layout."""
    if tiles is None:
        tiles = GFX950_WIDE_MACRO_TILES if wide else GFX950_MACRO_TILES
    groups = GFX950_WIDE_WAVE_GROUPS if wide else GFX950_WAVE_GROUPS
    for (mt0, mt1), wg, mfma, occ, dk in product(tiles, groups, SUPPORTED_MFMAS, occs, depths):
        if mt0 % (mfma[0] * wg[0]) or mt1 % (mfma[1] * wg[1]):
            continue
        wt = (mt0 // (mfma[0] * wg[0]), mt1 // (mfma[1] * wg[1]))
        p = make_point(mfma, wg, wt, dk, knobs["vmem_stage"], knobs["wgm"], knobs["plr"], knobs["gw"],
                       knobs["map_k_idx"], knobs["xcd"], occ=occ, trans=trans)
        if p:
            yield p


def knob_points(cfg: GemmSolutionConfig, split_ks: Sequence[int] = (1,), occs: Sequence[int] = (0,),
                gws: Sequence[int] = (1,), wss: Sequence[int] = (0,), kss: Sequence[int] = (0,)) -> Iterable[Point]:
    """Stage-2 candidates of one geometry; ``split_ks`` and ``occs`` add the
    gfx950-only split-K (0 = chosen per problem) and occupancy knobs, ``gws``
    the epilogue flavour (1: staged through LDS, 0: stores straight from the
    accumulators), ``wss`` wave specialisation (1: loading waves beside the
    computing ones; no split-K, no occupancy cap, one to three extra LDS
    buffers), ``kss`` the in-group K split (1: a second group of waves
    multiplies half of the K tiles in its own LDS ring; no split-K, no
    occupancy cap, not with ws).  The layout is ``cfg``'s."""
    for dk, st, wgm, xcd, plr, pd, sk, occ, gw, ws, ks in product(GFX950_DEPTH_K, GFX950_VMEM_STAGES + [3],
                                                                  GFX950_WGM, GFX950_XCD, GFX950_PLR, GFX950_PD,
                                                                  split_ks, occs, gws, wss, kss):
        if pd == 2 and plr < 2:
            continue
        if st == 3 and not ws:   # the fourth buffer pays only for the wave-specialised ring
            continue
        if ws and (sk != 1 or occ or pd != 1):
            continue
        if ks and (ws or sk != 1 or occ):
            continue
        p = make_point(cfg.mfma, cfg.wave_group, cfg.wave_tiling, dk, st, wgm, plr, gw, 0, xcd, pd, occ, sk,
                       (cfg.trans_a, cfg.trans_b), ws, ks)
        if p:
            yield p


def reference_points(trans: Tuple[bool, bool] = (False, False)) -> Iterable[Point]:
    for wg, wt, mfma, dk, wgm, plr, gw, mk, st in product(
            SUPPORTED_WAVE_GROUPS, SUPPORTED_WAVE_TILINGS, SUPPORTED_MFMAS, SUPPORTED_DEPTH_K, SUPPORTED_WGM,
            SUPPORTED_PLR, SUPPORTED_GW, SUPPORTED_MAP_K_IDX, SUPPORTED_VMEM_STAGES):
        p = make_point(mfma, wg, wt, dk, st, wgm, plr, gw, mk, 0, trans=trans)
        if p:
            yield p


# --------------------------------------------------------------- building
POINTS_DIR: Optional[str] = None


def point_dir(out: str) -> str:
    return POINTS_DIR or os.path.join(out, "points")


def point_source(p: Point) -> Tuple[str, str]:
    """(HIP source, source_sha) of a point: the sha covers everything the code
    object is built from -- the generated source (kernel template plus the
    point's defines) and the compiler and its flags."""
    cfg, opt = p
    cfg.name = point_key(cfg, opt)
    src = gemm(None, "generated_gemm", ARCH, cfg, opt, default_arguments())
    h = hashlib.sha256()
    for part in (src, DEFAULT_HIPCC_PATH, " ".join(HIPCC_KERNEL_FLAGS), ARCH):
        h.update(part.encode())
        h.update(b"\0")
    return src, h.hexdigest()[:16]


def built_sha(out: str, key: str) -> Optional[str]:
    """source_sha recorded in a compiled point's .toml (None if absent)."""
    co = os.path.join(point_dir(out), f"{key}.co")
    toml = os.path.join(point_dir(out), f"{key}.toml")
    if not (os.path.exists(co) and os.path.exists(toml)):
        return None
    return read_toml(toml).get("source_sha")


def build_point(out: str, p: Point) -> Tuple[str, int]:
    """Compiles one point unless an up-to-date build is there: a .co/.toml pair
    whose source_sha matches the current source (an edit to the kernel
    template, the generator's defines or the flags rebuilds it)."""
    cfg, opt = p
    key = point_key(cfg, opt)
    d = point_dir(out)
    src, sha = point_source(p)
    if built_sha(out, key) == sha:
        return key, 0
    rc = compile(key, src, ARCH, d, cfg, opt, extra_keys={"source_sha": sha})
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
    """Times candidates through the ctypes shim with inputs uploaded once.

    Each candidate first runs for ``warm_ms`` milliseconds of launches: the
    engine clock falls within ~20 ms of idle (loading a candidate is enough)
    and takes ~35 ms of load to come back, so without it every point is timed
    on a ramping clock (1024^3 then measures ~12% low)."""

    def __init__(self, m, n, k, warmup, runs, warm_ms=50.0):
        from shim import sgemm_shim as S
        self.S = S
        self.m, self.n, self.k, self.warmup, self.runs = m, n, k, warmup, runs
        self.warm_ms = warm_ms
        A = S.fill_matrix(m, k, 1, 0)
        B = S.fill_matrix(k, n, 1, 1)
        self.dA, self.dB = S.DeviceBuffer.from_array(A), S.DeviceBuffer.from_array(B)
        self.dD = S.DeviceBuffer(m * n * 4)

    def __call__(self, co, toml, timeout) -> Tuple[int, float]:
        with self.S.Kernel(co, toml) as kern:
            args = (self.dA, self.dB, None, self.dD, self.m, self.n, self.k, 1.0, 0.0)
            t0 = time.perf_counter()
            while (time.perf_counter() - t0) * 1e3 < self.warm_ms:
                kern.time(*args, warmup=0, runs=5)
            ms = kern.time(*args, warmup=self.warmup, runs=self.runs) / self.runs
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
    for p in points:
        cfg, opt = p
        key = point_key(cfg, opt)
        _, sha = point_source(p)
        rkey = f"{shape}:{key}"
        # resume only results of the same source: a record of an older kernel
        # template, generator or flags is benchmarked again
        if rkey in done and done[rkey].get("source_sha") == sha:
            recs.append(done[rkey])
            continue
        rec = {"key": rkey, "point": key, "shape": [m, n, k], "tile": list(cfg.tile_size), "mfma": list(cfg.mfma),
               "wave_group": list(cfg.wave_group), "wave_tiling": list(cfg.wave_tiling), "depth_k": cfg.depth_k,
               "vmem_stage": cfg.vmem_stage, "trans_a": cfg.trans_a, "trans_b": cfg.trans_b, **opt.to_dict(),
               "source_sha": sha, "gflops": 0.0, "status": "ok"}
        co = os.path.join(point_dir(out), f"{key}.co")
        toml = os.path.join(point_dir(out), f"{key}.toml")
        if compiled.get(key, 0) != 0 or not os.path.exists(co):
            rec["status"] = "compile_error"
        elif built_sha(out, key) != sha:
            rec["status"] = "stale_build"   # built from other sources (--no-compile over an old build)
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


def validation_shape(m: int, n: int, k: int) -> Tuple[int, int, int]:
    """The tuned shape clipped to at most 1024 per dimension: a CPU reference
    GEMM of it takes about a second on a few host threads."""
    return min(m, 1024), min(n, 1024), min(k, 1024)


class RunnerValidator:
    """The reference's check: the runner with validation_flag = 1 (its own CPU
    GEMM; normwise 1e-5 * sqrt(K) and elementwise |gpu - cpu| < 1e-3) on
    validation_shape(m, n, k)."""

    def __init__(self, bench, m, n, k, timeout=600.0):
        self.bench, self.shape, self.timeout = bench, validation_shape(m, n, k), timeout

    def __call__(self, co, toml) -> Tuple[bool, str]:
        m, n, k = self.shape
        ret = subprocess.run([self.bench, co, toml, str(m), str(n), str(k), "0", "1", "1"], stdout=subprocess.PIPE,
                             stderr=subprocess.STDOUT, timeout=self.timeout)
        out = ret.stdout.decode(errors="replace")
        ok = ret.returncode == 0 and "validation: PASS" in out
        detail = [ln for ln in out.splitlines() if ln.startswith(("normwise", "# of mismatches", "validation"))]
        return ok, f"{m}x{n}x{k}: " + "; ".join(detail)


class ShimValidator:
    """For --in-process sweeps without a runner executable: the kernel through
    the C-ABI shim on validation_shape(m, n, k), against a float64 numpy GEMM
    of the same seeded inputs, normwise bar 1e-5 * sqrt(K)."""

    def __init__(self, m, n, k):
        self.shape = validation_shape(m, n, k)

    def __call__(self, co, toml) -> Tuple[bool, str]:
        import numpy as np
        from shim import sgemm_shim as S
        m, n, k = self.shape
        with S.Kernel(co, toml) as kern:
            sa = (k, m) if kern.info.trans_a else (m, k)
            sb = (n, k) if kern.info.trans_b else (k, n)
            A = S.fill_matrix(*sa, 7, 0)
            B = S.fill_matrix(*sb, 7, 1)
            C = S.fill_matrix(m, n, 7, 2)
            D, _ = kern.run(A, B, C, m, n, k, alpha=1.0, beta=1.0)
            opA = A.T if kern.info.trans_a else A
            opB = B.T if kern.info.trans_b else B
        ref = opA.astype(np.float64) @ opB.astype(np.float64) + C.astype(np.float64)
        err = float(np.max(np.abs(D - ref)) / max(np.max(np.abs(ref)), 1e-30))
        tol = 1e-5 * max(k, 1) ** 0.5
        return bool(err <= tol), f"{m}x{n}x{k}: normwise error vs float64 {err:.3e} (tolerance {tol:.3e})"


def playoff(recs: List[Dict], out: str, bench, top: int, rounds: int, timeout: float) -> List[Dict]:
    """Times the ``top`` fastest points again, ``rounds`` times round-robin
    with the order reversed every other round, and stores each one's median
    as ``playoff_gflops`` (its timings in ``playoff``).  A single timing per
    point ranks points within 1-2% of each other by noise and by what ran
    before them; the median of interleaved timings does not.  Returns the
    participants, fastest median first."""
    cands = sorted((r for r in recs if r["status"] == "ok" and r["gflops"] > 0), key=lambda r: -r["gflops"])[:top]
    if len(cands) < 2 or rounds < 1:
        return cands
    for rec in cands:
        rec["playoff"] = []
    for r in range(rounds):
        for rec in (cands if r % 2 == 0 else cands[::-1]):
            co = os.path.join(point_dir(out), f"{rec['point']}.co")
            toml = os.path.join(point_dir(out), f"{rec['point']}.toml")
            try:
                rc, gflops = bench(co, toml, timeout)
            except Exception as e:  # a point that fails now drops out of the ranking
                print(f"playoff: {rec['point']} failed ({e})", flush=True)
                continue
            if rc == 0 and gflops > 0:
                rec["playoff"].append(gflops)
    for rec in cands:
        rec["playoff_gflops"] = statistics.median(rec["playoff"]) if rec["playoff"] else 0.0
        print(f"playoff: {rec['playoff_gflops']:.1f} Gflops median of {len(rec['playoff'])} "
              f"(single timing {rec['gflops']:.1f}), {rec['point']}", flush=True)
    return sorted(cands, key=lambda r: -r["playoff_gflops"])


def emit_best(out: str, recs: List[Dict], validate=None) -> Optional[Dict]:
    """Copies the fastest point that passes ``validate(co, toml) -> (ok, detail)``
    to <out>/generated_gemm.co + .toml and returns its record (None if no
    point passes); a point that fails is marked and the next one tried.
    Points that went through ``playoff`` come first, by their median; the
    others follow by their single timing."""
    src = point_dir(out)

    def rank(r):
        if "playoff_gflops" in r:
            return (0, -r["playoff_gflops"])
        return (1, -r["gflops"])

    ok = [r for r in recs if r["status"] == "ok" and r["gflops"] > 0 and r.get("playoff_gflops", 1.0) > 0]
    for rec in sorted(ok, key=rank):
        co = os.path.join(src, f"{rec['point']}.co")
        toml = os.path.join(src, f"{rec['point']}.toml")
        if validate is not None:
            ok, detail = validate(co, toml)
            rec["validation"] = detail
            print(f"validation of {rec['point']}: {'PASS' if ok else 'FAIL'} ({detail})", flush=True)
            if not ok:
                continue
        for ext, path in (("co", co), ("toml", toml)):
            shutil.copyfile(path, os.path.join(out, f"generated_gemm.{ext}"))
        return rec
    return None


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
    ap.add_argument("--warm-ms", type=float, default=50.0,
                    help="--in-process: milliseconds of launches before timing each candidate (clock ramp)")
    ap.add_argument("--jobs", type=int, default=min(16, os.cpu_count() or 1))
    ap.add_argument("--points-dir", default=None, help="compiled candidates (default <out>/points)")
    ap.add_argument("--all-shapes", action="store_true",
                    help="with --compile-only: build the stage-2 candidates of every geometry")
    ap.add_argument("--split-k", default="1",
                    help="comma-separated split-K values for stage 2 (0 = chosen per problem; default 1: no split)")
    ap.add_argument("--occ", default="0,2",
                    help="comma-separated occupancy targets (waves per SIMD) for stages 1 and 2 (0 = compiler's "
                         "choice; 2 / 4 = registers capped for two / four)")
    ap.add_argument("--gw", default="1",
                    help="comma-separated epilogue flavours for stage 2 (1 = staged through LDS, 0 = direct stores)")
    ap.add_argument("--ws", default="0",
                    help="comma-separated wave-specialisation settings for stage 2 (1 = loading waves beside the "
                         "computing ones, K buffers ordered by LDS counters; default 0)")
    ap.add_argument("--ksplit", default="0",
                    help="comma-separated in-group K split settings for stage 2 (1 = a second group of waves "
                         "multiplies half of the K tiles, the sums meet in LDS; default 0)")
    ap.add_argument("--tiles", default=None,
                    help="comma-separated macro-tiles MT0xMT1 for stage 1 (default: the --space list)")
    ap.add_argument("--stage1-depths", default=",".join(str(d) for d in STAGE1_DEPTHS),
                    help="comma-separated K depths every stage-1 geometry is tried at")
    ap.add_argument("--summary", default=None, help="write a markdown summary of the sweep to this path")
    ap.add_argument("--playoff", type=int, default=0, metavar="N",
                    help="time the N fastest points again, interleaved, and emit by median (0: off)")
    ap.add_argument("--playoff-rounds", type=int, default=6)
    ap.add_argument("--trans-a", action="store_true", help="op(A) = A^T: A stored k x m (lda >= k)")
    ap.add_argument("--trans-b", action="store_true", help="op(B) = B^T: B stored n x k (ldb >= n)")
    args = ap.parse_args(argv)
    m, n, k, out = args.m, args.n, args.k, args.output_folder
    split_ks = [int(x) for x in args.split_k.split(",") if x.strip()]
    occs = [int(x) for x in args.occ.split(",") if x.strip()]
    gws = [int(x) for x in args.gw.split(",") if x.strip()]
    wss = [int(x) for x in args.ws.split(",") if x.strip()]
    kss = [int(x) for x in args.ksplit.split(",") if x.strip()]
    depths = [int(x) for x in args.stage1_depths.split(",") if x.strip()]
    tiles = None
    if args.tiles:
        tiles = [tuple(int(v) for v in t.lower().split("x")) for t in args.tiles.split(",") if t.strip()]
    os.makedirs(out, exist_ok=True)
    global POINTS_DIR
    POINTS_DIR = args.points_dir
    results_path = args.results or os.path.join(out, "results.jsonl")

    trans = (args.trans_a, args.trans_b)
    if args.space == "reference":
        stage1 = [p for p in reference_points(trans) if fits(p[0], m, n, k)]
    else:
        stage1 = [p for p in geometry_points(DEFAULT_KNOBS, wide=args.space == "gfx950-wide", occs=occs,
                                             depths=depths, tiles=tiles, trans=trans) if fits(p[0], m, n, k)]

    if args.compile_only:
        pts = list(stage1)
        if args.all_shapes and args.space != "reference":
            for cfg, _ in stage1:
                pts += [p for p in knob_points(cfg, split_ks, occs, gws, wss, kss) if fits(p[0], m, n, k)]
        res = build_points(out, pts, args.jobs)
        bad = sum(1 for v in res.values() if v)
        print(f"compiled {len(res) - bad} of {len(res)} candidates into {point_dir(out)}")
        return 0

    if args.in_process:
        bench = InProcessBench(m, n, k, args.warmup, args.runs, args.warm_ms)
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
            for p in knob_points(cfg, split_ks, occs, gws, wss, kss):
                kk = point_key(*p)
                if kk not in seen and fits(p[0], m, n, k):
                    seen.add(kk)
                    stage2.append(p)
        recs += sweep(stage2, out, m, n, k, bench, args.timeout, results_path, compiled_for(stage2))

    ok = [r for r in recs if r["status"] == "ok" and r["gflops"] > 0]
    if not ok:
        print("No valid configurations found.")
        return 1
    if args.playoff > 1:
        playoff(recs, out, bench, args.playoff, args.playoff_rounds, args.timeout)
    # the emitted pair is checked first: the runner's own CPU validation when
    # the --bench executable exists, else the shim against a float64 GEMM
    validate = RunnerValidator(args.bench, m, n, k) if os.path.isfile(args.bench) else ShimValidator(m, n, k)
    best = emit_best(out, recs, validate)
    if best is None:
        print("No configuration passed validation.")
        return 1
    print(f"Best: {best['gflops']:.1f} Gflops ({best['gflops'] / 1e3 / 157.3 * 100:.1f}% of the FP32 MFMA peak), "
          f"MT: {tuple(best['tile'])}, DK: {best['depth_k']}, MI: {tuple(best['mfma'])}, wg: {tuple(best['wave_group'])}, "
          f"wgm: {best['wgm']}, plr: {best['plr']}, gw: {best['gw']}, map_k_idx: {best['map_k_idx']}, "
          f"vmem_stage: {best['vmem_stage']}, xcd: {best['xcd']}, split_k: {best.get('split_k', 1)}, "
          f"trans_a: {best.get('trans_a', False)}, trans_b: {best.get('trans_b', False)}, "
          f"occ: {best.get('occ', 0)} -> {out}/generated_gemm.co")
    if args.summary:
        write_summary(args.summary, recs, best, m, n, k, argv if argv is not None else sys.argv[1:])
    return 0


def write_summary(path: str, recs: List[Dict], best: Dict, m: int, n: int, k: int, argv: Sequence[str],
                  top: int = 10):
    """Markdown summary of a sweep: the command, points by status, the top
    points by Gflops and the emitted (validated) winner."""
    from collections import Counter
    status = Counter(r["status"] if not r["status"].startswith("error") else "error" for r in recs)
    ok = sorted((r for r in recs if r["status"] == "ok" and r["gflops"] > 0), key=lambda r: -r["gflops"])
    lines = [f"# Tuner sweep at {m}x{n}x{k}", "", "Command (from the repository root on the GPU box):", "",
             "    python amdgpu-arch-gemm_amd/tuner/sgemm_tuner.py " + " ".join(argv), "",
             f"{len(recs)} points: " + ", ".join(f"{v} {s}" for s, v in sorted(status.items())) + ".", "",
             f"| rank | point | tile | TFLOP/s | % of {157.3} |", "|---|---|---|---|---|"]
    for i, r in enumerate(ok[:top], 1):
        lines.append(f"| {i} | `{r['point']}` | {r['tile'][0]}x{r['tile'][1]} | {r['gflops'] / 1e3:.2f} | "
                     f"{r['gflops'] / 1e3 / 157.3 * 100:.1f} |")
    po = sorted((r for r in recs if "playoff_gflops" in r), key=lambda r: -r["playoff_gflops"])
    if po:
        lines += ["", f"Playoff ({len(po[0]['playoff'])} interleaved rounds, order reversed every other round):", "",
                  "| point | single timing TFLOP/s | median TFLOP/s |", "|---|---|---|"]
        lines += [f"| `{r['point']}` | {r['gflops'] / 1e3:.2f} | {r['playoff_gflops'] / 1e3:.2f} |" for r in po]
    speed = (f"{best['playoff_gflops'] / 1e3:.2f} TFLOP/s (playoff median)" if "playoff_gflops" in best
             else f"{best['gflops'] / 1e3:.2f} TFLOP/s")
    lines += ["", f"Emitted `generated_gemm.co` + `.toml`: `{best['point']}`, {speed}; "
              f"validation {best.get('validation', 'not run')}.", ""]
    os.makedirs(os.path.dirname(os.path.abspath(path)), exist_ok=True)
    with open(path, "w") as f:
        f.write("\n".join(lines))


if __name__ == "__main__":
    sys.exit(main())
