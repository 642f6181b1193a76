"""Measure how gfx950's LDS serves wave-wide accesses (bank conflicts).

Three kinds of patterns are replayed by ``lds_probe`` (one dispatch each) under
``rocprofv3 --pmc SQ_LDS_BANK_CONFLICT SQ_LDS_IDX_ACTIVE``:

* pair tests -- lane 0 at byte 0, lane j at byte 256 (the same banks, another
  dword), every other lane reading or writing one shared address elsewhere:
  a conflict shows that lanes 0 and j are served in the same LDS cycle, so the
  tests map which lanes share a cycle for 4-, 8- and 16-byte accesses;
* strides -- lane l at l x stride bytes;
* the SGEMM kernel's own tile accesses (``generator.lds_tile_accesses``: the
  A/B tile writes of every wave and the operand reads, the address formulas of
  ``csrc/sgemm_gfx950.hip``) for each LDS pad and for the generator's chosen
  layout (pads and B-chunk swizzle), per catalog instance.

  python lds_banks.py --out <dir>            # GPU: write patterns, run, summarise
  python lds_banks.py --out <dir> --analyze  # summarise an earlier run

The summary (markdown) maps the lanes served per cycle, the conflict cycles of
strided patterns, and per instance and layout the measured and modelled
conflict cycles per K tile.  The SGEMM kernels are not run; only ``lds_probe``.
"""
from __future__ import annotations

import argparse
import csv
import glob
import os
import statistics
import subprocess
import sys
import zlib
from typing import Dict, List, Tuple

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
ROOT = os.path.dirname(PKG)
sys.path.insert(0, PKG)

from generator import catalog  # noqa: E402
from generator.generator import lds_access_cycles, lds_epilogue_accesses, lds_lane_cycle, lds_tile_accesses  # noqa: E402

PROBE = os.path.join(HERE, "lds_probe")
LDS_BYTES = 64 * 1024
ITERS = 256
WAVES = 256
PADS = (0, 4, 8, 12, 16)
# instances whose kernel accesses are measured
INSTANCES = (
    "mt256x128_a32_wg2x2_dk16_s3_occ2",
    "mt256x128_a32_wg4x2_dk16_s3_occ4_plr2",
    "mt128x64_a16_wg2x4_dk64",
    "mt256x256_a32_wg2x2_dk24_s3",
    "mt256x256_a32_wg2x2_dk16_s3",
    "mt128x64_a16_wg2x2_dk32_s3_occ2",
    "mt64x64_a16_wg1x4_dk32_s3",
    "mt16x128_a16_wg1x4_dk64_s2",
    "mt64x16_a16_wg4x1_dk64_s3",
    "mt256x256_a32_wg2x2_dk16_s3_tn",
    "mt256x256_a32_wg2x2_dk16_s3_nt",
    "mt256x128_a32_wg2x2_dk16_s3_occ2_tn",
    "mt256x128_a32_wg4x2_dk16_s3_occ4_plr2_tt",
    "mt128x64_a16_wg2x4_dk64_nt",
)

Pattern = Tuple[str, str, int, List[int]]  # name, r|w, bytes per lane, 64 byte addresses


def pair_patterns() -> List[Pattern]:
    out = []
    for width in (4, 8, 16):
        for op in ("r", "w"):
            for j in range(1, 64):
                for tag, aj in (("pair", 256), ("same", 0)):
                    addr = [64] * 64  # banks 16.. : away from lanes 0 and j
                    addr[0] = 0
                    addr[j] = aj
                    out.append((f"{tag}_b{width * 8}_{op}_{j}", op, width, addr))
    return out


def stride_patterns() -> List[Pattern]:
    out = []
    for width in (4, 8, 16):
        for op in ("r", "w"):
            for s in (1, 2, 3, 4, 5, 8, 16, 17, 32, 33, 64):
                stride = width * s
                if 63 * stride + width > LDS_BYTES:
                    continue
                out.append((f"stride_b{width * 8}_{op}_{stride}B", op, width, [l * stride for l in range(64)]))
    return out


def kernel_layouts(name: str):
    """(label, operand, pad, chunk swizzle, row swizzle) of the layouts
    measured for an instance: each pad without a swizzle, and the generator's
    choice."""
    cfg, _ = catalog.SOLUTIONS[name]
    pad_a, pad_b, shift, mask, a_shift, a_mask, r_shift, r_mask = cfg.lds_layout
    out = [(f"pad{p}", op, p, (0, 0), (0, 0)) for op in ("a", "b") for p in PADS]
    out += [("chosen", "a", pad_a, (a_shift, a_mask), (r_shift, r_mask)), ("chosen", "b", pad_b, (shift, mask), (0, 0))]
    return out


def kernel_accesses(name: str, operand: str, pad: int, swz: Tuple[int, int], rsw: Tuple[int, int] = (0, 0)):
    cfg, _ = catalog.SOLUTIONS[name]
    return lds_tile_accesses(cfg.mfma, cfg.wave_group, cfg.wave_tiling, cfg.depth_k, cfg.trans_a, cfg.trans_b,
                             operand, pad, swz, rsw)


# staged-epilogue layouts measured per instance: (label, column pad in floats,
# run swizzle, 16-byte grouped writes)
EPILOGUE_LAYOUTS = (
    ("one write per slot, pad 4", 4, False, False),
    ("grouped writes, pad 4", 4, False, True),
    ("kernel: grouped writes, run ^ column, pad 0", 0, True, True),
)


def epilogue_accesses(name: str, pad: int, swizzle: bool, grouped: bool):
    cfg, _ = catalog.SOLUTIONS[name]
    return lds_epilogue_accesses(cfg.mfma, cfg.wave_group, cfg.wave_tiling, pad, swizzle, grouped)


def kernel_patterns() -> List[Pattern]:
    """Every distinct wave-wide access of each measured layout (the waves'
    operand reads differ by uniform offsets; their tile writes are listed per
    wave), named by its address pattern so that layouts share dispatches."""
    out, seen = [], set()

    def add(accesses):
        for kind, wave, addrs, width, write, _ in accesses:
            key = _pattern_key(addrs, width, write)
            if key not in seen and max(addrs) + width <= LDS_BYTES:
                seen.add(key)
                out.append((key, "w" if write else "r", width, list(addrs)))

    for name in INSTANCES:
        for _, operand, pad, swz, rsw in kernel_layouts(name):
            add(kernel_accesses(name, operand, pad, swz, rsw))
        for _, pad, swizzle, grouped in EPILOGUE_LAYOUTS:
            add(epilogue_accesses(name, pad, swizzle, grouped))
    return out


def _pattern_key(addrs, width, write) -> str:
    digest = zlib.crc32(",".join(str(a) for a in addrs).encode())
    return f"k{'w' if write else 'r'}{width}_{digest:08x}"


def write_patterns(path: str) -> List[Pattern]:
    pats = pair_patterns() + stride_patterns() + kernel_patterns()
    with open(path, "w") as f:
        for name, op, width, addr in pats:
            f.write(f"{name} {op} {width} {' '.join(str(a) for a in addr)}\n")
    return pats


def run(cmd: List[str], timeout: int) -> None:
    print("+", " ".join(cmd), flush=True)
    subprocess.run(cmd, check=True, timeout=timeout)


def collect(out: str, pats: List[Pattern]) -> Dict[str, Tuple[float, float]]:
    """pattern name -> (conflict cycles, active cycles) per wave-wide instruction."""
    files = glob.glob(os.path.join(out, "pmc", "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise RuntimeError(f"no counter file under {out}/pmc")
    per: Dict[int, Dict[str, float]] = {}
    with open(files[0]) as f:
        for row in csv.DictReader(f):
            if "lds_probe_kernel" not in row["Kernel_Name"]:
                continue
            d = per.setdefault(int(row["Dispatch_Id"]), {})
            d[row["Counter_Name"]] = d.get(row["Counter_Name"], 0.0) + float(row["Counter_Value"])
    ids = sorted(per)
    if len(ids) != len(pats):
        raise RuntimeError(f"{len(ids)} probe dispatches for {len(pats)} patterns")
    instr = float(WAVES * 8 * ITERS)
    return {p[0]: (per[i]["SQ_LDS_BANK_CONFLICT"] / instr, per[i]["SQ_LDS_IDX_ACTIVE"] / instr)
            for p, i in zip(pats, ids)}


def summarise(res: Dict[str, Tuple[float, float]], pats: List[Pattern], cmd: str) -> str:
    lines = ["# LDS bank behaviour of gfx950 (`lds_probe`)", "",
             "Command (from the repository root on the GPU box):", "", f"    {cmd}", "",
             "Figures are `SQ_LDS_BANK_CONFLICT` and `SQ_LDS_IDX_ACTIVE` per wave-wide LDS instruction "
             f"({WAVES} one-wave work-groups x {ITERS} x 8 instructions per dispatch).", ""]
    lines += ["## Which lanes share an LDS cycle", "",
              "Lane 0 at byte 0 and lane j at byte 256 (same banks, different dword); the other lanes share "
              "one address. `pair` minus `same` (lane j at byte 0 instead) is the conflict the pair causes.", "",
              "| access | lanes j whose pair conflicts with lane 0 | conflict cycles of such a pair |", "|---|---|---|"]
    for width in (4, 8, 16):
        for op in ("r", "w"):
            hits, extra = [], []
            for j in range(1, 64):
                d = res[f"pair_b{width * 8}_{op}_{j}"][0] - res[f"same_b{width * 8}_{op}_{j}"][0]
                if d > 0.5:
                    hits.append(j)
                    extra.append(d)
            lines.append(f"| ds_{'read' if op == 'r' else 'write'}_b{width * 8} | {_ranges(hits)} | "
                         f"{statistics.median(extra) if extra else 0:.2f} |")
    lines += ["", "## Strided lanes", "", "| pattern | conflict / instr | active / instr | model conflict |",
              "|---|---|---|---|"]
    for name, op, width, addr in pats:
        if name.startswith("stride_"):
            c, a = res[name]
            groups = len({lds_lane_cycle(l, width, op == "w") for l in range(64)})
            lines.append(f"| {name} | {c:.2f} | {a:.2f} | {lds_access_cycles(addr, width, op == 'w') - groups} |")
    lines += ["", "## The SGEMM kernel's tile accesses per layout", "",
              "LDS conflict cycles per K tile of one work-group (every wave's tile writes and operand reads), "
              "measured (sum over the kernel's instructions of the probe's conflict cycles per instruction) and "
              "modelled (`generator.lds_access_cycles`). `chosen` is the generator's layout: pad (floats) and, "
              "for B, the chunk swizzle `(shift, mask)`.", "",
              "| instance | operand | layout | measured | model | conflict-free cycles |", "|---|---|---|---|---|---|"]
    for name in INSTANCES:
        for label, operand, pad, swz, rsw in kernel_layouts(name):
            meas = model = base = 0.0
            for _, _, addrs, width, write, count in kernel_accesses(name, operand, pad, swz, rsw):
                key = _pattern_key(addrs, width, write)
                groups = len({lds_lane_cycle(l, width, write) for l in range(64)})
                meas = meas + count * res[key][0] if key in res and meas is not None else None
                model += count * (lds_access_cycles(addrs, width, write) - groups)
                base += count * groups
            desc = f"pad {pad}" + (f", swizzle {swz}" if swz[1] else "") + (f", row swizzle {rsw}" if rsw[1] else "")
            shown = "n/a (beyond the probe's LDS)" if meas is None else f"{meas:.0f}"
            lines.append(f"| `{name}` | {operand.upper()} | {label}: {desc} | {shown} | {model:.0f} | {base:.0f} |")
    lines += ["", "## The staged epilogue per layout", "",
              "LDS conflict cycles of one work-group's epilogue (every wave's accumulator scatter and float4 "
              "read-back, `generator.lds_epilogue_accesses`), measured and modelled as above.", "",
              "| instance | layout | measured | model | conflict-free cycles |", "|---|---|---|---|---|"]
    for name in INSTANCES:
        for label, pad, swizzle, grouped in EPILOGUE_LAYOUTS:
            meas = model = base = 0.0
            for _, _, addrs, width, write, count in epilogue_accesses(name, pad, swizzle, grouped):
                key = _pattern_key(addrs, width, write)
                groups = len({lds_lane_cycle(l, width, write) for l in range(64)})
                meas = meas + count * res[key][0] if key in res and meas is not None else None
                model += count * (lds_access_cycles(addrs, width, write) - groups)
                base += count * groups
            shown = "n/a (beyond the probe's LDS)" if meas is None else f"{meas:.0f}"
            lines.append(f"| `{name}` | {label} | {shown} | {model:.0f} | {base:.0f} |")
    return "\n".join(lines) + "\n"


def _ranges(xs: List[int]) -> str:
    if not xs:
        return "none"
    out, start, prev = [], xs[0], xs[0]
    for x in xs[1:] + [None]:
        if x is not None and x == prev + 1:
            prev = x
            continue
        out.append(f"{start}" if start == prev else f"{start}-{prev}")
        if x is not None:
            start = prev = x
    return ", ".join(out)


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--out", required=True, help="raw output folder (keep it out of the repository)")
    ap.add_argument("--summary", default=None, help="markdown summary path (default: <out>/lds_banks.md)")
    ap.add_argument("--analyze", action="store_true", help="summarise an earlier run in --out (no GPU work)")
    args = ap.parse_args()
    os.makedirs(args.out, exist_ok=True)
    pat_file = os.path.join(args.out, "patterns.txt")
    pats = write_patterns(pat_file)
    cmd = f"python amdgpu-arch-gemm_amd/profiler/lds_banks.py --out {os.path.relpath(args.out, ROOT)}"
    if not args.analyze:
        run(["timeout", "-s", "KILL", "300", "rocprofv3", "--pmc", "SQ_LDS_BANK_CONFLICT", "SQ_LDS_IDX_ACTIVE",
             "--output-format", "csv", "-d", os.path.join(args.out, "pmc"), "-o", "run", "--",
             PROBE, pat_file, str(ITERS)], 360)
    text = summarise(collect(args.out, pats), pats, cmd)
    path = args.summary or os.path.join(args.out, "lds_banks.md")
    with open(path, "w") as f:
        f.write(text)
    print(text)
    return 0


if __name__ == "__main__":
    sys.exit(main())
