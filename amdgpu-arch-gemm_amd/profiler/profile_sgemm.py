"""rocprofv3 measurement of one SGEMM kernel instance on one workload.

    python amdgpu-arch-gemm_amd/profiler/profile_sgemm.py --kernel NAME \
        --workload cfg3 --out prof_out/cfg3 [--summary profiles/NAME_cfg3.md]

This script never touches the GPU itself: every measurement is a child
process -- rocprofv3 wrapping the GeneratorRunner executable (the product's
CLI, validation off) or the copy_probe calibration kernel -- each under its own
time limit.  Passes, one rocprofv3 run each (counters are never mixed with
tracing, and no pass asks for more than the hardware collects at once):

  1. --kernel-trace --stats          kernel durations
  2. --pmc FETCH_SIZE                HBM read KiB per dispatch
  3. --pmc WRITE_SIZE                HBM write KiB per dispatch
  4. --pmc SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE SQ_BUSY_CYCLES
                                     MFMA utilisation and the shader clock
  5. --pmc SQ_LDS_BANK_CONFLICT SQ_LDS_IDX_ACTIVE
  (--issue) --pmc SQ_WAVES SQ_WAVE_CYCLES SQ_WAIT_ANY SQ_WAIT_INST_ANY
     SQ_WAIT_INST_LDS SQ_ACTIVE_INST_ANY SQ_INSTS_LDS SQ_INSTS_SALU
                                     where the waves' cycles go (per wave)
  6./7. FETCH_SIZE and WRITE_SIZE of copy_probe (a plain copy of a known byte
     count), whose ratio to the true bytes scales the SGEMM's counters.

The summary (markdown) lists the commands and the figures; a one-line
``<kernel>_<workload>_traffic.txt`` next to it carries the scaled HBM bytes per
launch that bench.py reports as roofline.traffic.

How the MFMA figures are derived (all per dispatch, medians over the
dispatches after the first):
  * SQ_VALU_MFMA_BUSY_CYCLES summed over the SIMDs is compared with the ideal
    MFMA cycle count, 2MNK / (64 FLOP per SIMD-cycle); a ratio of 1 says every
    MFMA cycle issued is useful work.
  * SQ_BUSY_CYCLES is summed over the shader engines (the agent's Array_Count,
    32 on MI355X): divided by them it is the cycles the kernel kept each
    engine busy.  MfmaUtil = MFMA busy cycles per SIMD / busy cycles per
    engine, both from the same dispatch, so no timestamp enters it.
  * The shader clock is busy cycles per engine over the same PMC dispatch's
    duration (a lower bound if the engines idle inside that window); a clock
    above the agent's maximum engine clock marks the figure invalid.  Counter
    collection serialises dispatches, so a PMC dispatch runs a few
    microseconds longer than the same kernel back to back; the kernel-trace
    pass gives the unperturbed duration and achieved rate, and the busy
    cycles are also shown as time at the maximum clock for comparison.
  * GRBM_GUI_ACTIVE is reported only as the counter window: it covers the
    profiler's own work around a dispatch as well, so for short kernels it
    overstates the kernel's cycles (it read 2.9 GHz over a 20 us dispatch).
"""
from __future__ import annotations

import argparse
import csv
import glob
import os
import shlex
import statistics
import subprocess
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
ROOT = os.path.dirname(PKG)
sys.path.insert(0, PKG)

from generator import catalog  # noqa: E402

RUNNER = os.path.join(PKG, "runner", "GeneratorRunner")
PROBE = os.path.join(HERE, "copy_probe")
SIMD_PER_CU = 4
PEAK_TFLOPS = 157.3
HBM_PEAK_GBS = 8000.0
PROBE_BYTES = 1 << 30

WORKLOADS = {
    "cfg2": (1024, 1024, 1024, 1, 0),
    "cfg3": (4096, 4096, 4096, 2, 0),
    "cfg4": (8192, 8192, 256, 3, 1),
    "cfg5": (16384, 128, 4096, 4, 0),
    "deepk": (512, 512, 16384, 5, 0),   # few tiles, deep K: the split-K kernel
}
# runner warm-up launches per workload: about 0.1 s of each, long enough for
# the engine clock to leave its idle state (5 launches of a 20 us kernel are not)
WARMUP = {"cfg2": 4000, "cfg3": 120, "cfg4": 400, "cfg5": 800, "deepk": 1200}


def log(msg):
    print(msg, flush=True)


def run(cmd, timeout):
    log("+ " + " ".join(shlex.quote(c) for c in cmd))
    t0 = time.time()
    ret = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, timeout=timeout)
    out = ret.stdout.decode(errors="replace")
    log(f"  rc={ret.returncode} in {time.time() - t0:.1f} s")
    if ret.returncode != 0:
        log(out[-3000:])
        raise RuntimeError(f"command failed with rc={ret.returncode}: {cmd[0]}")
    return out


def find(out_dir, pattern):
    hits = sorted(glob.glob(os.path.join(out_dir, "**", pattern), recursive=True))
    if not hits:
        raise RuntimeError(f"no {pattern} under {out_dir}")
    return hits[-1]


def counters_per_dispatch(csv_path, kernel_substr):
    """{counter: [value per dispatch]} for dispatches whose kernel name matches,
    plus "duration_s": the dispatch's own start/end timestamps."""
    per = {}
    with open(csv_path) as f:
        for row in csv.DictReader(f):
            if kernel_substr not in row.get("Kernel_Name", ""):
                continue
            d = row["Dispatch_Id"]
            per.setdefault(row["Counter_Name"], {})[d] = float(row["Counter_Value"])
            per.setdefault("duration_s", {})[d] = (int(row["End_Timestamp"]) - int(row["Start_Timestamp"])) * 1e-9
    return {k: [v[d] for d in sorted(v, key=int)] for k, v in per.items()}


def steady(values):
    """Median over the dispatches after the first (clocks ramp up on the first)."""
    return statistics.median(values[1:] if len(values) > 2 else values)


def trace_durations(out_dir, kernel_substr):
    """Per-dispatch durations (s) of the kernel from --kernel-trace, in dispatch order."""
    rows = []
    with open(find(out_dir, "run_kernel_trace.csv")) as f:
        for row in csv.DictReader(f):
            if kernel_substr in row["Kernel_Name"]:
                rows.append((int(row["Start_Timestamp"]), (int(row["End_Timestamp"]) - int(row["Start_Timestamp"])) * 1e-9))
    return [d for _, d in sorted(rows)]


def kernel_stats(csv_path, kernel_substr):
    with open(csv_path) as f:
        for row in csv.DictReader(f):
            if kernel_substr in row["Name"]:
                return {"calls": int(row["Calls"]), "avg_ns": float(row["AverageNs"]),
                        "min_ns": float(row["MinNs"]), "max_ns": float(row["MaxNs"])}
    raise RuntimeError(f"{kernel_substr} not in {csv_path}")


def gpu_agent(out_dir):
    """(XCD count, CU count, SIMD count, shader engine count, max engine clock MHz)
    of the GPU agent from rocprofv3's agent info."""
    with open(find(out_dir, "run_agent_info.csv")) as f:
        for row in csv.DictReader(f):
            if row.get("Agent_Type") == "GPU":
                return (int(row["Num_Xcc"]), int(row["Cu_Count"]), int(row["Simd_Count"]), int(row["Array_Count"]),
                        float(row["Max_Engine_Clk_Fcompute"]))
    raise RuntimeError(f"no GPU agent in {out_dir}")


def derive(values, probe_vals, trace_durs, agent, m, n, k):
    """The summary's figures from the measurements, no I/O: ``values`` maps
    each counter (and ``duration_s_<pass>``) to its per-dispatch list,
    ``probe_vals`` copy_probe's FETCH_SIZE / WRITE_SIZE lists (KiB per
    dispatch of a PROBE_BYTES copy), ``trace_durs`` the kernel-trace durations
    (s) and ``agent`` what gpu_agent returns.  Medians skip the first
    dispatch (steady)."""
    xcc, cus, simds, engines, max_mhz = agent
    f = {"med": {c: steady(v) for c, v in values.items()}}
    med = f["med"]
    probe_kib = PROBE_BYTES / 1024.0
    f["fetch_scale"] = probe_kib / statistics.median(probe_vals["FETCH_SIZE"])
    f["write_scale"] = probe_kib / statistics.median(probe_vals["WRITE_SIZE"])
    f["fetch_bytes"] = med["FETCH_SIZE"] * 1024.0 * f["fetch_scale"]
    f["write_bytes"] = med["WRITE_SIZE"] * 1024.0 * f["write_scale"]
    f["traffic"] = f["fetch_bytes"] + f["write_bytes"]
    f["avg_s"] = steady(trace_durs)
    f["flops"] = 2.0 * m * n * k
    f["alg_bytes"] = 4.0 * (m * k + k * n + m * n)
    f["tflops"] = f["flops"] / f["avg_s"] / 1e12
    # MFMA cycles per SIMD: measured, and the ideal at 64 FLOP per SIMD-cycle
    f["ideal_per_simd"] = f["flops"] / 64.0 / simds
    f["busy_per_simd"] = med["SQ_VALU_MFMA_BUSY_CYCLES"] / simds
    # per dispatch of the PMC pass: shader-busy cycles per engine, MfmaUtil and
    # the clock over that dispatch's own duration
    disp = list(zip(values["SQ_VALU_MFMA_BUSY_CYCLES"], values["SQ_BUSY_CYCLES"], values["GRBM_GUI_ACTIVE"],
                    values["duration_s_mfma"]))
    f["sq_per_engine"] = steady([q / engines for _, q, _, _ in disp])
    f["mfma_util"] = 100.0 * steady([(b / simds) / (q / engines) for b, q, _, _ in disp])
    f["clock_mhz"] = steady([q / engines / dur / 1e6 for _, q, _, dur in disp])
    f["pmc_dur"] = steady([dur for _, _, _, dur in disp])
    f["gui_window_mhz"] = steady([a / xcc / dur / 1e6 for _, _, a, dur in disp])
    f["clock_ok"] = f["clock_mhz"] <= max_mhz
    f["tflops_pmc"] = f["flops"] / f["pmc_dur"] / 1e12
    f["clock_peak"] = cus * 256 * f["clock_mhz"] * 1e6 / 1e12
    f["busy_us_at_max"] = f["sq_per_engine"] / max_mhz  # the engine-busy cycles at the maximum clock, in us
    f["lds_rate"] = med["SQ_LDS_BANK_CONFLICT"] / max(med["SQ_LDS_IDX_ACTIVE"] - med["SQ_LDS_BANK_CONFLICT"], 1.0)
    f["util_holds"] = f["mfma_util"] >= 100.0 * f["tflops_pmc"] / PEAK_TFLOPS - 1e-9
    return f


def rocprof(args, out_dir, program, timeout):
    cmd = ["rocprofv3", *args, "--output-format", "csv", "-d", out_dir, "-o", "run", "--", *program]
    return run(["timeout", "-s", "KILL", str(timeout), *cmd], timeout + 30)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--kernel", required=True)
    ap.add_argument("--workload", default="cfg3", choices=sorted(WORKLOADS))
    ap.add_argument("--out", required=True, help="raw rocprofv3 output folder (large; keep it out of the repository)")
    ap.add_argument("--summary", default=None, help="markdown summary path (default: <out>/summary.md)")
    ap.add_argument("--runs", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=None,
                    help="untimed runner launches first (default: about 0.1 s of the workload, so the "
                         "engine clock has ramped up before the dispatches the medians describe)")
    ap.add_argument("--cus", type=int, default=256)
    ap.add_argument("--issue", action="store_true",
                    help="one more pass: wave cycles, waits and LDS / scalar instructions per wave")
    ap.add_argument("--analyze-only", action="store_true",
                    help="derive the summary from the rocprofv3 output already in --out (no GPU work)")
    args = ap.parse_args()

    m, n, k, seed, dist = WORKLOADS[args.workload]
    co, toml = catalog.paths(args.kernel)
    os.makedirs(args.out, exist_ok=True)
    warmup = args.warmup if args.warmup is not None else WARMUP[args.workload]
    runner = [RUNNER, co, toml, str(m), str(n), str(k), str(warmup), str(args.runs), "0", str(seed), str(dist), "1", "0"]
    probe = [PROBE, str(PROBE_BYTES), "3"]
    cmds = {}

    def profile(pass_args, out_dir, program, timeout):
        if not args.analyze_only:
            rocprof(pass_args, out_dir, program, timeout)

    d = os.path.join(args.out, "trace")
    profile(["--kernel-trace", "--stats"], d, runner, 300)
    cmds["trace"] = "rocprofv3 --kernel-trace --stats --output-format csv -d <out>/trace -o run -- " + " ".join(
        os.path.relpath(c, ROOT) if os.path.isabs(c) else c for c in runner)
    ks = kernel_stats(find(d, "run_kernel_stats.csv"), "generated_gemm")

    passes = {
        "fetch": ["FETCH_SIZE"],
        "write": ["WRITE_SIZE"],
        "mfma": ["SQ_VALU_MFMA_BUSY_CYCLES", "GRBM_GUI_ACTIVE", "SQ_BUSY_CYCLES"],
        "lds": ["SQ_LDS_BANK_CONFLICT", "SQ_LDS_IDX_ACTIVE"],
    }
    if args.issue:
        passes["issue"] = ["SQ_WAVES", "SQ_WAVE_CYCLES", "SQ_WAIT_ANY", "SQ_WAIT_INST_ANY", "SQ_WAIT_INST_LDS",
                           "SQ_ACTIVE_INST_ANY", "SQ_INSTS_LDS", "SQ_INSTS_SALU"]
    values = {}
    for key, counters in passes.items():
        d = os.path.join(args.out, f"pmc_{key}")
        profile(["--pmc", *counters], d, runner, 120)
        cmds[key] = f"rocprofv3 --pmc {' '.join(counters)} --output-format csv -d <out>/pmc_{key} -o run -- <runner>"
        per = counters_per_dispatch(find(d, "run_counter_collection.csv"), "generated_gemm")
        for c in counters:
            if c not in per:
                raise RuntimeError(f"counter {c} missing from pass {key}")
            values[c] = per[c]
        values[f"duration_s_{key}"] = per["duration_s"]
    probe_vals = {}
    for c in ("FETCH_SIZE", "WRITE_SIZE"):
        d = os.path.join(args.out, f"probe_{c.lower()}")
        profile(["--pmc", c], d, probe, 120)
        per = counters_per_dispatch(find(d, "run_counter_collection.csv"), "copy_probe")
        probe_vals[c] = per[c]

    agent = gpu_agent(os.path.join(args.out, "pmc_mfma"))
    xcc, cus, simds, engines, max_mhz = agent
    fig = derive(values, probe_vals, trace_durations(os.path.join(args.out, "trace"), "generated_gemm"), agent, m, n, k)
    (med, fetch_scale, write_scale, fetch_bytes, write_bytes, traffic, avg_s, alg_bytes, tflops, ideal_per_simd,
     busy_per_simd, sq_per_engine, mfma_util, clock_mhz, pmc_dur, gui_window_mhz, clock_ok, tflops_pmc, clock_peak,
     busy_us_at_max, lds_rate) = (fig[x] for x in (
        "med", "fetch_scale", "write_scale", "fetch_bytes", "write_bytes", "traffic", "avg_s", "alg_bytes", "tflops",
        "ideal_per_simd", "busy_per_simd", "sq_per_engine", "mfma_util", "clock_mhz", "pmc_dur", "gui_window_mhz",
        "clock_ok", "tflops_pmc", "clock_peak", "busy_us_at_max", "lds_rate"))
    valid = "valid" if clock_ok else f"INVALID (above the {max_mhz:.0f} MHz maximum)"
    util_check = "holds" if fig["util_holds"] else "FAILS"

    summary = args.summary or os.path.join(args.out, "summary.md")
    os.makedirs(os.path.dirname(os.path.abspath(summary)), exist_ok=True)
    lines = [
        f"# rocprofv3: `{args.kernel}` on {args.workload} ({m}x{n}x{k}, seed {seed}, "
        f"{'N(0,1)' if dist else 'U[-1,1)'}, alpha=1, beta=0)",
        "",
        "Command (from the repository root on the GPU box):",
        "",
        f"    python amdgpu-arch-gemm_amd/profiler/profile_sgemm.py --kernel {args.kernel} "
        f"--workload {args.workload}{' --issue' if args.issue else ''} --out {args.out} "
        f"--summary {os.path.relpath(summary, ROOT)}",
        "",
        "which runs, each in its own process (`<runner>` = `"
        + " ".join(os.path.relpath(c, ROOT) if os.path.isabs(c) else c for c in runner) + "`):",
        "",
        f"    {cmds['trace']}",
        *[f"    {cmds[k2]}" for k2 in passes],
        f"    rocprofv3 --pmc FETCH_SIZE|WRITE_SIZE ... -- amdgpu-arch-gemm_amd/profiler/copy_probe {PROBE_BYTES} 3",
        "",
        "| figure | value |",
        "|---|---|",
        f"| kernel-trace calls / mean / min / max | {ks['calls']} / {ks['avg_ns'] / 1e3:.2f} us / "
        f"{ks['min_ns'] / 1e3:.2f} us / {ks['max_ns'] / 1e3:.2f} us |",
        f"| kernel-trace duration, median after the first dispatch | {avg_s * 1e6:.2f} us |",
        f"| achieved (median duration) | {tflops:.2f} TFLOP/s = {100 * tflops / PEAK_TFLOPS:.1f}% of {PEAK_TFLOPS} (nominal) |",
        f"| MFMA busy cycles per SIMD (SQ_VALU_MFMA_BUSY_CYCLES / {simds}) vs the ideal 2MNK / 64 / {simds} | "
        f"{busy_per_simd:.6g} / {ideal_per_simd:.6g} = {busy_per_simd / ideal_per_simd:.4f} |",
        f"| shader-busy cycles per engine (SQ_BUSY_CYCLES / {engines}) | {sq_per_engine:.6g} |",
        f"| PMC-pass dispatch duration, median (counter collection serialises dispatches) | {pmc_dur * 1e6:.2f} us "
        f"= {tflops_pmc:.2f} TFLOP/s |",
        f"| MfmaUtil = MFMA busy per SIMD / shader-busy per engine (same dispatch) | {mfma_util:.1f}% "
        f"(>= achieved / peak of that dispatch, {100 * tflops_pmc / PEAK_TFLOPS:.1f}%: {util_check}) |",
        f"| shader clock = busy cycles per engine / the same dispatch's duration | {clock_mhz:.0f} MHz, {valid} -> "
        f"clock-adjusted peak {clock_peak:.1f} TFLOP/s; that dispatch reached {100 * tflops_pmc / clock_peak:.1f}% of it |",
        f"| busy cycles per engine at the {max_mhz:.0f} MHz maximum | {busy_us_at_max:.2f} us (kernel-trace median "
        f"{avg_s * 1e6:.2f} us) |",
        f"| GRBM_GUI_ACTIVE / {xcc} XCDs over the PMC dispatch (counter window, not the kernel's cycles) | "
        f"{gui_window_mhz:.0f} MHz equivalent |",
        f"| LDS bank conflicts / conflict-free accesses (SQ_LDS_BANK_CONFLICT, SQ_LDS_IDX_ACTIVE) | "
        f"{lds_rate:.4f} ({med['SQ_LDS_BANK_CONFLICT']:.4g} / {med['SQ_LDS_IDX_ACTIVE']:.4g}) |",
        f"| FETCH_SIZE / WRITE_SIZE raw (KiB per dispatch, median) | {med['FETCH_SIZE']:.1f} / {med['WRITE_SIZE']:.1f} |",
        f"| copy_probe calibration ({PROBE_BYTES} B read + written) | FETCH_SIZE {statistics.median(probe_vals['FETCH_SIZE']):.1f} KiB "
        f"(scale {fetch_scale:.4f}), WRITE_SIZE {statistics.median(probe_vals['WRITE_SIZE']):.1f} KiB (scale {write_scale:.4f}) |",
        f"| HBM traffic per launch (scaled) | read {fetch_bytes / 1e6:.1f} MB + write {write_bytes / 1e6:.1f} MB = "
        f"{traffic / 1e6:.1f} MB ({traffic / alg_bytes:.2f}x the {alg_bytes / 1e6:.1f} MB algorithmic) |",
        f"| HBM bandwidth | {traffic / avg_s / 1e9:.1f} GB/s measured, {alg_bytes / avg_s / 1e9:.1f} GB/s algorithmic "
        f"(peak {HBM_PEAK_GBS:.0f}) |",
    ]
    if args.issue:
        # per wave, in cycles (the SQ_WAVE_CYCLES / WAIT / ACTIVE counters count quad-cycles)
        waves = max(med["SQ_WAVES"], 1.0)
        wc = 4.0 * med["SQ_WAVE_CYCLES"] / waves
        lines += [
            f"| waves per dispatch / wave cycles per wave (SQ_WAVES, 4 x SQ_WAVE_CYCLES) | {waves:.0f} / {wc:.0f} |",
            f"| per wave: waiting for anything / for instruction issue / for LDS issue (4 x SQ_WAIT_ANY, "
            f"_INST_ANY, _INST_LDS) | {4.0 * med['SQ_WAIT_ANY'] / waves:.0f} / "
            f"{4.0 * med['SQ_WAIT_INST_ANY'] / waves:.0f} / {4.0 * med['SQ_WAIT_INST_LDS'] / waves:.0f} cycles |",
            f"| per wave: cycles working on any instruction (4 x SQ_ACTIVE_INST_ANY) | "
            f"{4.0 * med['SQ_ACTIVE_INST_ANY'] / waves:.0f} |",
            f"| per wave: LDS / scalar ALU instructions issued (SQ_INSTS_LDS, SQ_INSTS_SALU) | "
            f"{med['SQ_INSTS_LDS'] / waves:.0f} / {med['SQ_INSTS_SALU'] / waves:.0f} |",
        ]
    lines.append("")
    with open(summary, "w") as f:
        f.write("\n".join(lines))
    traffic_path = os.path.join(os.path.dirname(os.path.abspath(summary)), f"{args.kernel}_{args.workload}_traffic.txt")
    with open(traffic_path, "w") as f:
        f.write(f"# from {os.path.relpath(summary, ROOT)}\n")
        f.write(f"hbm_bytes_per_launch: {traffic:.0f}\n")
        f.write(f"fetch_bytes_per_launch: {fetch_bytes:.0f}\n")
        f.write(f"write_bytes_per_launch: {write_bytes:.0f}\n")
        f.write(f"mfma_util_pct: {mfma_util:.2f}\n")
        f.write(f"shader_clock_mhz: {clock_mhz:.0f}\n")
        f.write(f"clock_valid: {int(clock_ok)}\n")
    log("\n".join(lines))


if __name__ == "__main__":
    main()
