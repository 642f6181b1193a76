"""The gfx950 tuner end to end on the GPU (reference tuner/sgemm_tuner.py:41-128).

A small sweep (a few stage-1 geometries at 512 x 512 x 256) runs through the
tuner's command line exactly as a user would run it; the emitted
generated_gemm.co + .toml must then validate in this build's runner, in the
reference's own runner when it was built, and against the oracle through the
C-ABI shim.  The candidates were compiled by __graft_entry__.build() into the
package's kernels/ folder, so the sweep only times them (a point whose source
changed since is rebuilt by the tuner itself).
"""
import json
import os
import subprocess
import sys

import numpy as np
import pytest

import __graft_entry__ as graft
import oracle
from shim import sgemm_shim as S

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "amdgpu-arch-gemm_amd")
RUNNER = os.path.join(PKG, "runner", "GeneratorRunner")
TUNER = os.path.join(PKG, "tuner", "sgemm_tuner.py")


def _say(msg):
    print(msg, flush=True)


def test_small_sweep_emits_a_validated_drop_in_pair(kernels, tmp_path):
    out = str(tmp_path / "tune")
    c = graft.TUNER_CHECK
    cmd = [sys.executable, TUNER, "--m", str(c["m"]), "--n", str(c["n"]), "--k", str(c["k"]), "--bench", RUNNER,
           "--output-folder", out, "--points-dir", graft.TUNER_CHECK_POINTS, "--in-process", "--refine", "0",
           "--tiles", c["tiles"], "--occ", c["occ"], "--stage1-depths", c["depths"], "--warmup", "3", "--runs", "10",
           "--jobs", "16", "--timeout", "60"]
    _say("+ " + " ".join(cmd))
    ret = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, timeout=600)
    log = ret.stdout.decode(errors="replace")
    _say(log[-3000:])
    assert ret.returncode == 0, log
    recs = [json.loads(x) for x in open(os.path.join(out, "results.jsonl")).read().splitlines()]
    ok = [r for r in recs if r["status"] == "ok"]
    assert len(recs) >= 4 and len(ok) >= 4, [(r["point"], r["status"]) for r in recs]
    assert all(r["gflops"] > 1000.0 for r in ok)                 # every timed point ran on the GPU
    best = max(ok, key=lambda r: r["gflops"])
    assert f"validation of {best['point']}: PASS" in log          # the winner was checked before emission
    assert "Best: " in log
    co, toml = os.path.join(out, "generated_gemm.co"), os.path.join(out, "generated_gemm.toml")
    assert open(co, "rb").read() == open(os.path.join(graft.TUNER_CHECK_POINTS, best["point"] + ".co"), "rb").read()

    # the emitted pair in this build's runner, on a shape the reference tuner would skip
    r = subprocess.run([RUNNER, co, toml, "700", "333", "515", "1", "2", "1", "3"], stdout=subprocess.PIPE,
                       stderr=subprocess.STDOUT, timeout=300)
    out_runner = r.stdout.decode()
    _say(out_runner)
    assert r.returncode == 0 and "validation: PASS" in out_runner and "# of mismatches: 0/" in out_runner

    # against the oracle through the shim at the tuned shape
    m, n, k = c["m"], c["n"], c["k"]
    A, B, C = S.fill_matrix(m, k, 9, 0), S.fill_matrix(k, n, 9, 1), S.fill_matrix(m, n, 9, 2)
    with S.Kernel(co, toml) as kern:
        D, _ = kern.run(A, B, C, m, n, k, alpha=1.5, beta=-0.5)
    err = oracle.normwise_error(D, oracle.cpu_gemm(A, B, C, 1.5, -0.5))
    assert err <= oracle.tolerance(k), err

    # and in the reference's own runner, built unmodified from its source
    if os.path.exists(oracle.REF_RUNNER_PATH):
        r = subprocess.run([oracle.REF_RUNNER_PATH, co, toml, "512", "512", "256", "1", "2", "1"],
                           stdout=subprocess.PIPE, stderr=subprocess.STDOUT, timeout=300)
        out_ref = r.stdout.decode()
        _say(out_ref[-600:])
        assert r.returncode == 0 and "# of mismatches: 0/" in out_ref

    # resume: a second run times nothing again and emits the same winner
    ret2 = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, timeout=600)
    log2 = ret2.stdout.decode(errors="replace")
    assert ret2.returncode == 0, log2
    assert "Gflops: " not in "\n".join(ln for ln in log2.splitlines() if not ln.startswith(("Best", "validation")))
    assert len(open(os.path.join(out, "results.jsonl")).read().splitlines()) == len(recs)


def test_playoff_emits_the_best_interleaved_median(kernels, tmp_path):
    """--playoff: the three fastest points are timed again, round-robin in
    alternating order, and the emitted pair is the best median among them."""
    out = str(tmp_path / "tune_po")
    c = graft.TUNER_CHECK
    summary = str(tmp_path / "summary.md")
    cmd = [sys.executable, TUNER, "--m", str(c["m"]), "--n", str(c["n"]), "--k", str(c["k"]), "--bench", RUNNER,
           "--output-folder", out, "--points-dir", graft.TUNER_CHECK_POINTS, "--in-process", "--refine", "0",
           "--tiles", c["tiles"], "--occ", c["occ"], "--stage1-depths", c["depths"], "--warmup", "3", "--runs", "10",
           "--jobs", "16", "--timeout", "60", "--playoff", "3", "--playoff-rounds", "4", "--summary", summary]
    _say("+ " + " ".join(cmd))
    ret = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, timeout=600)
    log = ret.stdout.decode(errors="replace")
    _say(log[-3000:])
    assert ret.returncode == 0, log
    medians = {}
    for line in log.splitlines():
        if line.startswith("playoff: ") and "Gflops median of 4" in line:
            medians[line.rsplit(", ", 1)[1]] = float(line.split()[1])
    assert len(medians) == 3 and all(v > 1000.0 for v in medians.values()), medians
    best = max(medians, key=medians.get)
    assert f"validation of {best}: PASS" in log
    co = os.path.join(out, "generated_gemm.co")
    assert open(co, "rb").read() == open(os.path.join(graft.TUNER_CHECK_POINTS, best + ".co"), "rb").read()
    text = open(summary).read()
    assert "Playoff (4 interleaved rounds" in text and f"`{best}`" in text and "(playoff median)" in text


def test_transposed_sweep_emits_a_validated_tt_pair(kernels, tmp_path):
    """The same sweep for op(A) = A^T, op(B) = B^T (--trans-a --trans-b): the
    emitted pair is a TT kernel, and it validates in this build's runner and
    against the oracle on transposed storage (the reference's runner ignores
    the layout fields, so it is not asked)."""
    out = str(tmp_path / "tune_tt")
    c = graft.TUNER_CHECK
    cmd = [sys.executable, TUNER, "--m", str(c["m"]), "--n", str(c["n"]), "--k", str(c["k"]), "--bench", RUNNER,
           "--output-folder", out, "--points-dir", graft.TUNER_CHECK_POINTS, "--in-process", "--refine", "0",
           "--tiles", c["tiles"], "--occ", c["occ"], "--stage1-depths", c["depths"], "--warmup", "3", "--runs", "10",
           "--jobs", "16", "--timeout", "60", "--trans-a", "--trans-b"]
    _say("+ " + " ".join(cmd))
    ret = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, timeout=600)
    log = ret.stdout.decode(errors="replace")
    _say(log[-2000:])
    assert ret.returncode == 0, log
    recs = [json.loads(x) for x in open(os.path.join(out, "results.jsonl")).read().splitlines()]
    ok = [r for r in recs if r["status"] == "ok"]
    assert len(ok) >= 4 and all(r["trans_a"] and r["trans_b"] and r["point"].endswith("_tt") for r in ok)
    assert "compile" not in " ".join(r["status"] for r in recs)    # every point came prebuilt
    best = max(ok, key=lambda r: r["gflops"])
    assert f"validation of {best['point']}: PASS" in log
    co, toml = os.path.join(out, "generated_gemm.co"), os.path.join(out, "generated_gemm.toml")
    with S.Kernel(co, toml) as kern:
        assert kern.info.trans_a and kern.info.trans_b
    r = subprocess.run([RUNNER, co, toml, "700", "333", "515", "1", "2", "1", "3"], stdout=subprocess.PIPE,
                       stderr=subprocess.STDOUT, timeout=300)
    out_runner = r.stdout.decode()
    _say(out_runner[-600:])
    assert r.returncode == 0 and "validation: PASS" in out_runner and "# of mismatches: 0/" in out_runner
    m, n, k = c["m"], c["n"], c["k"]
    A, B, C = S.fill_matrix(k, m, 9, 0), S.fill_matrix(n, k, 9, 1), S.fill_matrix(m, n, 9, 2)
    with S.Kernel(co, toml) as kern:
        D, _ = kern.run(A, B, C, m, n, k, alpha=1.5, beta=-0.5)
    ref = oracle.cpu_gemm(np.asfortranarray(A.T), np.asfortranarray(B.T), C, 1.5, -0.5)
    assert oracle.normwise_error(D, ref) <= oracle.tolerance(k)
