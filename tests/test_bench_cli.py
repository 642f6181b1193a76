"""bench.py's command line and its one-line JSON contract.

The CPU tests stop before any GPU call (a second GPU is refused up front,
an unknown layout by argparse); the GPU test runs a short cfg2 bench in each
layout and checks the fields the harness reads."""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "bench.py")


def _bench(*args, timeout=600):
    return subprocess.run([sys.executable, BENCH, *args], stdout=subprocess.PIPE, stderr=subprocess.PIPE,
                          timeout=timeout, cwd=ROOT)


def test_more_than_one_gpu_is_refused_with_a_message():
    r = _bench("--gpus", "2", "--steps", "1", "--warmup", "0", timeout=300)
    assert r.returncode == 2
    assert b"one GPU" in r.stderr or b"single MI355X" in r.stderr
    assert r.stdout == b""


def test_unknown_layout_is_an_argument_error():
    r = _bench("--layout", "xy", timeout=300)
    assert r.returncode == 2 and b"--layout" in r.stderr


@pytest.mark.gpu
@pytest.mark.parametrize("layout", ["nn", "tn", "nt", "tt"])
def test_short_bench_prints_the_contract_line(kernels, layout):
    r = _bench("--workload", "cfg2", "--layout", layout, "--steps", "5", "--warmup", "2", "--cpu-seconds", "0.5")
    print(r.stderr.decode()[-1500:], flush=True)
    assert r.returncode == 0
    lines = [ln for ln in r.stdout.decode().splitlines() if ln.strip()]
    assert len(lines) == 1, lines
    d = json.loads(lines[0])
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
                "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert key in d, key
    assert d["n_gpus"] == 1 and d["steps"] == 5 and d["warmup"] == 2 and d["unit"] == "TFLOP/s"
    assert d["dtype"] == "f32" and d["data"] == "synthetic" and d["higher_is_better"] is True
    assert d["value"] > 10.0 and abs(d["value"] - 2.0 * 1024 ** 3 / (d["ms_per_step"] * 1e-3) / 1e12) < 0.05 * d["value"]
    cfg = d["config"]
    assert cfg["workload"] == f"sgemm_{layout}_colmajor_1024x1024x1024"
    assert cfg["kernel"].endswith("" if layout == "nn" else "_" + layout)
    assert layout.upper() in d["metric"]
    roof = d["roofline"]
    assert roof["bound"] == "mfma" and roof["peak"] == 157.3 and 0.0 < roof["frac"] < 1.0
    assert abs(roof["frac"] - roof["achieved"] / roof["peak"]) < 1e-3
    cpu = d["cpu_baseline"]
    assert cpu["kind"] in ("reference", "port") and cpu["cores"] == 1 and cpu["value"] > 0.0
    assert d["parity"]["pass"] is True
