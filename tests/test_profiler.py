"""The profiler's parsing and arithmetic (CPU): every figure in profiles/*.md
and *_traffic.txt comes from profiler/profile_sgemm.py's CSV readers and
derive().  Synthetic rocprofv3 CSVs pin the readers; a constructed dispatch --
a known shader clock, MFMA utilisation, duration and copy-probe ratio, turned
into the counter values the hardware would report -- must come back out of
derive() unchanged."""
import csv
import importlib.util
import os

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
spec = importlib.util.spec_from_file_location(
    "profile_sgemm", os.path.join(ROOT, "amdgpu-arch-gemm_amd", "profiler", "profile_sgemm.py"))
P = importlib.util.module_from_spec(spec)
spec.loader.exec_module(P)

AGENT = (8, 256, 1024, 32, 2400.0)  # XCDs, CUs, SIMDs, shader engines, max engine clock (MHz): MI355X


def _write_csv(path, header, rows):
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(header)
        w.writerows(rows)


def test_counters_per_dispatch_orders_dispatches_and_filters_kernels(tmp_path):
    p = tmp_path / "run_counter_collection.csv"
    hdr = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value", "Start_Timestamp", "End_Timestamp"]
    rows = []
    for d, v in ((10, 7.0), (2, 3.0), (9, 5.0)):  # numeric, not text, order: 2, 9, 10
        rows.append([d, "generated_gemm", "FETCH_SIZE", v, 1000 * d, 1000 * d + 500 + d])
        rows.append([d, "generated_gemm", "WRITE_SIZE", 2 * v, 1000 * d, 1000 * d + 500 + d])
        rows.append([d, "copy_probe", "FETCH_SIZE", 99.0, 0, 1])
    _write_csv(p, hdr, rows)
    per = P.counters_per_dispatch(str(p), "generated_gemm")
    assert per["FETCH_SIZE"] == [3.0, 5.0, 7.0]
    assert per["WRITE_SIZE"] == [6.0, 10.0, 14.0]
    assert per["duration_s"] == pytest.approx([502e-9, 509e-9, 510e-9])
    assert P.counters_per_dispatch(str(p), "copy_probe")["FETCH_SIZE"] == [99.0, 99.0, 99.0]


def test_steady_skips_the_first_dispatch():
    assert P.steady([100.0, 1.0, 2.0, 3.0]) == 2.0
    assert P.steady([100.0, 1.0, 3.0]) == 2.0
    assert P.steady([5.0, 1.0]) == 3.0   # two dispatches: both count
    assert P.steady([4.0]) == 4.0


def test_kernel_stats_and_agent_readers(tmp_path):
    s = tmp_path / "run_kernel_stats.csv"
    _write_csv(s, ["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage", "MinNs", "MaxNs"],
               [["copy_kernel", 3, 30, 10.0, 1, 9, 11], ["generated_gemm", 20, 18000, 900.5, 99, 880, 950]])
    assert P.kernel_stats(str(s), "generated_gemm") == {"calls": 20, "avg_ns": 900.5, "min_ns": 880.0,
                                                        "max_ns": 950.0}
    with pytest.raises(RuntimeError):
        P.kernel_stats(str(s), "absent")
    d = tmp_path / "pmc"
    d.mkdir()
    _write_csv(d / "run_agent_info.csv", ["Agent_Type", "Num_Xcc", "Cu_Count", "Simd_Count", "Array_Count",
                                          "Max_Engine_Clk_Fcompute"],
               [["CPU", 0, 0, 0, 0, 0], ["GPU", 8, 256, 1024, 32, 2400]])
    assert P.gpu_agent(str(d)) == AGENT


def _scenario(m, n, k, clock_mhz, util, pmc_us, trace_us, fetch_bytes, write_bytes, probe_fetch_ratio=0.5):
    """Counter values a dispatch of this shape would report at `clock_mhz`
    with MFMA utilisation `util` over `pmc_us`, HBM traffic fetch/write_bytes
    (FETCH_SIZE reporting `probe_fetch_ratio` of the bytes, WRITE_SIZE all),
    and a first dispatch that differs (it must not enter a median)."""
    xcc, cus, simds, engines, _ = AGENT
    busy_per_engine = clock_mhz * 1e6 * pmc_us * 1e-6
    sq = busy_per_engine * engines
    mfma = util * busy_per_engine * simds

    def later(first, v):  # a first dispatch, then two identical later ones
        return [first, v, v]

    values = {
        "FETCH_SIZE": later(1.0, fetch_bytes * probe_fetch_ratio / 1024.0),
        "WRITE_SIZE": later(1.0, write_bytes / 1024.0),
        "SQ_VALU_MFMA_BUSY_CYCLES": later(1.0, mfma),
        "SQ_BUSY_CYCLES": later(1e9, sq),
        "GRBM_GUI_ACTIVE": later(1.0, 1.1 * clock_mhz * 1e6 * pmc_us * 1e-6 * xcc),
        "duration_s_mfma": later(1.0, pmc_us * 1e-6),
        "SQ_LDS_BANK_CONFLICT": later(0.0, 10.0),
        "SQ_LDS_IDX_ACTIVE": later(0.0, 1010.0),
    }
    probe_kib = P.PROBE_BYTES / 1024.0
    probe = {"FETCH_SIZE": [probe_kib * probe_fetch_ratio] * 3, "WRITE_SIZE": [probe_kib] * 3}
    trace = [2 * trace_us * 1e-6, trace_us * 1e-6, trace_us * 1e-6]
    return P.derive(values, probe, trace, AGENT, m, n, k)


def test_derive_recovers_a_constructed_dispatch():
    m = n = k = 4096
    f = _scenario(m, n, k, clock_mhz=2300.0, util=0.97, pmc_us=950.0, trace_us=905.0,
                  fetch_bytes=538.0e6, write_bytes=67.1e6)
    assert f["clock_mhz"] == pytest.approx(2300.0)
    assert f["mfma_util"] == pytest.approx(97.0)
    assert f["sq_per_engine"] == pytest.approx(2300.0 * 950.0)
    assert f["clock_ok"]
    assert f["fetch_scale"] == pytest.approx(2.0) and f["write_scale"] == pytest.approx(1.0)
    assert f["fetch_bytes"] == pytest.approx(538.0e6) and f["write_bytes"] == pytest.approx(67.1e6)
    assert f["traffic"] == pytest.approx(605.1e6)
    assert f["alg_bytes"] == 4.0 * 3 * 4096 * 4096
    assert f["avg_s"] == pytest.approx(905e-6)
    assert f["tflops"] == pytest.approx(2.0 * 4096 ** 3 / 905e-6 / 1e12)
    assert f["tflops_pmc"] == pytest.approx(2.0 * 4096 ** 3 / 950e-6 / 1e12)
    # 256 CUs x 256 FLOP per clock at 2300 MHz
    assert f["clock_peak"] == pytest.approx(256 * 256 * 2.3e9 / 1e12)
    assert f["busy_us_at_max"] == pytest.approx(2300.0 * 950.0 / 2400.0)
    assert f["gui_window_mhz"] == pytest.approx(1.1 * 2300.0)
    assert f["lds_rate"] == pytest.approx(10.0 / 1000.0)
    # ideal MFMA cycles per SIMD at 64 FLOP per SIMD-cycle
    assert f["ideal_per_simd"] == pytest.approx(2.0 * 4096 ** 3 / 64.0 / 1024)
    # the utilisation bound: MfmaUtil is at least achieved / nominal peak of the same dispatch
    assert f["util_holds"] == (97.0 >= 100.0 * f["tflops_pmc"] / P.PEAK_TFLOPS)


def test_derive_flags_a_clock_above_the_maximum():
    f = _scenario(1024, 1024, 1024, clock_mhz=2900.0, util=0.75, pmc_us=20.0, trace_us=18.0,
                  fetch_bytes=25e6, write_bytes=4.2e6)
    assert f["clock_mhz"] == pytest.approx(2900.0) and not f["clock_ok"]
