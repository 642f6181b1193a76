"""Host code under AddressSanitizer + UndefinedBehaviorSanitizer (CPU only).

`make -C amdgpu-arch-gemm_amd asan` builds the runner and the library's host
C++ with -fsanitize=address,undefined (no device code carries a sanitizer),
plus tests/asan/shim_host_check.cpp, which compiles the library's host C++
into itself.  These tests feed them what the reference's config boundary
(toml++ in /root/reference/runner/generator_runner.cpp:85-124) and CLI
(:192-223) would see at their worst: malformed and hostile .toml files,
extreme shapes through the shape check and the launch plan, aliasing
buffers, edge handles closed in every order, and bad command lines.  The
runner's multithreaded CPU validation GEMMs (runner/cpu_reference.hpp) run
under ASan + UBSan and under ThreadSanitizer from
tests/asan/cpu_reference_check.cpp.  Any sanitizer report fails the test; so
does a wrong return code.
"""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "amdgpu-arch-gemm_amd")
ASAN_DIR = os.path.join(PKG, "_asan")
CHECK = os.path.join(ASAN_DIR, "shim_host_check")
RUNNER = os.path.join(ASAN_DIR, "GeneratorRunner")
KERNELS = os.path.join(PKG, "kernels")

SGEMM_E_IO, SGEMM_E_CONFIG = -2, -3

ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:exitcode=99", UBSAN_OPTIONS="print_stacktrace=1:exitcode=98",
           TSAN_OPTIONS="halt_on_error=1:exitcode=97", HIP_VISIBLE_DEVICES="")
CPU_REF_CHECK = os.path.join(ROOT, "tests", "asan", "cpu_reference_check.cpp")

VALID = """a_type = 0
b_type = 0
cd_type = 0
scalar_type = 0
depth_k = 16
vmem_stage = 2
wavefront_size = 64
lds_usage_bytes = 53248
wave_group = [2, 2]
mfma = [32, 32, 1, 2]
wave_tiling = [4, 2]
trans_a = false
trans_b = false
name = "generated_gemm"
"""


def _with(key, value):
    """VALID with `key`'s line replaced (value None: line removed)."""
    out = []
    for line in VALID.splitlines():
        if line.split("=")[0].strip() == key:
            if value is not None:
                out.append(f"{key} = {value}")
        else:
            out.append(line)
    return "\n".join(out) + "\n"


# (label, file bytes, expected return code of sgemm_open with a missing .co):
# SGEMM_E_IO means the config was accepted and the missing code object was next
TOML_CASES = [
    ("valid", VALID, SGEMM_E_IO),
    ("valid_crlf", VALID.replace("\n", "\r\n"), SGEMM_E_IO),
    ("valid_comments", "# generated\n" + VALID.replace("\n", "  # trailing\n"), SGEMM_E_IO),
    ("hash_in_string", _with("name", '"gen#erated"'), SGEMM_E_IO),
    ("duplicate_key_last_wins", VALID + "depth_k = 32\n", SGEMM_E_IO),
    ("empty_items_skipped", _with("mfma", "[32,,32, 1,2,]"), SGEMM_E_IO),
    ("extra_float_key", VALID + "alpha = 1.5\n", SGEMM_E_IO),
    ("empty_file", "", SGEMM_E_CONFIG),
    ("only_comments", "# nothing\n\n   \n", SGEMM_E_CONFIG),
    ("missing_mfma", _with("mfma", None), SGEMM_E_CONFIG),
    ("missing_trans_b", _with("trans_b", None), SGEMM_E_CONFIG),
    ("table", "[kernel]\n" + VALID, SGEMM_E_CONFIG),
    ("no_equals", VALID + "depth_k 16\n", SGEMM_E_CONFIG),
    ("unterminated_string", _with("name", '"generated_gemm'), SGEMM_E_CONFIG),
    ("lone_quote", _with("name", '"'), SGEMM_E_CONFIG),
    ("unterminated_array", _with("mfma", "[32, 32, 1, 2"), SGEMM_E_CONFIG),
    ("array_of_words", _with("mfma", "[a, b, c, d]"), SGEMM_E_CONFIG),
    ("array_of_floats", _with("wave_group", "[2.0, 2.0]"), SGEMM_E_CONFIG),
    ("short_array", _with("wave_tiling", "[4]"), SGEMM_E_CONFIG),
    ("empty_array", _with("wave_group", "[]"), SGEMM_E_CONFIG),
    ("scalar_for_array", _with("mfma", "32"), SGEMM_E_CONFIG),
    ("array_for_scalar", _with("depth_k", "[16]"), SGEMM_E_CONFIG),
    ("string_for_bool", _with("trans_a", '"false"'), SGEMM_E_CONFIG),
    ("int_past_int64", _with("depth_k", "99999999999999999999999"), SGEMM_E_CONFIG),
    ("int_past_int32", _with("depth_k", "4294967312"), SGEMM_E_CONFIG),
    ("item_past_int32", _with("wave_tiling", "[4294967300, 2]"), SGEMM_E_CONFIG),
    ("huge_wave_group", _with("wave_group", "[2147483647, 2147483647]"), SGEMM_E_CONFIG),
    ("huge_wave_tiling", _with("wave_tiling", "[100000, 100000]"), SGEMM_E_CONFIG),
    ("negative_depth", _with("depth_k", "-16"), SGEMM_E_CONFIG),
    ("zero_depth", _with("depth_k", "0"), SGEMM_E_CONFIG),
    ("negative_wave_group", _with("wave_group", "[-2, 2]"), SGEMM_E_CONFIG),
    ("zero_stage", _with("vmem_stage", "0"), SGEMM_E_CONFIG),
    ("negative_lds", _with("lds_usage_bytes", "-1"), SGEMM_E_CONFIG),
    ("wave32", _with("wavefront_size", "32"), SGEMM_E_CONFIG),
    ("fp16_type", _with("a_type", "1"), SGEMM_E_CONFIG),
    ("bad_atom", _with("mfma", "[16, 16, 4, 1]"), SGEMM_E_CONFIG),
    ("too_many_waves", _with("wave_group", "[8, 4]"), SGEMM_E_CONFIG),
    ("split_k_out_of_range", VALID + "split_k = 17\n", SGEMM_E_CONFIG),
    ("stream_k_out_of_range", VALID + "stream_k = 3\n", SGEMM_E_CONFIG),
    ("bom", "﻿" + VALID, SGEMM_E_CONFIG),
    ("long_line", VALID + "name = \"" + "x" * (1 << 20) + "\"\n", SGEMM_E_IO),
    ("long_garbage_line", VALID + "=" * (1 << 20) + "\n", SGEMM_E_CONFIG),
]


@pytest.fixture(scope="module")
def asan_build():
    ret = subprocess.run(["make", "-s", "-C", PKG, "asan"], stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    assert ret.returncode == 0, ret.stdout.decode()[-3000:]
    return True


def _clean(out: str):
    assert "Sanitizer" not in out and "runtime error" not in out, out[-4000:]


def _run(cmd, **kw):
    ret = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, env=ENV, timeout=120, **kw)
    out = ret.stdout.decode(errors="replace")
    _clean(out)
    return ret.returncode, out


def test_toml_reader_under_sanitizers(asan_build, tmp_path):
    paths = []
    for label, text, _ in TOML_CASES:
        p = tmp_path / f"{label}.toml"
        p.write_bytes(text.encode("utf-8"))
        paths.append(str(p))
    # binary garbage: NUL bytes, invalid UTF-8, a truncated multi-byte sequence
    garbage = tmp_path / "garbage.toml"
    garbage.write_bytes(bytes(range(256)) * 64 + b"\xe2\x82")
    paths.append(str(garbage))
    nul = tmp_path / "nul_in_key.toml"
    nul.write_bytes(VALID.replace("depth_k", "depth\x00_k").encode())
    paths.append(str(nul))
    rc, out = _run([CHECK, "toml"] + paths)
    assert rc == 0, out
    lines = out.splitlines()
    assert len(lines) == len(paths), out
    expected = [e for _, _, e in TOML_CASES] + [SGEMM_E_CONFIG, SGEMM_E_CONFIG]
    labels = [c[0] for c in TOML_CASES] + ["garbage", "nul_in_key"]
    for label, want, line in zip(labels, expected, lines):
        got = int(line.split()[0])
        assert got == want, f"{label}: {line}"
        if want == SGEMM_E_IO:
            assert "cannot open code object" in line, f"{label}: {line}"


def test_every_committed_kernel_config_parses(asan_build):
    """Every .toml the generator wrote for the catalog passes the reader."""
    tomls = sorted(os.path.join(KERNELS, f) for f in os.listdir(KERNELS) if f.endswith(".toml")) \
        if os.path.isdir(KERNELS) else []
    if not tomls:
        pytest.skip("no generated kernels (run __graft_entry__.build())")
    rc, out = _run([CHECK, "toml"] + tomls)
    assert rc == 0, out
    assert all(line.startswith(f"{SGEMM_E_IO} cannot open code object") for line in out.splitlines()), out


@pytest.mark.parametrize("mode", ["shapes", "alias", "edges"])
def test_host_helpers_under_sanitizers(asan_build, mode):
    rc, out = _run([CHECK, mode])
    assert rc == 0, out


def test_runner_cli_under_sanitizers(asan_build, tmp_path):
    toml = tmp_path / "k.toml"
    toml.write_text(VALID)
    bad = tmp_path / "bad.toml"
    bad.write_text(_with("mfma", "[32, 32"))
    co = str(tmp_path / "missing.co")
    cases = [
        ([], "usage"),
        (["a", "b", "1", "2", "x", "1", "1", "0"], "usage"),
        (["a", "b", "-1", "2", "3", "1", "1", "0"], "usage"),
        (["a", "b", "99999999999", "2", "3", "1", "1", "0"], "usage"),
        (["a", "b", "", "2", "3", "1", "1", "0"], "usage"),
        (["a", "b", "1", "2", "3", "1", "1", "0", "1", "2x"], "usage"),
        ([co, str(tmp_path / "none.toml"), "64", "64", "64", "1", "1", "1"], "cannot open"),
        ([co, str(bad), "64", "64", "64", "1", "1", "1"], "bad array"),
        ([co, str(toml), "64", "64", "64", "1", "1", "1", "0", "0", "nan", "inf"], "cannot open code object"),
        ([co, str(toml), "4294967295", "4294967295", "4294967295", "0", "0", "1"], "cannot open code object"),
    ]
    for args, needle in cases:
        rc, out = _run([RUNNER] + args)
        assert rc == 255, (args, out)
        assert needle in out, (args, out)


@pytest.mark.parametrize("sanitizer", ["address,undefined", "thread"])
def test_runner_cpu_reference_under_sanitizers(tmp_path, sanitizer):
    """The column-split, blocked and float64 loops share each output among
    threads; they must agree bitwise at every thread count, including more
    threads than column blocks and empty dimensions, with no report from
    either sanitizer (ThreadSanitizer would name two threads writing one
    column)."""
    exe = str(tmp_path / "cpu_reference_check")
    ret = subprocess.run(["g++", "-std=c++17", "-ffp-contract=off", "-pthread", "-g", "-O1",
                          "-fno-omit-frame-pointer", f"-fsanitize={sanitizer}", "-fno-sanitize-recover=all",
                          "-I", os.path.join(PKG, "runner"), CPU_REF_CHECK, "-o", exe],
                         stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    assert ret.returncode == 0, ret.stdout.decode()[-3000:]
    rc, out = _run([exe])
    assert rc == 0 and out.strip().endswith("ok (0 failed checks)"), out
