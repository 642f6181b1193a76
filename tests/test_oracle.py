"""Pins the CPU oracle before it is trusted as the parity checker (CPU only)."""
import json
import math
import os

import numpy as np
import pytest

import oracle
from shim import sgemm_shim as S

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _golden(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


# ------------------------------------------------------------ inputs
def test_splitmix64_published_outputs():
    kat = _golden("splitmix64_kat.json")
    got = [oracle.splitmix64_at(kat["state"], i) for i in range(len(kat["outputs_hex"]))]
    assert got == [int(h, 16) for h in kat["outputs_hex"]]


def test_fill_matches_golden_vectors_in_all_three_implementations():
    for vec in _golden("fill_vectors.json"):
        seed, mid, idx = vec["seed"], vec["matrix_id"], vec["index"]
        key = oracle.stream_key(seed, mid)
        assert [hex(oracle.splitmix64_at(key, i)) for i in idx] == vec["word_hex"]
        count = max(idx) + 1
        expected = np.array(vec["value"], dtype=np.float32)
        for impl in (oracle.fill, oracle.fill_numpy, S.fill):
            vals = impl(count, seed, mid, 0)
            assert np.array_equal(vals[idx], expected), impl


def test_uniform_values_are_exact_multiples_in_range():
    v = oracle.fill(1 << 16, 9, 0, 0).astype(np.float64)
    assert v.min() >= -1.0 and v.max() < 1.0
    scaled = (v + 1.0) * 2 ** 23
    assert np.array_equal(scaled, np.round(scaled))
    assert abs(v.mean()) < 0.01 and abs(v.std() - 1 / math.sqrt(3)) < 0.01


def test_normal_values_close_between_c_numpy_and_shim():
    c = oracle.fill(1 << 15, 3, 1, 1)
    npy = oracle.fill_numpy(1 << 15, 3, 1, 1)
    sh = S.fill(1 << 15, 3, 1, 1)
    assert np.array_equal(c, sh)  # same C library, same formula
    # numpy's transcendental functions may differ from libm in the last bit of
    # the double; after rounding to float32 they agree to one float32 ulp
    assert np.all(np.abs(c - npy) <= np.spacing(np.abs(c)))
    assert abs(float(c.mean())) < 0.03 and abs(float(c.std()) - 1.0) < 0.03


def test_fill_is_a_pure_function_of_the_index():
    full = S.fill(3 << 20, 5, 2, 0)  # multi-threaded path
    assert np.array_equal(full[:1000], oracle.fill(1000, 5, 2, 0))
    assert np.array_equal(full, oracle.fill_numpy(3 << 20, 5, 2, 0))
    assert not np.array_equal(S.fill(64, 5, 0, 0), S.fill(64, 5, 1, 0))
    assert not np.array_equal(S.fill(64, 5, 0, 0), S.fill(64, 6, 0, 0))


def test_fill_rejects_unknown_distribution():
    with pytest.raises(S.SgemmError, match="unknown distribution"):
        S.fill(8, 0, 0, 7)


# ------------------------------------------------------------ cpu gemm
def test_cpu_gemm_hand_computed():
    # 2x2x3 by hand: A = [[1,2,3],[4,5,6]], B = [[1,0],[0,1],[1,1]], C = [[1,1],[1,1]]
    A = np.array([[1, 2, 3], [4, 5, 6]], dtype=np.float32)
    B = np.array([[1, 0], [0, 1], [1, 1]], dtype=np.float32)
    C = np.ones((2, 2), dtype=np.float32)
    D = oracle.cpu_gemm(A, B, C, alpha=2.0, beta=-1.0)
    assert np.array_equal(D, np.array([[2 * 4 - 1, 2 * 5 - 1], [2 * 10 - 1, 2 * 11 - 1]], dtype=np.float32))


def test_cpu_gemm_is_not_transposed_or_alpha_beta_swapped():
    rng = np.random.default_rng(0)
    A = rng.standard_normal((5, 7)).astype(np.float32)
    B = rng.standard_normal((7, 3)).astype(np.float32)
    C = rng.standard_normal((5, 3)).astype(np.float32)
    D = oracle.cpu_gemm(A, B, C, alpha=0.5, beta=3.0)
    exact = 0.5 * (A.astype(np.float64) @ B.astype(np.float64)) + 3.0 * C
    assert np.allclose(D, exact, rtol=1e-5, atol=1e-5)


def test_cpu_gemm_sums_in_order_in_float():
    # k = 3 with 1 + 2^-24 + 2^-24: a left-to-right float sum loses both small
    # terms (1 + 2^-24 rounds to 1 twice), a double or reordered sum does not.
    A = np.array([[1.0, 1.0, 1.0]], dtype=np.float32)
    B = np.array([[1.0], [2.0 ** -24], [2.0 ** -24]], dtype=np.float32)
    D = oracle.cpu_gemm(A, B)
    assert D[0, 0] == np.float32(1.0)
    assert oracle.gemm_f64(A, B)[0, 0] == 1.0 + 2.0 ** -23


def test_cpu_gemm_threads_are_bitwise_identical():
    A = oracle.fill_matrix(33, 129, 1, 0)
    B = oracle.fill_matrix(129, 47, 1, 1)
    C = oracle.fill_matrix(33, 47, 1, 2)
    D1 = oracle.cpu_gemm(A, B, C, 1.0, 1.0)
    for t in (2, 3, 8, 64):
        assert np.array_equal(D1, oracle.cpu_gemm_mt(A, B, C, 1.0, 1.0, threads=t))


@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (31, 3, 7), (32, 4, 64), (33, 5, 17), (37, 29, 301),
                                   (64, 8, 1000), (100, 1, 33), (1, 100, 33), (65, 9, 0)])
def test_blocked_cpu_gemm_is_bitwise_cpu_gemm(m, n, k):
    """The blocked loop nest (whole-matrix checker) against the plain
    restatement: full blocks, edge blocks in rows and columns, k = 0, and
    every thread split, bit for bit."""
    A = oracle.fill_matrix(m, k, 9, 0, 1)
    B = oracle.fill_matrix(k, n, 9, 1, 1)
    C = oracle.fill_matrix(m, n, 9, 2)
    D = oracle.cpu_gemm(A, B, C, 0.75, -1.25)
    for t in (1, 2, 3, 8, 300):
        assert np.array_equal(oracle.cpu_gemm_blocked(A, B, C, 0.75, -1.25, threads=t), D), t


def test_blocked_cpu_gemm_special_values_and_order():
    """Cases a reordered or fused sum would get wrong: a sum that depends on
    the order of l (1 + 2^-24 + 2^-24 rounds to 1 left to right, not right to
    left), a fused multiply-add (the product 1 + 2^-23 squared loses its low
    bit only when rounded before the add), and NaN/Inf propagation with
    beta = 0 (0 * NaN in C stays NaN, as in the reference's d = beta*c + alpha*acc)."""
    A = np.array([[1.0, 1.0, 1.0]] * 32, dtype=np.float32)
    B = np.array([[1.0] * 4, [2.0 ** -24] * 4, [2.0 ** -24] * 4], dtype=np.float32)
    D = oracle.cpu_gemm_blocked(A, B)
    assert np.all(D == np.float32(1.0))
    x = np.float32(1.0 + 2.0 ** -23)
    A = np.full((32, 2), x, dtype=np.float32)
    A[:, 0] = -1.0
    B = np.array([[1.0] * 4, [x] * 4], dtype=np.float32)
    # acc = -1, then acc + x*x: the rounded product 1 + 2^-22 gives 2^-22 exactly;
    # fma(x, x, -1) would keep the product's 2^-46 as well
    assert np.all(oracle.cpu_gemm_blocked(A, B) == np.float32(2.0 ** -22))
    A = oracle.fill_matrix(40, 9, 4, 0)
    B = oracle.fill_matrix(9, 6, 4, 1)
    A[3, 2] = np.inf
    B[4, 5] = np.nan
    C = np.zeros((40, 6), dtype=np.float32)
    C[7, 1] = np.nan
    for beta in (0.0, 1.0):
        got = oracle.cpu_gemm_blocked(A, B, C, 1.0, beta, threads=3)
        want = oracle.cpu_gemm(A, B, C, 1.0, beta)
        assert np.array_equal(np.isnan(got), np.isnan(want)) and np.isnan(got[7, 1])
        ok = ~np.isnan(want)
        assert np.array_equal(got[ok], want[ok])


def test_blocked_cpu_gemm_catches_a_misplaced_output():
    """A planted mistake (two output rows swapped) is seen by the bitwise
    comparison the GPU tests use."""
    A = oracle.fill_matrix(64, 50, 5, 0)
    B = oracle.fill_matrix(50, 8, 5, 1)
    D = oracle.cpu_gemm_blocked(A, B)
    bad = D.copy()
    bad[[3, 40]] = bad[[40, 3]]
    assert not np.array_equal(bad, oracle.cpu_gemm(A, B))
    assert oracle.normwise_error(bad, oracle.gemm_f64(A, B)) > oracle.tolerance(50)


def test_cpu_gemm_column_slice_equals_full_gemm_columns():
    A = oracle.fill_matrix(64, 80, 2, 0)
    B = oracle.fill_matrix(80, 40, 2, 1)
    D = oracle.cpu_gemm(A, B)
    cols = [0, 7, 39]
    assert np.array_equal(D[:, cols], oracle.cpu_gemm(A, B[:, cols]))


def test_oracle_equals_reference_cpu_gemm_bitwise():
    """The restatement against the reference's own cpuGemm compiled from its
    source (oracle/_ref/libref_runner.so, built by `make -C oracle ref`)."""
    if oracle.ref_lib() is None:
        pytest.skip("oracle/_ref not built (reference sources not mounted at build time)")
    for (m, n, k, seed, dist, alpha, beta) in ((32, 32, 32, 0, 0, 1.0, 0.0), (96, 40, 200, 7, 1, 1.0, 1.0),
                                               (17, 5, 1, 3, 0, -2.0, 0.5), (128, 64, 1024, 1, 0, 1.0, 1.0)):
        A = oracle.fill_matrix(m, k, seed, 0, dist)
        B = oracle.fill_matrix(k, n, seed, 1, dist)
        C = oracle.fill_matrix(m, n, seed, 2, dist)
        ref = oracle.ref_cpu_gemm(A, B, C, alpha, beta)
        assert np.array_equal(oracle.cpu_gemm(A, B, C, alpha, beta), ref)
        assert np.array_equal(oracle.cpu_gemm_blocked(A, B, C, alpha, beta, threads=3), ref)


def test_reference_arange_cases_against_exact_golden():
    for case in _golden("reference_arange_cases.json"):
        m, n, k = case["m"], case["n"], case["k"]
        A = np.arange(m * k, dtype=np.float32).reshape(k, m).T
        B = np.arange(k * n, dtype=np.float32).reshape(n, k).T
        C = np.ones((m, n), dtype=np.float32)
        exact = np.array(case["d_colmajor"], dtype=np.float64).reshape(n, m).T
        assert np.array_equal(A.astype(np.float64) @ B.astype(np.float64) + 1.0, exact)
        D = oracle.cpu_gemm(A, B, C, 1.0, 1.0)
        assert np.allclose(D, exact, rtol=1e-5)  # the reference's own bar (test_vm.py:537)


def test_cpu_gemm_error_against_f64_within_parity_bar():
    for (m, n, k) in ((64, 64, 4096), (32, 16, 16384)):
        A = oracle.fill_matrix(m, k, 2, 0)
        B = oracle.fill_matrix(k, n, 2, 1)
        err = oracle.normwise_error(oracle.cpu_gemm(A, B), oracle.gemm_f64(A, B))
        assert err <= oracle.tolerance(k)


def test_normwise_error_metric():
    R = np.array([[1.0, -4.0], [2.0, 0.5]])
    assert oracle.normwise_error(R, R) == 0.0
    assert oracle.normwise_error(R + np.array([[0, 0], [0.4, 0]]), R) == pytest.approx(0.1)
    assert oracle.normwise_error(np.array([[np.nan]]), np.array([[1.0]])) == math.inf
    assert oracle.tolerance(4096) == pytest.approx(6.4e-4)
