"""TEST INFRASTRUCTURE -- Python face of the CPU oracle.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only to check or to time the CPU baseline; the product
(amdgpu-arch-gemm_amd/) never imports it.

* ``cpu_gemm`` / ``cpu_gemm_mt``: liboracle.so's restatement of the reference
  runner's cpuGemm (/root/reference/runner/generator_runner.cpp:16-33).
* ``cpu_gemm_blocked``: the same arithmetic, cache- and register-blocked over
  threads (every output keeps its one float accumulator and its order over l),
  bitwise equal to ``cpu_gemm``; the whole-matrix checker at full sizes.
* ``ref_cpu_gemm``: the reference's own cpuGemm, compiled from its source into
  ``_ref/libref_runner.so`` (see Makefile); ``None`` when that was not built.
* ``gemm_f64``: double-accumulated reference for error bounds.
* ``fill``: liboracle.so's restatement of the seeded input generator, and
  ``fill_numpy``: an independent numpy restatement of the same definition.
* ``normwise_error``: the parity metric max|D - D_ref| / max|D_ref|, checked
  against ``tolerance(k) = 1e-5 * sqrt(k)``.
"""
from __future__ import annotations

import ctypes
import math
import os
from typing import Optional

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_LIB_PATH = os.path.join(HERE, "_ref", "libref_runner.so")
REF_RUNNER_PATH = os.path.join(HERE, "_ref", "GeneratorRunner")
# Itanium mangling of `void cpuGemm(const float*, const float*, const float*,
# float*, float, float, uint32_t, uint32_t, uint32_t)`.
REF_CPU_GEMM_SYMBOL = "_Z7cpuGemmPKfS0_S0_Pfffjjj"

_lib = None
_ref = None

_vp = ctypes.c_void_p
_f = ctypes.c_float
_u32 = ctypes.c_uint32


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle`")
        L = ctypes.CDLL(LIB_PATH)
        L.oracle_cpu_gemm.argtypes = [_vp, _vp, _vp, _vp, _f, _f, _u32, _u32, _u32]
        L.oracle_cpu_gemm.restype = None
        L.oracle_cpu_gemm_mt.argtypes = [_vp, _vp, _vp, _vp, _f, _f, _u32, _u32, _u32, ctypes.c_int]
        L.oracle_cpu_gemm_mt.restype = ctypes.c_int
        L.oracle_cpu_gemm_blocked.argtypes = [_vp, _vp, _vp, _vp, _f, _f, _u32, _u32, _u32, ctypes.c_int]
        L.oracle_cpu_gemm_blocked.restype = ctypes.c_int
        L.oracle_gemm_f64.argtypes = [_vp, _vp, _vp, _vp, ctypes.c_double, ctypes.c_double, _u32, _u32, _u32]
        L.oracle_gemm_f64.restype = None
        L.oracle_splitmix64_at.argtypes = [ctypes.c_uint64, ctypes.c_uint64]
        L.oracle_splitmix64_at.restype = ctypes.c_uint64
        L.oracle_stream_key.argtypes = [ctypes.c_uint64, _u32]
        L.oracle_stream_key.restype = ctypes.c_uint64
        L.oracle_fill.argtypes = [_vp, ctypes.c_size_t, ctypes.c_uint64, _u32, ctypes.c_int]
        L.oracle_fill.restype = ctypes.c_int
        _lib = L
    return _lib


def ref_lib() -> Optional[ctypes.CDLL]:
    """The reference's cpuGemm built from its source, or None if not built."""
    global _ref
    if _ref is None:
        if not os.path.exists(REF_LIB_PATH):
            return None
        L = ctypes.CDLL(REF_LIB_PATH)
        fn = getattr(L, REF_CPU_GEMM_SYMBOL)
        fn.argtypes = [_vp, _vp, _vp, _vp, _f, _f, _u32, _u32, _u32]
        fn.restype = None
        _ref = L
    return _ref


def _f32(a) -> np.ndarray:
    return np.asfortranarray(a, dtype=np.float32)


def _zeros_like_c(m: int, n: int, c) -> np.ndarray:
    return _f32(c) if c is not None else np.zeros((m, n), dtype=np.float32, order="F")


def cpu_gemm(A, B, C=None, alpha: float = 1.0, beta: float = 0.0) -> np.ndarray:
    """D = beta*C + alpha*(A@B) with the reference cpuGemm's float arithmetic."""
    A, B = _f32(A), _f32(B)
    m, k = A.shape
    k2, n = B.shape
    assert k == k2
    C = _zeros_like_c(m, n, C)
    D = np.empty((m, n), dtype=np.float32, order="F")
    lib().oracle_cpu_gemm(A.ctypes.data, B.ctypes.data, C.ctypes.data, D.ctypes.data, alpha, beta, m, n, k)
    return D


def cpu_gemm_mt(A, B, C=None, alpha: float = 1.0, beta: float = 0.0, threads: int = 8) -> np.ndarray:
    A, B = _f32(A), _f32(B)
    m, k = A.shape
    _, n = B.shape
    C = _zeros_like_c(m, n, C)
    D = np.empty((m, n), dtype=np.float32, order="F")
    lib().oracle_cpu_gemm_mt(A.ctypes.data, B.ctypes.data, C.ctypes.data, D.ctypes.data, alpha, beta, m, n, k,
                             threads)
    return D


def cpu_gemm_blocked(A, B, C=None, alpha: float = 1.0, beta: float = 0.0, threads: int = 8) -> np.ndarray:
    """cpuGemm's result (bitwise) from the blocked loop nest: seconds at 4096^3."""
    A, B = _f32(A), _f32(B)
    m, k = A.shape
    k2, n = B.shape
    assert k == k2
    C = _zeros_like_c(m, n, C)
    D = np.empty((m, n), dtype=np.float32, order="F")
    lib().oracle_cpu_gemm_blocked(A.ctypes.data, B.ctypes.data, C.ctypes.data, D.ctypes.data, alpha, beta, m, n, k,
                                  threads)
    return D


def ref_cpu_gemm(A, B, C=None, alpha: float = 1.0, beta: float = 0.0) -> Optional[np.ndarray]:
    """The reference's own cpuGemm (needs a C buffer: it always reads C)."""
    L = ref_lib()
    if L is None:
        return None
    A, B = _f32(A), _f32(B)
    m, k = A.shape
    _, n = B.shape
    C = _zeros_like_c(m, n, C)
    D = np.empty((m, n), dtype=np.float32, order="F")
    getattr(L, REF_CPU_GEMM_SYMBOL)(A.ctypes.data, B.ctypes.data, C.ctypes.data, D.ctypes.data, alpha, beta,
                                     m, n, k)
    return D


def gemm_f64(A, B, C=None, alpha: float = 1.0, beta: float = 0.0) -> np.ndarray:
    A, B = _f32(A), _f32(B)
    m, k = A.shape
    _, n = B.shape
    C = _zeros_like_c(m, n, C)
    D = np.empty((m, n), dtype=np.float64, order="F")
    lib().oracle_gemm_f64(A.ctypes.data, B.ctypes.data, C.ctypes.data, D.ctypes.data, alpha, beta, m, n, k)
    return D


def splitmix64_at(key: int, i: int) -> int:
    return int(lib().oracle_splitmix64_at(key, i))


def stream_key(seed: int, matrix_id: int) -> int:
    return int(lib().oracle_stream_key(seed, matrix_id))


def fill(count: int, seed: int, matrix_id: int, dist: int = 0) -> np.ndarray:
    out = np.empty(int(count), dtype=np.float32)
    rc = lib().oracle_fill(out.ctypes.data, out.size, seed, matrix_id, dist)
    if rc:
        raise ValueError(f"unknown distribution {dist}")
    return out


def fill_matrix(rows: int, cols: int, seed: int, matrix_id: int, dist: int = 0) -> np.ndarray:
    return fill(rows * cols, seed, matrix_id, dist).reshape(cols, rows).T


# ------------------------------------------------------- numpy restatement
_M64 = (1 << 64) - 1
GAMMA = 0x9E3779B97F4A7C15


def _mix64_np(z: np.ndarray) -> np.ndarray:
    z = z.astype(np.uint64)
    z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def _mix64_int(z: int) -> int:
    z &= _M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & _M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & _M64
    return z ^ (z >> 31)


def fill_numpy(count: int, seed: int, matrix_id: int, dist: int = 0) -> np.ndarray:
    key = _mix64_int(seed ^ ((0xD1B54A32D192ED03 * (matrix_id + 1)) & _M64))
    with np.errstate(over="ignore"):
        if dist == 0:
            i = np.arange(count, dtype=np.uint64)
            w = _mix64_np(np.uint64(key) + (i + np.uint64(1)) * np.uint64(GAMMA))
            u = (w >> np.uint64(40)).astype(np.float32) * np.float32(2.0 ** -24)
            return (u * np.float32(2.0) - np.float32(1.0)).astype(np.float32)
        if dist == 1:
            i = np.arange(count, dtype=np.uint64)
            p = i >> np.uint64(1)
            w1 = _mix64_np(np.uint64(key) + (np.uint64(2) * p + np.uint64(1)) * np.uint64(GAMMA))
            w2 = _mix64_np(np.uint64(key) + (np.uint64(2) * p + np.uint64(2)) * np.uint64(GAMMA))
            u1 = ((w1 >> np.uint64(11)) + np.uint64(1)).astype(np.float64) * 2.0 ** -53
            u2 = (w2 >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
            r = np.sqrt(-2.0 * np.log(u1))
            th = 2.0 * math.pi * u2
            z = np.where((i & np.uint64(1)) == np.uint64(1), r * np.sin(th), r * np.cos(th))
            return z.astype(np.float32)
        if dist == 2:
            return np.zeros(count, dtype=np.float32)
    raise ValueError(f"unknown distribution {dist}")


# ----------------------------------------------------------------- parity
def tolerance(k: int) -> float:
    """Normwise relative tolerance 1e-5 * sqrt(K) of the parity contract."""
    return 1e-5 * math.sqrt(max(int(k), 1))


def normwise_error(D, D_ref) -> float:
    D = np.asarray(D, dtype=np.float64)
    R = np.asarray(D_ref, dtype=np.float64)
    if not np.all(np.isfinite(D)):
        return math.inf
    denom = float(np.max(np.abs(R))) if R.size else 0.0
    err = float(np.max(np.abs(D - R))) if R.size else 0.0
    return err / denom if denom > 0 else err
