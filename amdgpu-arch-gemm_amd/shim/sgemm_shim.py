"""ctypes binding of libsgemm_shim.so (include/sgemm_shim.h).

This is the only way Python reaches HIP in this package: no torch, no hip
Python bindings.  Every call checks the return code and raises
``SgemmError`` with the library's message.  There is no CPU fallback: if the
library or a GPU is missing, calls fail loudly.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional, Tuple

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY_PATH = os.path.join(_HERE, "libsgemm_shim.so")

SGEMM_DIST_UNIFORM = 0
SGEMM_DIST_NORMAL = 1
SGEMM_DIST_ZERO = 2
# static split-K scratch of sgemm_launch_noalloc (include/sgemm_shim.h)
SGEMM_NOALLOC_PARTIAL_BYTES = 32 << 20
SGEMM_NOALLOC_MAX_TILES = 16384

# every symbol the header declares, with (restype, argtypes)
_u32 = ctypes.c_uint32
_f32 = ctypes.c_float
_vp = ctypes.c_void_p
_int = ctypes.c_int
_LAUNCH_ARGS = [_vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _f32, _f32]


class KernelInfo(ctypes.Structure):
    _fields_ = [
        ("mfma", ctypes.c_int * 4),
        ("wave_group", ctypes.c_int * 2),
        ("wave_tiling", ctypes.c_int * 2),
        ("depth_k", ctypes.c_int),
        ("vmem_stage", ctypes.c_int),
        ("wavefront_size", ctypes.c_int),
        ("lds_usage_bytes", ctypes.c_int),
        ("tile_m", ctypes.c_int),
        ("tile_n", ctypes.c_int),
        ("workitems", ctypes.c_int),
        ("trans_a", ctypes.c_int),
        ("trans_b", ctypes.c_int),
        ("split_k", ctypes.c_int),
        ("split_k_max", ctypes.c_int),
        ("stream_k", ctypes.c_int),
        ("stream_k_groups", ctypes.c_int),
        ("stream_k_rounds", ctypes.c_int),
    ]


SIGNATURES = {
    "sgemm_last_error": (ctypes.c_char_p, []),
    "sgemm_abi_version": (_int, []),
    "sgemm_device_info": (_int, [ctypes.c_char_p, ctypes.c_size_t, ctypes.POINTER(_int), ctypes.POINTER(_int),
                                 ctypes.POINTER(_int)]),
    "sgemm_open": (_int, [ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(_vp)]),
    "sgemm_close": (None, [_vp]),
    "sgemm_get_info": (_int, [_vp, ctypes.POINTER(KernelInfo)]),
    "sgemm_check_shape": (_int, [_vp, _u32, _u32, _u32, _u32, _u32, _u32, _u32]),
    "sgemm_set_split_k": (_int, [_vp, _int]),
    "sgemm_workspace_size": (_int, [_vp, _u32, _u32, _u32, ctypes.POINTER(ctypes.c_size_t)]),
    "sgemm_launch_splits": (_int, [_vp, _u32, _u32, _u32, ctypes.POINTER(_int)]),
    "sgemm_set_stream_k": (_int, [_vp, _int]),
    "sgemm_set_edge_kernel": (_int, [_vp, _vp]),
    "sgemm_set_edge_kernels": (_int, [_vp, _vp, _vp]),
    "sgemm_edge_interior": (_int, [_vp, _u32, _u32, _u32, ctypes.POINTER(_u32), ctypes.POINTER(_u32)]),
    "sgemm_stream_k_tiles": (_int, [_vp, _u32, _u32, _u32, ctypes.POINTER(_int)]),
    "sgemm_set_stream": (_int, [_vp, _vp]),
    "sgemm_malloc": (_int, [ctypes.POINTER(_vp), ctypes.c_size_t]),
    "sgemm_free": (_int, [_vp]),
    "sgemm_memcpy_h2d": (_int, [_vp, _vp, ctypes.c_size_t]),
    "sgemm_memcpy_d2h": (_int, [_vp, _vp, ctypes.c_size_t]),
    "sgemm_memset": (_int, [_vp, _int, ctypes.c_size_t]),
    "sgemm_launch": (_int, _LAUNCH_ARGS),
    "sgemm_launch_noalloc": (_int, _LAUNCH_ARGS),
    "sgemm_time": (_int, _LAUNCH_ARGS + [_int, _int, ctypes.POINTER(_f32)]),
    "sgemm_time_each": (_int, _LAUNCH_ARGS + [_int, ctypes.POINTER(_f32)]),
    "sgemm_synchronize": (_int, [_vp]),
    "sgemm_run": (_int, [_vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _f32, _f32, _int, _int,
                         ctypes.POINTER(ctypes.c_double)]),
    "sgemm_fill": (_int, [_vp, ctypes.c_size_t, ctypes.c_uint64, _u32, _int]),
}


class SgemmError(RuntimeError):
    def __init__(self, func: str, code: int, message: str):
        super().__init__(f"{func} failed ({code}): {message}")
        self.func = func
        self.code = code
        self.message = message


_lib: Optional[ctypes.CDLL] = None


def load_library(path: str = LIBRARY_PATH) -> ctypes.CDLL:
    """Loads the shim once; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is missing: build it first (python -c 'import __graft_entry__ as g; g.build()')")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def _check(func: str, code: int):
    if code != 0:
        msg = load_library().sgemm_last_error().decode(errors="replace")
        raise SgemmError(func, code, msg)


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def fill(count: int, seed: int, matrix_id: int, dist: int = SGEMM_DIST_UNIFORM) -> np.ndarray:
    """Seeded input values (float32), identical on every host for a given (seed, matrix_id, i)."""
    out = np.empty(int(count), dtype=np.float32)
    _check("sgemm_fill", load_library().sgemm_fill(_ptr(out), out.size, int(seed), int(matrix_id), int(dist)))
    return out


def fill_matrix(rows: int, cols: int, seed: int, matrix_id: int, dist: int = SGEMM_DIST_UNIFORM) -> np.ndarray:
    """Column-major rows x cols matrix as a Fortran-ordered float32 array."""
    return fill(rows * cols, seed, matrix_id, dist).reshape(cols, rows).T


def device_info() -> dict:
    lib = load_library()
    name = ctypes.create_string_buffer(256)
    cus, clk, lds = _int(), _int(), _int()
    _check("sgemm_device_info", lib.sgemm_device_info(name, 256, ctypes.byref(cus), ctypes.byref(clk),
                                                      ctypes.byref(lds)))
    return {"name": name.value.decode(), "compute_units": cus.value, "clock_khz": clk.value,
            "lds_per_block": lds.value}


class DeviceBuffer:
    """Device allocation owned by Python; freed on close() or garbage collection."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = _vp()
        _check("sgemm_malloc", load_library().sgemm_malloc(ctypes.byref(p), self.nbytes))
        self.ptr = p.value

    @staticmethod
    def column_major_bytes(a: np.ndarray) -> np.ndarray:
        """The float32 values of `a` in the order the device holds them: a 2-D
        array column by column (element (i, j) at i + j * rows), whatever its
        numpy order or strides; a 1-D array as it is.  Arrays of other ranks
        are refused: their device layout would be a guess."""
        a = np.asarray(a, dtype=np.float32)
        if a.ndim not in (1, 2):
            raise ValueError(f"device buffers hold 1-D or 2-D (column-major) arrays, not {a.ndim}-D")
        return np.ascontiguousarray(a.ravel(order="F"))

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        flat = cls.column_major_bytes(a)
        buf = cls(flat.nbytes)
        buf.upload(flat)
        return buf

    def upload(self, a: np.ndarray):
        """Copies `a` to the start of the buffer, column-major like from_array."""
        flat = self.column_major_bytes(a)
        if flat.nbytes > self.nbytes:
            raise ValueError("array larger than the device buffer")
        _check("sgemm_memcpy_h2d", load_library().sgemm_memcpy_h2d(self.ptr, _ptr(flat), flat.nbytes))

    def download(self, count: Optional[int] = None) -> np.ndarray:
        count = self.nbytes // 4 if count is None else int(count)
        out = np.empty(count, dtype=np.float32)
        _check("sgemm_memcpy_d2h", load_library().sgemm_memcpy_d2h(_ptr(out), self.ptr, out.nbytes))
        return out

    def zero(self):
        _check("sgemm_memset", load_library().sgemm_memset(self.ptr, 0, self.nbytes))

    def view(self, offset: int, nbytes: int) -> "DeviceView":
        """The bytes [offset, offset + nbytes) of this allocation, usable
        wherever a DeviceBuffer is (a launch needs 4-byte aligned pointers)."""
        return DeviceView(self, offset, nbytes)

    def close(self):
        if self.ptr:
            load_library().sgemm_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DeviceView(DeviceBuffer):
    """A byte range of a DeviceBuffer; it owns nothing and keeps its owner alive."""

    def __init__(self, owner: DeviceBuffer, offset: int, nbytes: int):
        offset, nbytes = int(offset), int(nbytes)
        if offset < 0 or nbytes < 0 or offset + nbytes > owner.nbytes:
            raise ValueError(f"view [{offset}, {offset + nbytes}) outside a {owner.nbytes}-byte buffer")
        self.owner = owner
        self.nbytes = nbytes
        self.ptr = owner.ptr + offset

    def close(self):
        self.ptr = None


class Kernel:
    """One loaded code object (.co + .toml)."""

    def __init__(self, co_path: str, toml_path: str):
        lib = load_library()
        h = _vp()
        _check("sgemm_open", lib.sgemm_open(co_path.encode(), toml_path.encode(), ctypes.byref(h)))
        self.handle = h.value
        self.co_path = co_path
        self.toml_path = toml_path
        info = KernelInfo()
        _check("sgemm_get_info", lib.sgemm_get_info(self.handle, ctypes.byref(info)))
        self.info = info

    @property
    def tile(self) -> Tuple[int, int, int]:
        return self.info.tile_m, self.info.tile_n, self.info.depth_k

    def default_lds(self, m, n, k) -> Tuple[int, int]:
        """Tight (lda, ldb) for this kernel's transposition."""
        return (k if self.info.trans_a else m), (n if self.info.trans_b else k)

    def check_shape(self, m, n, k, lda=None, ldb=None, ldc=None, ldd=None) -> Optional[str]:
        lib = load_library()
        da, db = self.default_lds(m, n, k)
        rc = lib.sgemm_check_shape(self.handle, m, n, k, lda or da, ldb or db, ldc or m, ldd or m)
        return None if rc == 0 else lib.sgemm_last_error().decode()

    def _refresh_info(self):
        _check("sgemm_get_info", load_library().sgemm_get_info(self.handle, ctypes.byref(self.info)))

    @property
    def split_k(self) -> int:
        return self.info.split_k

    def set_split_k(self, splits: int):
        """K ranges per output tile for later launches (1 = the reference's kernel)."""
        _check("sgemm_set_split_k", load_library().sgemm_set_split_k(self.handle, int(splits)))
        self._refresh_info()

    def workspace_size(self, m, n, k) -> int:
        out = ctypes.c_size_t()
        _check("sgemm_workspace_size", load_library().sgemm_workspace_size(self.handle, m, n, k, ctypes.byref(out)))
        return int(out.value)

    def launch_splits(self, m, n, k) -> int:
        """K ranges a launch of this shape uses with the current setting (1 = no split)."""
        out = _int()
        _check("sgemm_launch_splits", load_library().sgemm_launch_splits(self.handle, m, n, k, ctypes.byref(out)))
        return int(out.value)

    def set_stream_k(self, mode: int):
        """0: never stream-K; 1: when a partial last round of work-groups costs >= 3%; 2: whenever tiles > groups."""
        _check("sgemm_set_stream_k", load_library().sgemm_set_stream_k(self.handle, int(mode)))
        self._refresh_info()

    def set_edge_kernel(self, edge: Optional["Kernel"]):
        """One small-tile kernel for both thin edge strips (None detaches); it must stay open while attached."""
        self.set_edge_kernels(edge, edge)

    def set_edge_kernels(self, rows: Optional["Kernel"], cols: Optional["Kernel"]):
        """Kernels for the thin strip of rows past the last tile row and of columns past the last tile
        column (either may be None); they must stay open while attached."""
        _check("sgemm_set_edge_kernels", load_library().sgemm_set_edge_kernels(
            self.handle, rows.handle if rows else None, cols.handle if cols else None))
        self.edges = (rows, cols)

    def edge_interior(self, m, n, k) -> Tuple[int, int]:
        """(m, n) of the part of an m x n x k launch this kernel runs itself."""
        mi, ni = _u32(), _u32()
        _check("sgemm_edge_interior", load_library().sgemm_edge_interior(self.handle, m, n, k, ctypes.byref(mi),
                                                                         ctypes.byref(ni)))
        return int(mi.value), int(ni.value)

    def stream_k_tiles(self, m, n, k) -> int:
        """Tiles of the stream-K phase of an m x n x k launch (0: no stream-K)."""
        out = _int()
        _check("sgemm_stream_k_tiles", load_library().sgemm_stream_k_tiles(self.handle, m, n, k, ctypes.byref(out)))
        return int(out.value)

    def _args(self, a, b, c, d, m, n, k, lda, ldb, ldc, ldd, alpha, beta):
        cp = c.ptr if c is not None else None
        da, db = self.default_lds(m, n, k)
        return (self.handle, a.ptr if a is not None else None, b.ptr if b is not None else None, cp, d.ptr,
                m, n, k, lda or da, ldb or db, ldc or m, ldd or m, alpha, beta)

    def launch(self, a, b, c, d, m, n, k, alpha=1.0, beta=0.0, lda=None, ldb=None, ldc=None, ldd=None):
        _check("sgemm_launch", load_library().sgemm_launch(*self._args(a, b, c, d, m, n, k, lda, ldb, ldc, ldd,
                                                                         alpha, beta)))

    def launch_noalloc(self, a, b, c, d, m, n, k, alpha=1.0, beta=0.0, lda=None, ldb=None, ldc=None, ldd=None):
        """launch() without device allocation: a split launch works in the
        library's static per-device scratch (calls on one device must not overlap)."""
        _check("sgemm_launch_noalloc", load_library().sgemm_launch_noalloc(
            *self._args(a, b, c, d, m, n, k, lda, ldb, ldc, ldd, alpha, beta)))

    def time(self, a, b, c, d, m, n, k, alpha=1.0, beta=0.0, warmup=1, runs=10,
             lda=None, ldb=None, ldc=None, ldd=None) -> float:
        """Event time (ms) of `runs` back-to-back launches after `warmup`."""
        total = _f32()
        _check("sgemm_time", load_library().sgemm_time(*self._args(a, b, c, d, m, n, k, lda, ldb, ldc, ldd,
                                                                     alpha, beta), warmup, runs, ctypes.byref(total)))
        return float(total.value)

    def time_each(self, a, b, c, d, m, n, k, alpha=1.0, beta=0.0, runs=10,
                  lda=None, ldb=None, ldc=None, ldd=None) -> np.ndarray:
        out = np.zeros(runs, dtype=np.float32)
        _check("sgemm_time_each", load_library().sgemm_time_each(
            *self._args(a, b, c, d, m, n, k, lda, ldb, ldc, ldd, alpha, beta), runs,
            out.ctypes.data_as(ctypes.POINTER(_f32))))
        return out

    def set_stream(self, stream: Optional[int]):
        """Launch on a caller-owned hipStream_t (an integer handle; None: the handle's own stream)."""
        _check("sgemm_set_stream", load_library().sgemm_set_stream(self.handle, stream or None))

    def synchronize(self):
        _check("sgemm_synchronize", load_library().sgemm_synchronize(self.handle))

    def run(self, A: np.ndarray, B: np.ndarray, C: Optional[np.ndarray], m: int, n: int, k: int,
            alpha: float = 1.0, beta: float = 0.0, warmup: int = 0, runs: int = 1) -> Tuple[np.ndarray, float]:
        """Host-buffer flow: returns (D as a column-major m x n array, ms per run).
        A and B are the stored matrices: m x k (k x m for a trans_a kernel) and
        k x n (n x k for a trans_b kernel)."""
        A = np.asfortranarray(A, dtype=np.float32)
        B = np.asfortranarray(B, dtype=np.float32)
        sa = (k, m) if self.info.trans_a else (m, k)
        sb = (n, k) if self.info.trans_b else (k, n)
        if A.shape != sa or B.shape != sb:
            raise ValueError(f"A must be {sa[0]}x{sa[1]} and B {sb[0]}x{sb[1]}, got {A.shape} and {B.shape}")
        cptr = None
        if C is not None:
            C = np.asfortranarray(C, dtype=np.float32)
            if C.shape != (m, n):
                raise ValueError(f"C must be {m}x{n}")
            cptr = C.ctypes.data
        D = np.zeros((m, n), dtype=np.float32, order="F")
        ms = ctypes.c_double()
        _check("sgemm_run", load_library().sgemm_run(self.handle, A.ctypes.data, B.ctypes.data, cptr, D.ctypes.data,
                                                     m, n, k, alpha, beta, warmup, runs, ctypes.byref(ms)))
        return D, ms.value

    def close(self):
        if getattr(self, "handle", None):
            load_library().sgemm_close(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
