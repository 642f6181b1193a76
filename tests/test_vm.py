"""The GPU-free oracle: this project's compiled gfx950 kernels executed by the
virtual machine (oracle/vm) and checked against numpy (CPU only).

Mirrors the reference's VM tests (/root/reference/test/test_vm.py): MFMA
layout known-answer tests (:409-445), whole-kernel SGEMMs on arange inputs
(:447-627), the work-group remap closed form (:630-740) and result
invariance under map_k_idx / extra LDS stages (:743-963) -- but every kernel
here is the real hipcc output for gfx950, not an emitter's instruction list.
"""
import copy
import json
import os
import struct

import numpy as np
import pytest

import oracle
from generator import catalog
from generator import generator as g
from vm import gcn_virtual_machine as V
from vm.gcn_virtual_machine import GcnVirtualMachine, parse_operand, run_kernel, run_sgemm, pack_kernargs
from ksplit import k_split_ranges

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
_PROGRAMS = {}


def program(name, kernel="generated_gemm"):
    """Parsed gfx950 assembly of a catalog instance's kernel (hipcc -S of its source)."""
    if (name, kernel) not in _PROGRAMS:
        cfg, opt = catalog.SOLUTIONS[name]
        if name not in _PROGRAMS:
            ctx = g.GpuContext()
            g.gemm(ctx, "generated_gemm", "gfx950", cfg, opt, g.default_arguments())
            _PROGRAMS[name] = ctx.assembly()
        _PROGRAMS[(name, kernel)] = (V.parse_assembly(_PROGRAMS[name], kernel), cfg)
    return _PROGRAMS[(name, kernel)]


def vm_sgemm(name, A, B, C=None, alpha=1.0, beta=0.0):
    prog, cfg = program(name)
    return run_sgemm(prog, cfg.tile_size, cfg.num_workitems, A, B, C, alpha, beta)


def fbits(x):
    return struct.unpack("<I", struct.pack("<f", float(x)))[0]


# ------------------------------------------------------------ MFMA KATs
def _mfma_once(mn, k, a_vals, b_vals):
    vm = GcnVirtualMachine(104, 256, 64)
    vm.v[0] = np.array([fbits(x) for x in a_vals], dtype=np.uint32)
    vm.v[1] = np.array([fbits(x) for x in b_vals], dtype=np.uint32)
    slots = 16 if mn == 32 else 4
    for j in range(slots):
        vm.a[j] = np.array([fbits(0.25 * (j + 1))] * 64, dtype=np.uint32)
    c = vm.accvgpr_to_ndarray(0, mn, mn, k)
    asm = f"generated_gemm:\n\tv_mfma_f32_{mn}x{mn}x{k}_f32 a[0:{slots - 1}], v0, v1, a[0:{slots - 1}]\n\ts_endpgm\n"
    vm.run(asm)
    d = vm.accvgpr_to_ndarray(0, mn, mn, k)
    a = vm.vgpr_to_ndarray(0, mn, k)
    b = vm.vgpr_to_ndarray(1, mn, k)
    return a, b, c, d


def test_mfma_16x16x4_known_answer():
    # reference test_vm.py:409-427: lane values, ref = b.T @ a + c
    a, b, c, d = _mfma_once(16, 4, [float(i) for i in range(64)], [float(i) for i in range(64)])
    assert np.allclose(d, b.T @ a + c)


def test_mfma_32x32x2_known_answer():
    # reference test_vm.py:429-445: lane % 7
    a, b, c, d = _mfma_once(32, 2, [float(i % 7) for i in range(64)], [float(i % 7) for i in range(64)])
    assert np.allclose(d, b.T @ a + c)


def test_mfma_layout_single_entry():
    # one nonzero A and B entry pins the (row, col) of the result slot exactly:
    # A[5][1] = 2 (lane 5 + 32*1), B[1][9] = 3 (lane 9 + 32*1) -> D[5][9] = 6
    av = [0.0] * 64
    bv = [0.0] * 64
    av[5 + 32] = 2.0
    bv[9 + 32] = 3.0
    _, _, c, d = _mfma_once(32, 2, av, bv)
    delta = d - c
    assert delta[9, 5] == 6.0 and np.count_nonzero(delta) == 1
    # and in register terms: D[5][9] is slot (5%4) + 8*(5//8) = 1 of lane 9 + 32*((5//4)%2) = 41
    rows, cols = V._ACC_INDEX[32]
    assert rows[1, 41] == 5 and cols[1, 41] == 9


# ------------------------------------------------------ whole kernels
def test_baseline_config1_32cube_in_vm():
    """32^3, U[-1,1) seed 0, C = 0, alpha = 1, beta = 0,
    one wave with the 32x32x2 atom, checked against a numpy float64 matmul."""
    m = n = k = 32
    A = oracle.fill_matrix(m, k, 0, 0)
    B = oracle.fill_matrix(k, n, 0, 1)
    D, info = vm_sgemm("mt32x32_a32_wg1x1_dk16", A, B, None, 1.0, 0.0)
    ref64 = A.astype(np.float64) @ B.astype(np.float64)
    assert oracle.normwise_error(D, ref64) <= oracle.tolerance(k)
    assert oracle.normwise_error(D, oracle.cpu_gemm(A, B)) <= oracle.tolerance(k)
    assert info["grid"] == (1, 1)


@pytest.mark.parametrize("case", json.load(open(os.path.join(GOLDEN, "reference_arange_cases.json"))),
                         ids=lambda c: c["atom"])
def test_reference_arange_cases_in_vm(case):
    name = {"16x16x4": "mt16x16_a16_wg1x1_dk16", "32x32x2": "mt32x32_a32_wg1x1_dk16"}[case["atom"]]
    m, n, k = case["m"], case["n"], case["k"]
    A = np.arange(m * k, dtype=np.float32).reshape(k, m).T
    B = np.arange(k * n, dtype=np.float32).reshape(n, k).T
    C = np.ones((m, n), dtype=np.float32)
    D, _ = vm_sgemm(name, A, B, C, 1.0, 1.0)
    exact = np.array(case["d_colmajor"], dtype=np.float64).reshape(n, m).T
    assert np.allclose(D, exact, rtol=1e-5)


@pytest.mark.parametrize("name", ["mt64x64_a32_wg2x2_dk16", "mt128x64_a32_wg4x1_dk8_s3", "mt64x64_a16_wg2x2_dk8",
                                  "mt16x16_a16_wg1x1_dk16_mapk4", "mt64x64_a32_wg1x1_dk16",
                                  "mt128x64_a16_wg4x1_dk32", "mt64x64_a32_wg2x2_dk16_gw0"])
def test_multi_wave_and_knob_variants_in_vm(name):
    _, cfg = program(name)
    t0, t1 = cfg.tile_size
    m, n, k = 2 * t0, 2 * t1, 3 * cfg.depth_k
    A = oracle.fill_matrix(m, k, 4, 0)
    B = oracle.fill_matrix(k, n, 4, 1)
    C = oracle.fill_matrix(m, n, 4, 2)
    D, _ = vm_sgemm(name, A, B, C, 0.5, -1.25)
    assert oracle.normwise_error(D, oracle.gemm_f64(A, B, C, 0.5, -1.25)) <= oracle.tolerance(k)


def test_beta_zero_does_not_read_c_in_vm():
    m = n = 32
    k = 16
    A = oracle.fill_matrix(m, k, 1, 0)
    B = oracle.fill_matrix(k, n, 1, 1)
    C = np.full((m, n), np.nan, dtype=np.float32)
    D, _ = vm_sgemm("mt32x32_a32_wg1x1_dk16", A, B, C, 1.0, 0.0)
    assert np.all(np.isfinite(D))


def test_map_k_and_stages_invariance_in_vm():
    # reference test_vm.py:743-963: M=64, N=48, K=64, same D for map_k_idx=4 and vmem_stage=2
    m, n, k = 64, 48, 64
    A = np.arange(m * k, dtype=np.float32).reshape(k, m).T / 64
    B = np.arange(k * n, dtype=np.float32).reshape(n, k).T / 64
    C = np.ones((m, n), dtype=np.float32)
    exact = A.astype(np.float64) @ B.astype(np.float64) + 1.0
    for name in ("mt16x16_a16_wg1x1_dk16", "mt16x16_a16_wg1x1_dk16_mapk4", "mt16x16_a16_wg1x1_dk16_s3"):
        D, _ = vm_sgemm(name, A, B, C, 1.0, 1.0)
        assert np.allclose(D, exact, rtol=1e-5), name


# ------------------------------------------------------ work-group order
def _tile_owner_map(name, nwgx, nwgy):
    """Runs every work-group and records which D tile each one wrote."""
    prog, cfg = program(name)
    t0, t1 = cfg.tile_size
    m, n, k = nwgx * t0, nwgy * t1, cfg.depth_k
    A = np.ones((m, k), dtype=np.float32, order="F")
    B = np.ones((k, n), dtype=np.float32, order="F")
    mem = V.Memory(256 + 4 * (m * k + k * n + m * n) + 512, "vmem")
    offs = [256, 256 + 4 * m * k, 256 + 4 * (m * k + k * n)]
    mem.write_bytes(offs[0], A.ravel(order="F").tobytes())
    mem.write_bytes(offs[1], B.ravel(order="F").tobytes())
    ka = pack_kernargs(offs[0], offs[1], 0, offs[2], m, n, k, m, k, m, m, 1.0, 0.0, nwgx, nwgy)
    owner = {}
    seen = np.zeros((m, n), dtype=bool)

    def on_wg(wx, wy, waves):
        D = np.frombuffer(mem.read_bytes(offs[2], 4 * m * n), dtype=np.float32).reshape(n, m).T
        new = (D != 0) & ~seen
        rows, cols = np.nonzero(new)
        assert rows.size == t0 * t1, f"work-group ({wx},{wy}) wrote {rows.size} values"
        tx, ty = rows.min() // t0, cols.min() // t1
        assert rows.max() // t0 == tx and cols.max() // t1 == ty
        owner[(wx, wy)] = (int(tx), int(ty))
        seen[new] = True

    run_kernel(prog, (nwgx, nwgy), cfg.num_workitems, ka, mem, on_workgroup=on_wg)
    assert seen.all()
    return owner


def test_wgm_remap_matches_reference_closed_form():
    golden = json.load(open(os.path.join(GOLDEN, "wgm_8x8_wgm4.json")))
    owner = _tile_owner_map("mt16x16_a16_wg1x1_dk16_wgm4", golden["nwgx"], golden["nwgy"])
    for wx, wy, ex, ey in golden["map"]:
        assert owner[(wx, wy)] == (ex, ey), (wx, wy)


def test_xcd_and_wgm_order_is_a_bijection_with_contiguous_xcd_ranges():
    # mt64x64_a32_wg1x1_dk16: xcd=8, wgm=8 on a 4 x 4 grid (16 tiles, 2 per XCD)
    owner = _tile_owner_map("mt64x64_a32_wg1x1_dk16", 4, 4)
    assert sorted(owner.values()) == [(x, y) for x in range(4) for y in range(4)]
    # hardware id z runs on XCD z % 8; logical order z' = (z % 8) * 2 + z // 8, then
    # grouped 8 tiles wide along M (one group: x' = z' % 4 ... of a 4-wide grid)
    for (wx, wy), (tx, ty) in owner.items():
        z = wx + 4 * wy
        zl = (z % 8) * 2 + z // 8
        width = 4
        assert (tx, ty) == (zl % width, zl // width)
    # 15 tiles on 8 XCDs: XCD x owns 15 // 8 = 1 tile, plus one more for x < 7,
    # starting at x * 1 + min(x, 7) in the logical order
    owner = _tile_owner_map("mt64x64_a32_wg1x1_dk16", 3, 5)
    assert sorted(owner.values()) == [(x, y) for x in range(3) for y in range(5)]
    for (wx, wy), (tx, ty) in owner.items():
        z = wx + 3 * wy
        zl = (z % 8) * 1 + min(z % 8, 7) + z // 8
        assert (tx, ty) == (zl % 3, zl // 3)


# ------------------------------------------- the checker catches mistakes
def test_dropping_a_wait_is_caught():
    prog, cfg = program("mt32x32_a32_wg1x1_dk16")
    insts = [i for i in prog.insts]
    # the wait that makes the first MFMA's LDS operands arrive
    waits = [j for j, i in enumerate(insts[:-1]) if i.mnemonic == "s_waitcnt" and "lgkmcnt" in i.mods
             and insts[j + 1].mnemonic.startswith("v_mfma")]
    assert waits
    broken = V.Program([i for j, i in enumerate(insts) if j != waits[0]], {}, prog.desc)
    # labels move with the removed instruction
    broken.labels = {l: (p if p <= waits[0] else p - 1) for l, p in prog.labels.items()}
    m = n = 32
    k = 32
    A = oracle.fill_matrix(m, k, 0, 0)
    B = oracle.fill_matrix(k, n, 0, 1)
    # the missing wait must surface: either as a wrong result, or as an LDS
    # access through a register the skipped read had not filled yet
    try:
        D, _ = run_sgemm(broken, cfg.tile_size, cfg.num_workitems, A, B)
    except MemoryError:
        return
    assert oracle.normwise_error(D, oracle.gemm_f64(A, B)) > oracle.tolerance(k)


def test_a_transposed_mfma_layout_is_caught(monkeypatch):
    rows, cols = V._ACC_INDEX[32]
    monkeypatch.setitem(V._ACC_INDEX, 32, (cols, rows))
    m = n = k = 32
    A = oracle.fill_matrix(m, k, 0, 0)
    B = oracle.fill_matrix(k, n, 0, 1)
    D, _ = vm_sgemm("mt32x32_a32_wg1x1_dk16", A, B)
    assert oracle.normwise_error(D, oracle.gemm_f64(A, B)) > oracle.tolerance(k)


EDGE_CASES = [  # (instance, m, n, k): partial tiles in M and N, K remainders, k < DK, tiny problems
    ("mt32x32_a32_wg1x1_dk16", 35, 59, 33), ("mt32x32_a32_wg1x1_dk16", 5, 3, 1),
    ("mt64x64_a16_wg2x2_dk32_s3", 67, 123, 65), ("mt64x64_a16_wg2x2_dk32_s3", 128, 64, 29),
    ("mt128x64_a32_wg4x1_dk8_s3", 131, 123, 17), ("mt16x16_a16_wg1x1_dk16_s3_plr3", 15, 17, 48),
    ("mt64x64_a32_wg1x1_dk16", 63, 65, 48),
    ("mt256x128_a32_wg2x2_dk16", 250, 100, 40),  # the epilogue without an LDS stage
    ("mt256x128_a32_wg2x2_dk16_s3_occ2", 300, 200, 37),  # the 4096^3 instance
]


@pytest.mark.parametrize("name,m,n,k", EDGE_CASES)
@pytest.mark.parametrize("pad", [0, 1])
def test_edge_shapes_stay_inside_every_buffer(name, m, n, k, pad):
    """Arbitrary shapes: each of A, B, C, D is its own guarded region in the VM,
    so any read or write outside the matrices raises MemoryError.  pad = 1 makes
    every leading dimension odd and every buffer start 4 bytes past a 16-byte
    boundary."""
    prog, cfg = program(name)
    lda, ldb, ldc, ldd = m + pad, k + pad, m + 2 * pad, m + 3 * pad
    A = oracle.fill_matrix(lda, k, 3, 0)
    B = oracle.fill_matrix(ldb, n, 3, 1)
    C = oracle.fill_matrix(ldc, n, 3, 2)
    D, _ = run_sgemm(prog, cfg.tile_size, cfg.num_workitems, A, B, C, 0.5, 1.5, mnk=(m, n, k), ldd=ldd,
                     misalign=4 * pad)
    ref = oracle.gemm_f64(A[:m, :k], B[:k, :n], C[:m, :n], 0.5, 1.5)
    assert oracle.normwise_error(D[:m, :n], ref) <= oracle.tolerance(k)
    assert np.all(D[m:, :] == 0), "rows past m of D were written"


VECTOR_CASES = [  # (instance, m, n, k, pad, misalign): every shape takes the vector path
    ("mt64x64_a16_wg2x2_dk32_s3", 100, 70, 64, 0, 0), ("mt32x32_a32_wg1x1_dk16", 36, 40, 48, 0, 0),
    ("mt64x64_a16_wg2x2_dk32_s3_tn", 100, 70, 64, 0, 0), ("mt32x32_a32_wg1x1_dk16_tt", 36, 44, 48, 0, 0),
    ("mt16x16_a16_wg1x1_dk16_nt", 20, 36, 32, 0, 0),
    ("mt64x64_a16_wg2x2_dk32_s3", 100, 70, 100, 0, 0),   # and a K remainder (shifted K origin)
    # unaligned: m % 4 != 0, odd leading dimensions, dword-aligned pointers
    ("mt64x64_a16_wg2x2_dk32_s3", 99, 70, 64, 1, 4), ("mt32x32_a32_wg1x1_dk16", 35, 59, 66, 1, 8),
    ("mt64x64_a16_wg2x2_dk32_s3_tn", 101, 70, 67, 3, 12), ("mt32x32_a32_wg1x1_dk16_tt", 37, 45, 50, 1, 4),
    ("mt16x16_a16_wg1x1_dk16_nt", 21, 37, 35, 2, 4), ("mt64x64_a16_wg2x2_dk32_s3", 64, 64, 97, 1, 0),
    ("mt256x128_a32_wg2x2_dk16_s3_occ2", 256, 128, 100, 0, 0),   # the 4096^3 instance, K remainder
]


@pytest.mark.parametrize("name,m,n,k,pad,misalign", VECTOR_CASES)
def test_any_shape_keeps_the_vector_path(name, m, n, k, pad, misalign):
    """Every shape takes the vector path: chunks wholly past the edge load a
    chunk of the tile's first row or column, a chunk straddling the end of an
    operand reads 0 past it (per-dword buffer range check), a K remainder moves
    the K origin back (elementwise loads in the first K tile when it straddles
    a chunk along k), and the epilogue stores only elements inside D.  Every
    buffer is guarded, rows past m of D (ldd > m) must stay untouched, and the
    launch runs about as many instructions as the same grid of whole tiles."""
    prog, cfg = program(name)
    t0, t1 = cfg.tile_size
    ldd = m + 4 + pad
    A, B, C, opA, opB = _split_operands(cfg, m, n, k, 9, pad)
    D, info = run_sgemm(prog, cfg.tile_size, cfg.num_workitems, A, B, C, 0.5, 1.5, mnk=(m, n, k), ldd=ldd,
                        misalign=misalign)
    assert oracle.normwise_error(D[:m, :n], oracle.gemm_f64(opA, opB, C[:m, :n], 0.5, 1.5)) <= oracle.tolerance(k)
    assert np.all(D[m:, :] == 0), "rows past m of D were written"
    mw, nw = -(-m // t0) * t0, -(-n // t1) * t1
    kw = -(-k // cfg.depth_k) * cfg.depth_k
    A2, B2, C2, _, _ = _split_operands(cfg, mw, nw, kw, 9)
    _, info2 = run_sgemm(prog, cfg.tile_size, cfg.num_workitems, A2, B2, C2, 0.5, 1.5, mnk=(mw, nw, kw), ldd=mw)
    assert info["grid"] == info2["grid"]
    # (edge tiles run the epilogue with bounds checks, and a K remainder that
    # straddles a chunk along k costs one element-wise first K tile: up to
    # 25% more at these few K tiles; the element-wise path for the whole
    # launch runs two to three times as many)
    assert info["instructions"] <= 1.3 * info2["instructions"], (info["instructions"], info2["instructions"])


HEAD_CASES = [  # whole, aligned tiles with k % DK != 0 and k % 4 == 0 (instances without a K rotation)
    ("mt32x32_a32_wg1x1_dk16", 64, 32, 20), ("mt64x64_a16_wg2x2_dk32_s3", 128, 64, 36),
    ("mt64x64_a16_wg2x2_dk8", 128, 64, 12), ("mt16x16_a16_wg1x1_dk16_s3", 32, 16, 52),
    ("mt32x32_a32_wg1x1_dk16_s2_pd2", 64, 32, 36),
    ("mt64x64_a16_wg2x2_dk32_s3_tn", 64, 64, 36), ("mt32x32_a32_wg1x1_dk16_tt", 32, 64, 20),
]


@pytest.mark.parametrize("name,m,n,k", HEAD_CASES)
def test_k_remainder_keeps_the_vector_path(name, m, n, k):
    """A K remainder moves the K origin back so that the first K tile is the
    partial one, loaded with its missing values as zeros: parity against f64
    with every buffer guarded, and about as many instructions as the same
    launch with K rounded up to whole tiles (the element-wise path would run
    several times as many)."""
    prog, cfg = program(name)
    dk = cfg.depth_k
    assert k % dk and k % 4 == 0 and k > dk
    A, B, C, opA, opB = _split_operands(cfg, m, n, k, 7)
    D, info = run_sgemm(prog, cfg.tile_size, cfg.num_workitems, A, B, C, 0.5, 1.5, mnk=(m, n, k), ldd=m)
    assert oracle.normwise_error(D, oracle.gemm_f64(opA, opB, C, 0.5, 1.5)) <= oracle.tolerance(k)
    kr = -(-k // dk) * dk
    A2, B2, C2, _, _ = _split_operands(cfg, m, n, kr, 7)
    _, info2 = run_sgemm(prog, cfg.tile_size, cfg.num_workitems, A2, B2, C2, 0.5, 1.5, mnk=(m, n, kr), ldd=m)
    # (the first K tile's selects cost up to 15% at two or three K tiles)
    assert info["instructions"] <= 1.15 * info2["instructions"], (info["instructions"], info2["instructions"])


@pytest.mark.parametrize("name", ["mt32x32_a32_wg1x1_dk16_tt", "mt16x16_a16_wg1x1_dk16_nt",
                                  "mt64x64_a16_wg2x2_dk32_s3_tn", "mt128x64_a16_wg2x2_dk32_s3_tt"])
@pytest.mark.parametrize("shape,pad", [((None, None, None), 0), ((35, 59, 33), 1), ((5, 3, 1), 0)])
def test_transposed_layouts_in_vm(name, shape, pad):
    """op(A) = A^T and/or op(B) = B^T, with guarded buffers; the first and
    last instances store A^T's rows swizzled (one row per lane, and four
    atoms' rows per lane)."""
    if name.endswith("_tt"):
        assert catalog.SOLUTIONS[name][0].lds_a_row_swizzle[1] > 0
    prog, cfg = program(name)
    t0, t1 = cfg.tile_size
    m, n, k = (2 * t0, 2 * t1, 3 * cfg.depth_k) if shape[0] is None else shape
    ra, ca = (k, m) if cfg.trans_a else (m, k)
    rb, cb = (n, k) if cfg.trans_b else (k, n)
    A = oracle.fill_matrix(ra + pad, ca, 4, 0)
    B = oracle.fill_matrix(rb + pad, cb, 4, 1)
    C = oracle.fill_matrix(m, n, 4, 2)
    D, _ = run_sgemm(prog, cfg.tile_size, cfg.num_workitems, A, B, C, 0.5, 1.5, mnk=(m, n, k), ldd=m)
    opA = A[:ra, :ca].T if cfg.trans_a else A[:m, :k]
    opB = B[:rb, :cb].T if cfg.trans_b else B[:k, :n]
    assert oracle.normwise_error(D[:m, :n], oracle.gemm_f64(opA, opB, C, 0.5, 1.5)) <= oracle.tolerance(k)


# ------------------------------------------------------------- split-K
SPLIT_CASES = [
    ("mt32x32_a32_wg1x1_dk16_s3_sk4", 70, 45, 16 * 7 + 5, 3),   # ragged M, N, K
    ("mt32x32_a32_wg1x1_dk16_s3_sk4", 32, 64, 16 * 2, 4),       # ranges 2 and 3 are empty
    ("mt32x32_a32_wg1x1_dk16_s3_sk4", 40, 33, 16 * 16, 16),     # the largest split count
    ("mt64x64_a16_wg2x2_dk32_s3", 64, 70, 32 * 5, 5),           # a tuned instance, four waves
    ("mt32x32_a32_wg1x1_dk16_sk4_tt", 33, 31, 16 * 6 + 1, 3),   # op(A) = A^T, op(B) = B^T
]


SPLIT_UNALIGNED_CASES = [  # (instance, m, n, k, splits, pad, misalign)
    ("mt32x32_a32_wg1x1_dk16_s3_sk4", 45, 37, 16 * 5 + 3, 3, 1, 4),   # last range's first tile element-wise
    ("mt64x64_a16_wg1x4_dk32_s3", 67, 65, 32 * 4 + 6, 2, 3, 12),      # the split-K instance of the catalog
    ("mt32x32_a32_wg1x1_dk16_sk4_tt", 35, 33, 16 * 4 + 9, 4, 1, 8),   # transposed operands
]


@pytest.mark.parametrize("name,m,n,k,splits,pad,misalign", SPLIT_UNALIGNED_CASES)
def test_split_k_unaligned_in_vm(name, m, n, k, splits, pad, misalign):
    """generated_gemm_splitk with odd leading dimensions, buffers starting
    4-12 bytes past a 16-byte boundary and a K remainder that shifts the last
    range's K origin: f64 parity with every buffer guarded, rows past m of D
    untouched, tickets re-armed."""
    prog, cfg = program(name, "generated_gemm_splitk")
    A, B, C, opA, opB = _split_operands(cfg, m, n, k, 8, pad)
    D, info = run_sgemm(prog, cfg.tile_size, cfg.num_workitems, A, B, C, 0.5, 1.5, mnk=(m, n, k),
                        ldd=m + 2 + pad, splits=splits, misalign=misalign)
    assert oracle.normwise_error(D[:m, :n], oracle.gemm_f64(opA, opB, C[:m, :n], 0.5, 1.5)) <= oracle.tolerance(k)
    assert np.all(D[m:, :] == 0), "rows past m of D were written"
    assert not info["tickets"].any()


def _split_operands(cfg, m, n, k, seed, pad=0):
    """Stored A, B, C (each with ``pad`` extra rows: leading dimensions past the
    matrix) and op(A), op(B) as m x k and k x n."""
    ra, ca = (k, m) if cfg.trans_a else (m, k)
    rb, cb = (n, k) if cfg.trans_b else (k, n)
    A = oracle.fill_matrix(ra + pad, ca, seed, 0)
    B = oracle.fill_matrix(rb + pad, cb, seed, 1)
    C = oracle.fill_matrix(m + pad, n, seed, 2)
    opA = A[:ra].T if cfg.trans_a else A[:ra]
    opB = B[:rb].T if cfg.trans_b else B[:rb]
    return A, B, C, opA, opB


@pytest.mark.parametrize("name,m,n,k,splits", SPLIT_CASES)
def test_split_k_in_vm(name, m, n, k, splits):
    """generated_gemm_splitk: every (tile, K range) work-group writes a partial,
    the tile's last arrival sums them in range order and runs the epilogue.
    The sum must not depend on which work-group arrives last (the VM runs the
    grid in three different orders), and every ticket is re-armed to 0."""
    prog, cfg = program(name, "generated_gemm_splitk")
    A, B, C, opA, opB = _split_operands(cfg, m, n, k, 6)
    D, info = run_sgemm(prog, cfg.tile_size, cfg.num_workitems, A, B, C, 0.5, 1.5, mnk=(m, n, k), ldd=m,
                        splits=splits)
    assert oracle.normwise_error(D, oracle.gemm_f64(opA, opB, C, 0.5, 1.5)) <= oracle.tolerance(k)
    assert not info["tickets"].any()
    groups = [(x, y, z) for z in range(splits) for y in range(info["grid"][1]) for x in range(info["grid"][0])]
    rng = np.random.default_rng(0)
    for order in (groups[::-1], [groups[i] for i in rng.permutation(len(groups))]):
        D2, info2 = run_sgemm(prog, cfg.tile_size, cfg.num_workitems, A, B, C, 0.5, 1.5, mnk=(m, n, k), ldd=m,
                              splits=splits, order=order)
        assert np.array_equal(D2, D) and not info2["tickets"].any()


# ------------------------------------------------------------- stream-K
STREAM_CASES = [
    # (instance, m, n, k, groups): T tiles over G work-groups, stream-K tiles T % G + G
    ("mt32x32_a32_wg1x1_dk16_s3_stk", 96, 96, 16 * 7 + 5, 4),     # 9 tiles: 5 streamed, 4 whole; K remainder
    ("mt32x32_a32_wg1x1_dk16_s3_stk", 70, 45, 100, 4),            # 6 ragged tiles, all streamed
    ("mt32x32_a32_wg1x1_dk16_s3_stk", 33, 200, 40, 3),            # 14 tiles of 3 K tiles, 5 streamed
    ("mt32x32_a16_wg2x2_dk16_stk_tn", 64, 96, 50, 5),             # A^T, four waves, 6 tiles
]


@pytest.mark.parametrize("name,m,n,k,groups", STREAM_CASES)
def test_stream_k_in_vm(name, m, n, k, groups):
    """generated_gemm_streamk: the K iterations of the last partial round plus
    one whole round of tiles are cut into `groups` equal runs, a tile cut at a
    run boundary gets a head and a tail partial, and the later of the two
    work-groups adds them.  Checked against float64, with every ticket re-armed,
    and bit-identical whatever order the work-groups run in (the two-term sum
    is commutative)."""
    prog, cfg = program(name, "generated_gemm_streamk")
    t0, t1 = cfg.tile_size
    tiles = -(-m // t0) * -(-n // t1)
    sk = catalog.stream_k_tiles(tiles, groups, k, mode=2)
    assert groups <= sk <= tiles and (tiles - sk) % groups == 0
    A, B, C, opA, opB = _split_operands(cfg, m, n, k, 8)
    D, info = run_sgemm(prog, cfg.tile_size, cfg.num_workitems, A, B, C, 0.5, 1.5, mnk=(m, n, k), ldd=m,
                        stream_k=(groups, sk))
    assert oracle.normwise_error(D, oracle.gemm_f64(opA, opB, C, 0.5, 1.5)) <= oracle.tolerance(k)
    assert not info["tickets"].any()
    rng = np.random.default_rng(1)
    order = [(x, 0, 0) for x in range(groups)]
    for o in (order[::-1], [order[i] for i in rng.permutation(groups)]):
        D2, info2 = run_sgemm(prog, cfg.tile_size, cfg.num_workitems, A, B, C, 0.5, 1.5, mnk=(m, n, k), ldd=m,
                              stream_k=(groups, sk), order=o)
        assert np.array_equal(D2, D) and not info2["tickets"].any()


def test_stream_k_without_cuts_equals_the_plain_kernel():
    """T = 2 G tiles with G stream-K tiles: every run is exactly one tile, so no
    tile is cut and each is computed over its whole K like the plain kernel --
    the same bits."""
    name = "mt32x32_a32_wg1x1_dk16_s3_stk"
    plain, cfg = program(name)
    sk, _ = program(name, "generated_gemm_streamk")
    A, B, C, _, _ = _split_operands(cfg, 128, 64, 83, 9)          # 8 tiles
    D1, _ = run_sgemm(plain, cfg.tile_size, cfg.num_workitems, A, B, C, 0.5, 1.5)
    D2, info = run_sgemm(sk, cfg.tile_size, cfg.num_workitems, A, B, C, 0.5, 1.5, stream_k=(4, 4))
    assert np.array_equal(D1, D2) and not info["tickets"].any()


def test_stream_k_plan_rule():
    """The host rule (sgemm_set_stream_k): no stream-K until tiles exceed the
    groups, auto mode only when the partial last round costs >= 3%."""
    assert catalog.stream_k_tiles(512, 512, 4096) == 0           # one whole round
    assert catalog.stream_k_tiles(722, 512, 4096) == 722 - 512 + 512
    assert catalog.stream_k_tiles(1000, 512, 4096) == 0           # 2 rounds vs 1.95: under 3%
    assert catalog.stream_k_tiles(1000, 512, 4096, mode=2) == 1000 - 512 + 0 if False else 488 + 512
    assert catalog.stream_k_tiles(1024, 512, 4096, mode=2) == 512  # whole rounds, forced
    assert catalog.stream_k_tiles(100, 512, 4096, mode=2) == 0     # fewer tiles than groups: split-K's case
    assert catalog.stream_k_tiles(722, 512, 0) == 0 and catalog.stream_k_tiles(722, 512, 64, mode=0) == 0


def test_split_k_with_one_range_equals_the_plain_kernel():
    name = "mt32x32_a32_wg1x1_dk16_s3_sk4"
    plain, cfg = program(name)
    split, _ = program(name, "generated_gemm_splitk")
    A, B, C, _, _ = _split_operands(cfg, 45, 37, 83, 7)
    D1, _ = run_sgemm(plain, cfg.tile_size, cfg.num_workitems, A, B, C, 0.5, 1.5)
    D2, _ = run_sgemm(split, cfg.tile_size, cfg.num_workitems, A, B, C, 0.5, 1.5, splits=1)
    assert np.array_equal(D1, D2)


def test_split_k_sums_partials_in_range_order():
    """Partials 2^24, 1 and -2^24 (one nonzero row of B per K range): in range
    order (2^24 + 1) rounds to 2^24 and the sum is exactly 0; every other
    association (for instance starting from the last arrival's own partial)
    gives 1."""
    prog, cfg = program("mt32x32_a32_wg1x1_dk16_s3_sk4", "generated_gemm_splitk")
    m, n, k = 32, 32, 48
    A = np.ones((m, k), dtype=np.float32)
    B = np.zeros((k, n), dtype=np.float32)
    B[0, :], B[16, :], B[32, :] = 2.0 ** 24, 1.0, -(2.0 ** 24)
    for order in (None, [(0, 0, 2), (0, 0, 1), (0, 0, 0)], [(0, 0, 1), (0, 0, 2), (0, 0, 0)]):
        D, _ = run_sgemm(prog, cfg.tile_size, cfg.num_workitems, A, B, None, 1.0, 0.0, splits=3, order=order)
        assert np.array_equal(D, np.zeros((m, n), dtype=np.float32)), order


def test_vm_buffer_access_is_range_checked_like_the_hardware():
    """MUBUF with a raw resource: loads past num_records read 0, stores past
    it are dropped (per access)."""
    vm = GcnVirtualMachine(104, 256, 64)
    mem = V.Memory(8192, "vmem")
    mem.allocate_region(4096, 1024, "buf")
    mem.write_bytes(4096, np.arange(256, dtype=np.float32).tobytes())
    vm.vmem = mem
    vm.s[8], vm.s[9], vm.s[10], vm.s[11] = 4096, 0, 512, 0x20000   # 128 floats in range
    vm.v[1] = (np.arange(64, dtype=np.uint32) * 16)                  # lane l: float4 at l*16 bytes
    vm.v[10] = np.full(64, fbits(-1.0), dtype=np.uint32)
    vm.run("generated_gemm:\n buffer_load_dwordx4 v[2:5], v1, s[8:11], 0 offen sc1\n s_waitcnt vmcnt(0)\n"
           " buffer_store_dword v10, v1, s[8:11], 4 offen\n s_waitcnt vmcnt(0)\n s_endpgm\n")
    got = np.stack([vm.v[2 + i].view(np.float32) for i in range(4)], axis=1)
    want = np.zeros((64, 4), dtype=np.float32)
    want[:32] = np.arange(128, dtype=np.float32).reshape(32, 4)
    assert np.array_equal(got, want)
    after = np.frombuffer(mem.read_bytes(4096, 1024), dtype=np.float32)
    assert np.all(after[1:128:4] == -1.0) and np.array_equal(after[128:], np.arange(128, 256, dtype=np.float32))


def test_vm_buffer_range_check_is_per_dword():
    """The range check is per dword, as measured on an MI355X with a probe
    kernel (dwords 1000 + i, num_records = 20 bytes, lane l loading a dwordx4 at
    byte 4*l): a load straddling num_records keeps its in-range dwords and
    reads 0 for the rest; dword-aligned (not 16-byte aligned) dwordx4 loads
    read the dwords at their address.  Stores follow the same per-dword rule
    here (the kernels never issue a store that straddles its range)."""
    measured = [[1000, 1001, 1002, 1003], [1001, 1002, 1003, 1004], [1002, 1003, 1004, 0], [1003, 1004, 0, 0],
                [1004, 0, 0, 0], [0, 0, 0, 0], [0, 0, 0, 0], [0, 0, 0, 0]]
    vm = GcnVirtualMachine(104, 256, 64)
    mem = V.Memory(1024, "vmem")
    mem.write_bytes(0, (1000 + np.arange(256, dtype=np.uint32)).tobytes())
    vm.vmem = mem
    vm.s[8], vm.s[9], vm.s[10], vm.s[11] = 0, 0, 20, 0x20000
    vm.v[1] = np.arange(64, dtype=np.uint32) * 4
    vm.exec = 0xFF
    vm.run("generated_gemm:\n buffer_load_dwordx4 v[2:5], v1, s[8:11], 0 offen\n s_waitcnt vmcnt(0)\n s_endpgm\n")
    got = [[int(vm.v[2 + i][lane]) for i in range(4)] for lane in range(8)]
    assert got == measured
    # a store straddling num_records: lane 0 stores 4 dwords at byte 12, only the first two land
    vm.v[6], vm.v[7], vm.v[8], vm.v[9] = (np.full(64, x, dtype=np.uint32) for x in (7, 8, 9, 10))
    vm.v[1] = np.full(64, 12, dtype=np.uint32)
    vm.s[10] = 20
    vm.exec = 0x1
    vm.run("generated_gemm:\n buffer_store_dwordx4 v[6:9], v1, s[8:11], 0 offen\n s_waitcnt vmcnt(0)\n s_endpgm\n")
    after = np.frombuffer(mem.read_bytes(0, 32), dtype=np.uint32).tolist()
    assert after == [1000, 1001, 1002, 7, 8, 1005, 1006, 1007]
    # a register offset whose sum with the instruction's offset field passes
    # 2^32 (a "negative" register part): which offset the hardware range-checks
    # is not modelled, so the VM refuses it; the kernels write such offsets as
    # one expression with no constant split off
    vm.v[1] = np.full(64, 0xFFFFFFF8, dtype=np.uint32)
    vm.exec = 0x1
    with pytest.raises(NotImplementedError, match="past 32 bits"):
        vm.run("generated_gemm:\n buffer_load_dword v2, v1, s[8:11], 0 offen offset:8\n s_endpgm\n")
    # a lane outside EXEC does not count
    vm.exec = 0x2
    vm.v[1] = np.array([0xFFFFFFF8] + [0] * 63, dtype=np.uint32)
    vm.run("generated_gemm:\n buffer_load_dword v2, v1, s[8:11], 0 offen offset:8\n s_waitcnt vmcnt(0)\n s_endpgm\n")


# ------------------------------------------- memory instruction KATs
# The reference's per-instruction memory tests (test_vm.py:187-407): buffer
# loads and stores of 1, 2 and 4 dwords, LDS reads and writes of 32, 64 and
# 128 bits, scalar loads of 1, 2 and 4 dwords.  Here every dword of every
# lane is a distinct random word and lanes address memory through a random
# permutation, so a swapped dword order, a wrong lane stride, a dropped dword
# or a lane mix-up fails; a copy taken before the s_waitcnt must still hold
# the old register value (results land at the wait), and lanes outside EXEC
# neither load nor store.
_WIDTHS = [(1, "dword", "b32"), (2, "dwordx2", "b64"), (4, "dwordx4", "b128")]


def _words(count, seed):
    return np.random.default_rng(seed).integers(0, 2 ** 32, size=count, dtype=np.uint64).astype(np.uint32)


@pytest.mark.parametrize("nd,sfx,_", _WIDTHS)
def test_buffer_load_widths_known_answer(nd, sfx, _):
    stride = 4 * nd
    words = _words(64 * nd, 10 + nd)
    perm = np.random.default_rng(20 + nd).permutation(64)
    vm = GcnVirtualMachine(104, 256, 64)
    mem = V.Memory(8192, "vmem")
    mem.allocate_region(4096, 64 * stride, "buf")
    mem.write_bytes(4096, words.tobytes())
    vm.vmem = mem
    # base 16 bytes before the buffer; soffset 8 and the offset field 8 bring it back
    vm.s[8], vm.s[9], vm.s[10], vm.s[11] = 4096 - 16, 0, 64 * stride + 16, 0x20000
    vm.s[12] = 8
    vm.v[0] = (perm * stride).astype(np.uint32)
    vm.v[2:2 + nd] = 0xDEADBEEF
    dst = f"v[2:{1 + nd}]" if nd > 1 else "v2"
    vm.exec = 0xFFFF_FFFF_0000_FFFF
    vm.run(f"generated_gemm:\n buffer_load_{sfx} {dst}, v0, s[8:11], s12 offen offset:8\n"
           f" v_mov_b32 v30, v2\n s_waitcnt vmcnt(0)\n s_endpgm\n")
    live = vm.exec_mask()
    want = words.reshape(64, nd)[perm].T          # [dword][lane]
    for i in range(nd):
        assert np.array_equal(vm.v[2 + i][live], want[i][live]), i
        assert np.all(vm.v[2 + i][~live] == 0xDEADBEEF), i
    assert np.all(vm.v[30][live] == 0xDEADBEEF)   # read before the wait: the old value


@pytest.mark.parametrize("nd,sfx,_", _WIDTHS)
def test_buffer_store_widths_known_answer(nd, sfx, _):
    stride = 4 * nd
    words = _words(64 * nd, 30 + nd).reshape(nd, 64)
    perm = np.random.default_rng(40 + nd).permutation(64)
    vm = GcnVirtualMachine(104, 256, 64)
    mem = V.Memory(8192, "vmem")
    mem.allocate_region(4096, 64 * stride, "buf")
    mem.write_bytes(4096, np.full(64 * nd, 0x5A5A5A5A, dtype=np.uint32).tobytes())
    vm.vmem = mem
    vm.s[8], vm.s[9], vm.s[10], vm.s[11] = 4096, 0, 64 * stride, 0x20000
    vm.v[0] = (perm * stride).astype(np.uint32)
    vm.v[2:2 + nd] = words
    src = f"v[2:{1 + nd}]" if nd > 1 else "v2"
    vm.exec = 0x0F0F_0F0F_FFFF_FFFF
    vm.run(f"generated_gemm:\n buffer_store_{sfx} {src}, v0, s[8:11], 0 offen\n s_waitcnt vmcnt(0)\n s_endpgm\n")
    got = np.frombuffer(mem.read_bytes(4096, 64 * stride), dtype=np.uint32).reshape(64, nd)
    live = vm.exec_mask()
    for lane in range(64):
        slot = got[perm[lane]]
        if live[lane]:
            assert np.array_equal(slot, words[:, lane]), lane
        else:
            assert np.all(slot == 0x5A5A5A5A), lane


@pytest.mark.parametrize("nd,_,sfx", _WIDTHS)
def test_ds_write_then_read_widths_known_answer(nd, _, sfx):
    stride = 4 * nd
    words = _words(64 * nd, 50 + nd).reshape(nd, 64)
    perm = np.random.default_rng(60 + nd).permutation(64)
    vm = GcnVirtualMachine(104, 256, 64)
    vm.v[0] = (perm * stride).astype(np.uint32)
    vm.v[2:2 + nd] = words
    src = f"v[2:{1 + nd}]" if nd > 1 else "v2"
    dst = f"v[10:{9 + nd}]" if nd > 1 else "v10"
    vm.run(f"generated_gemm:\n ds_write_{sfx} v0, {src} offset:64\n s_waitcnt lgkmcnt(0)\n s_endpgm\n")
    lds = np.frombuffer(bytes(vm.lds.mem[64:64 + 64 * stride]), dtype=np.uint32).reshape(64, nd)
    for lane in range(64):
        assert np.array_equal(lds[perm[lane]], words[:, lane]), lane
    # read back through a different permutation: lane l gets slot q[l]
    q = np.random.default_rng(70 + nd).permutation(64)
    vm.v[1] = (q * stride).astype(np.uint32)
    vm.v[10:10 + nd] = 0xDEADBEEF
    vm.run(f"generated_gemm:\n ds_read_{sfx} {dst}, v1 offset:64\n v_mov_b32 v30, v10\n"
           f" s_waitcnt lgkmcnt(0)\n s_endpgm\n")
    for i in range(nd):
        assert np.array_equal(vm.v[10 + i], lds[q, i]), i
    assert np.all(vm.v[30] == 0xDEADBEEF)


@pytest.mark.parametrize("nd,sfx", [(1, "dword"), (2, "dwordx2"), (4, "dwordx4")])
def test_s_load_widths_known_answer(nd, sfx):
    words = _words(64, 80 + nd)
    vm = GcnVirtualMachine(104, 256, 64)
    vm.smem.write_bytes(0, words.tobytes())
    vm.s[0], vm.s[1] = 32, 0               # pointer 32 bytes in, offset field 0x10
    vm.s[4:4 + nd] = 0xDEADBEEF
    dst = f"s[4:{3 + nd}]" if nd > 1 else "s4"
    vm.run(f"generated_gemm:\n s_load_{sfx} {dst}, s[0:1], 0x10\n s_mov_b32 s30, s4\n"
           f" s_waitcnt lgkmcnt(0)\n s_endpgm\n")
    assert vm.s[4:4 + nd].tolist() == words[12:12 + nd].tolist()
    assert vm.s[30] == 0xDEADBEEF


def test_readlane_and_writelane_ignore_exec():
    """v_writelane_b32 / v_readlane_b32 (the compiler's way of parking scalar
    registers in vector lanes): one lane written and read, selected by a
    constant or an SGPR, whatever EXEC holds."""
    vm = GcnVirtualMachine(104, 256, 64)
    vm.v[5] = np.arange(64, dtype=np.uint32) + 100
    vm.s[4], vm.s[6] = 0xCAFE, 37
    vm.exec = 0   # no lane active: neither instruction looks at EXEC
    vm.run("generated_gemm:\n v_writelane_b32 v5, s4, 3\n v_writelane_b32 v5, 0x77, s6\n"
           " v_readlane_b32 s8, v5, 3\n v_readlane_b32 s9, v5, s6\n v_readlane_b32 s10, v5, 63\n s_endpgm\n")
    want = np.arange(64, dtype=np.uint32) + 100
    want[3], want[37] = 0xCAFE, 0x77
    assert np.array_equal(vm.v[5], want)
    assert (int(vm.s[8]), int(vm.s[9]), int(vm.s[10])) == (0xCAFE, 0x77, 163)


def test_bitop3_truth_tables():
    """v_bitop3_b32 (gfx950): bit i of the result is entry (S0_i, S1_i, S2_i)
    of the truth table, S0 the high index bit: 0xF0/0xCC/0xAA select one
    source, 0x96 is a three-way XOR, 0xE8 the majority, and the two tables the
    compiler emits for the B-tile swizzle, 0x36 = (S0 | S2) ^ S1 and
    0x6C = S1 ^ (S0 & S2)."""
    rng = np.random.default_rng(5)
    x, y, z = (rng.integers(0, 2 ** 32, 64, dtype=np.uint64).astype(np.uint32) for _ in range(3))
    want = {0xF0: x, 0xCC: y, 0xAA: z, 0x96: x ^ y ^ z, 0xE8: (x & y) | (x & z) | (y & z),
            0x36: (x | z) ^ y, 0x6C: y ^ (x & z), 0x00: np.zeros(64, np.uint32), 0xFF: np.full(64, 0xFFFFFFFF, np.uint32)}
    for table, expect in want.items():
        vm = GcnVirtualMachine(104, 256, 64)
        vm.v[1], vm.v[2], vm.v[3] = x, y, z
        vm.run(f"generated_gemm:\n v_bitop3_b32 v4, v1, v2, v3 bitop3:0x{table:x}\n s_endpgm\n")
        assert np.array_equal(vm.v[4], expect), hex(table)
    vm = GcnVirtualMachine(104, 256, 64)
    vm.v[1], vm.v[2] = x, y
    vm.run("generated_gemm:\n v_bitop3_b32 v4, v1, v2, 2 bitop3:0x36\n s_endpgm\n")   # inline constant
    assert np.array_equal(vm.v[4], (x | np.uint32(2)) ^ y)


def test_vm_atomics_and_lane_counts():
    vm = GcnVirtualMachine(104, 256, 64)
    mem = V.Memory(8192, "vmem")
    mem.allocate_region(4096, 64, "counter")
    mem.write_bytes(4096, struct.pack("<I", 5))
    vm.vmem = mem
    vm.s[8], vm.s[9] = 4096, 0
    vm.v[0] = np.zeros(64, dtype=np.uint32)
    vm.v[1] = np.full(64, 2, dtype=np.uint32)
    vm.s[20], vm.s[21] = 0xF0F0F0F0, 0x0000FFFF
    vm.run("generated_gemm:\n global_atomic_add v2, v0, v1, s[8:9] sc0\n s_waitcnt vmcnt(0)\n"
           " v_mbcnt_lo_u32_b32 v3, s20, 0\n v_mbcnt_hi_u32_b32 v3, s21, v3\n s_bcnt1_i32_b64 s22, s[20:21]\n"
           " s_endpgm\n")
    assert np.array_equal(vm.v[2], 5 + 2 * np.arange(64, dtype=np.uint32))   # lanes in order
    assert struct.unpack("<I", mem.read_bytes(4096, 4))[0] == 5 + 2 * 64
    mask = 0x0000FFFFF0F0F0F0
    want = [bin(mask & ((1 << l) - 1)).count("1") for l in range(64)]
    assert vm.v[3].tolist() == want and vm.s[22] == bin(mask).count("1")


def test_an_undersized_buffer_is_caught():
    # A one float short of m*k: the kernel's last read of A leaves the buffer
    prog, cfg = program("mt32x32_a32_wg1x1_dk16")
    m, n, k = 32, 32, 16
    mem = V.Memory(1 << 16, "vmem")
    offs = [4096, 16384, 32768]
    mem.allocate_region(offs[0], 4 * m * k - 4, "A")
    mem.allocate_region(offs[1], 4 * k * n, "B")
    mem.allocate_region(offs[2], 4 * m * n, "D")
    ka = pack_kernargs(offs[0], offs[1], 0, offs[2], m, n, k, m, k, m, m, 1.0, 0.0, 1, 1)
    with pytest.raises(MemoryError, match="outside every allocated buffer"):
        run_kernel(prog, (1, 1), cfg.num_workitems, ka, mem)


# ------------------------------------------------------ VM unit checks
def test_scalar_alu_wraps_and_sets_scc():
    vm = GcnVirtualMachine(104, 256, 64)
    vm.s[1], vm.s[2] = 0xFFFFFFFF, 2
    vm.run("generated_gemm:\n s_add_u32 s3, s1, s2\n s_addc_u32 s4, 0, 0\n s_mul_hi_u32 s5, s1, s1\n"
           " s_endpgm\n")
    assert vm.s[3] == 1 and vm.s[4] == 1 and vm.s[5] == 0xFFFFFFFE
    # and-not / or-not: s6 = 0x1234 & ~63, SCC set; s7 = 0 | ~0xFFFFFFFF = 0, SCC clear
    vm.s[6], vm.s[8] = 0x1234, 0
    vm.run("generated_gemm:\n s_andn2_b32 s6, s6, 63\n s_cselect_b32 s9, 1, 0\n s_orn2_b32 s7, s8, s1\n"
           " s_cselect_b32 s10, 1, 0\n s_endpgm\n")
    assert (vm.s[6], vm.s[9], vm.s[7], vm.s[10]) == (0x1200, 1, 0, 0)


def test_vector_64bit_subtract_chains():
    """x - y and y - x on 64-bit lanes through the borrow ops the compiler
    chains (v_sub_co/v_subb_co and v_subrev_co/v_subbrev_co), against Python
    integers modulo 2^64."""
    rng = np.random.default_rng(11)
    x = [int(v) for v in rng.integers(0, 2 ** 64, 64, dtype=np.uint64)]
    y = [int(v) for v in rng.integers(0, 2 ** 64, 64, dtype=np.uint64)]
    y[:4] = [x[0], x[1] + 1 & (2 ** 64 - 1), 0, 2 ** 64 - 1]  # equal, off by one, extremes
    vm = GcnVirtualMachine(104, 256, 64)
    for reg, vals in ((0, x), (2, y)):
        vm.v[reg] = np.array([v & 0xFFFFFFFF for v in vals], dtype=np.uint32)
        vm.v[reg + 1] = np.array([v >> 32 for v in vals], dtype=np.uint32)
    vm.run("generated_gemm:\n v_sub_co_u32_e32 v4, vcc, v0, v2\n v_subb_co_u32_e32 v5, vcc, v1, v3, vcc\n"
           " v_subrev_co_u32_e32 v6, vcc, v0, v2\n v_subbrev_co_u32_e32 v7, vcc, v1, v3, vcc\n s_endpgm\n")
    got_xy = [int(lo) | int(hi) << 32 for lo, hi in zip(vm.v[4], vm.v[5])]
    got_yx = [int(lo) | int(hi) << 32 for lo, hi in zip(vm.v[6], vm.v[7])]
    assert got_xy == [(a - b) % 2 ** 64 for a, b in zip(x, y)]
    assert got_yx == [(b - a) % 2 ** 64 for a, b in zip(x, y)]
    assert vm.vcc == sum(1 << i for i, (a, b) in enumerate(zip(x, y)) if a > b)  # borrow of y - x


def test_integer_clamp_saturates_and_saveexec_or():
    """VOP3 clamp on unsigned add/sub saturates to [0, 2^32 - 1] (the
    compiler uses it for max(a - b, 0)); without it the result wraps.
    s_or_saveexec_b64 reads its source before writing the old EXEC there;
    s_andn2_saveexec_b64 keeps the source lanes EXEC had off.  A modifier the VM does not model fails loudly."""
    vm = GcnVirtualMachine(104, 256, 64)
    vm.v[0] = np.array([5, 3, 0, 0xFFFFFFF0] * 16, dtype=np.uint32)
    vm.v[1] = np.array([3, 5, 1, 0x20] * 16, dtype=np.uint32)
    vm.exec = 0x00000000FFFF0000
    vm.s[4], vm.s[5] = 0x0000FFFF, 0x0
    vm.run("generated_gemm:\n v_sub_u32_e64 v2, v0, v1 clamp\n v_sub_u32_e64 v3, v0, v1\n"
           " v_add_u32_e64 v4, v0, v1 clamp\n v_subrev_u32_e64 v5, v0, v1 clamp\n"
           " s_or_saveexec_b64 s[4:5], s[4:5]\n s_endpgm\n")
    lanes = range(16, 32)  # lanes live under the starting EXEC
    assert [int(vm.v[2][i]) for i in lanes] == [2, 0, 0, 0xFFFFFFD0] * 4
    assert [int(vm.v[3][i]) for i in lanes] == [2, 0xFFFFFFFE, 0xFFFFFFFF, 0xFFFFFFD0] * 4
    assert [int(vm.v[4][i]) for i in lanes] == [8, 8, 1, 0xFFFFFFFF] * 4
    assert [int(vm.v[5][i]) for i in lanes] == [0, 2, 1, 0] * 4
    assert vm.exec == 0x00000000FFFFFFFF and (vm.s[4], vm.s[5]) == (0xFFFF0000, 0)
    # s_andn2_saveexec_b64: EXEC = S0 & ~EXEC, the old EXEC saved
    vm.s[6], vm.s[7] = 0x00FF00FF, 0x1
    vm.run("generated_gemm:\n s_andn2_saveexec_b64 s[8:9], s[6:7]\n s_endpgm\n")
    assert vm.exec == 0x0000000100000000 and (vm.s[8], vm.s[9]) == (0xFFFFFFFF, 0) and vm.scc == 1
    with pytest.raises(NotImplementedError):
        GcnVirtualMachine(104, 256, 64).run("generated_gemm:\n v_add_u32_e64 v2, v0, v1 mul:2\n s_endpgm\n")


def test_global_address_wraps_like_the_hardware():
    """saddr + zero-extended vaddr is taken modulo 2^64: a base below the memory
    (a K tile's base before the matrix) with offsets that land inside reads
    the right bytes; a lane whose sum stays outside is an error."""
    vm = GcnVirtualMachine(104, 256, 64)
    vm.vmem = V.Memory(1024, "vmem")
    vm.vmem.write_bytes(0, np.arange(256, dtype=np.uint32).tobytes())
    base = (1 << 64) - 64
    vm.s[0], vm.s[1] = base & 0xFFFFFFFF, base >> 32
    vm.v[0] = np.array([64 + 16 * (i % 8) for i in range(64)], dtype=np.uint32)  # lands at bytes 0..112
    vm.run("generated_gemm:\n global_load_dwordx4 v[4:7], v0, s[0:1]\n s_waitcnt vmcnt(0)\n s_endpgm\n")
    assert [int(vm.v[4][i]) for i in range(8)] == [4 * (i % 8) for i in range(8)]
    assert [int(vm.v[7][i]) for i in range(8)] == [4 * (i % 8) + 3 for i in range(8)]
    vm.v[0] = np.full(64, 48, dtype=np.uint32)  # base + 48 is still 16 bytes below the memory
    with pytest.raises(MemoryError):
        vm.run("generated_gemm:\n global_load_dwordx4 v[4:7], v0, s[0:1]\n s_waitcnt vmcnt(0)\n s_endpgm\n")


def test_integer_division_sequence_of_the_compiler():
    # the kernel's tile order divides by runtime values with v_rcp_iflag_f32 and
    # correction steps: check the emitted sequence over many numerators
    src = ('#include <hip/hip_runtime.h>\nextern "C" __global__ void generated_gemm(unsigned* o, unsigned a, '
           'unsigned b) { o[threadIdx.x] = (a + threadIdx.x) / b; o[64 + threadIdx.x] = (a + threadIdx.x) % b; }\n')
    prog = V.parse_assembly(g.compile_to_assembly(src))
    for a, b in ((0, 1), (1000, 7), (123456, 255), (4294967000, 3), (77, 100)):
        mem = V.Memory(1024, "vmem")
        ka = struct.pack("<QII", 512, a, b)
        run_kernel(prog, (1, 1), 64, ka, mem)
        out = np.frombuffer(mem.read_bytes(512, 512), dtype=np.uint32)
        t = (np.arange(64, dtype=np.uint64) + a) & 0xFFFFFFFF
        assert np.array_equal(out[:64], (t // b).astype(np.uint32)), (a, b)
        assert np.array_equal(out[64:], (t % b).astype(np.uint32)), (a, b)


def test_operand_parser_forms():
    assert parse_operand("v[4:7]").count == 4 and parse_operand("a12").kind == "a"
    assert parse_operand("1.0").value == 0x3F800000 and parse_operand("-4").value == -4
    assert parse_operand("0x50").value == 0x50 and parse_operand(".LBB0_2").kind == "label"
    with pytest.raises(NotImplementedError):
        parse_operand("v[1:2")


def test_unknown_instruction_fails_loudly():
    vm = GcnVirtualMachine(104, 256, 64)
    with pytest.raises(NotImplementedError, match="v_frobnicate"):
        vm.run("generated_gemm:\n v_frobnicate v0, v1\n s_endpgm\n")


# ------------------------------------------------------ wave specialisation
WS_NAME = "mt64x64_a16_wg1x4_dk32_s4_ws"


def _ws_workitems(name):
    cfg, opt = catalog.SOLUTIONS[name]
    wg, _ = g.launch_geometry(cfg, opt)
    return wg[0] * wg[1] * 64


@pytest.mark.parametrize("seed", [None, 1, 2, 3, 4])
def test_wave_specialised_kernel_in_vm(seed):
    """The loading / computing waves of the wave-specialised instance order
    their LDS buffers with counters only (no barrier per K tile).  In the VM a
    polling wave yields at s_sleep, and with a seed every wave also loses its
    turn at random instructions, so the counters are exercised under many
    interleavings: 7 K tiles (the 4-buffer ring wraps) with a K remainder
    (a head tile), two tiles, alpha/beta -- every interleaving must give the
    same bits, within the parity bar of float64."""
    prog, cfg = program(WS_NAME)
    m, n, k = 128, 64, 32 * 6 + 5
    A = oracle.fill_matrix(m, k, 6, 0)
    B = oracle.fill_matrix(k, n, 6, 1)
    C = oracle.fill_matrix(m, n, 6, 2)
    D, info = run_sgemm(prog, cfg.tile_size, _ws_workitems(WS_NAME), A, B, C, 0.5, -1.25, preempt_seed=seed)
    assert info["grid"] == (2, 1)
    assert oracle.normwise_error(D, oracle.gemm_f64(A, B, C, 0.5, -1.25)) <= oracle.tolerance(k)
    D0, _ = run_sgemm(prog, cfg.tile_size, _ws_workitems(WS_NAME), A, B, C, 0.5, -1.25)
    assert np.array_equal(D, D0)


KS_NAME, KS_TWIN = "mt64x64_a16_wg1x4_dk32_s3_ks", "mt64x64_a16_wg1x4_dk32_s3"


def test_k_split_ranges_partition_k():
    for dk in (16, 32, 64):
        for k in range(0, 8 * dk + 3):
            k0, k1 = k_split_ranges(k, dk)
            assert k0 == k1 and 0 <= k0 <= k
            assert abs((k - k0) - k0) <= dk   # the halves differ by at most one K tile


@pytest.mark.parametrize("m,n,k", [(128, 64, 197), (64, 64, 160), (64, 64, 128), (64, 64, 45), (64, 64, 32),
                                   (64, 64, 17), (100, 70, 77), (64, 128, 3)])
def test_k_split_kernel_in_vm(m, n, k):
    """The in-group K split: group 0 sums K range [0, k0), group 1 [k1, k)
    (a zero head tile when the tile count is odd), and group 0 adds group 1's
    sums.  With alpha = 1, beta = 0, D is therefore exactly the fp32 sum of
    the one-group kernel's results on the two ranges (same tile boundaries and
    head shift, so the same MFMA sequence); the cases cover a shifted head, an
    odd and an even tile count, one K tile, the slow path for two shifted
    tiles, and edge tiles.  With alpha / beta and random preemption the
    result stays within the bar and bit-stable."""
    prog, cfg = program(KS_NAME)
    twin, tcfg = program(KS_TWIN)
    wi = _ws_workitems(KS_NAME)
    assert wi == 2 * tcfg.num_workitems and cfg.tile_size == tcfg.tile_size
    A = oracle.fill_matrix(m, k, 7, 0)
    B = oracle.fill_matrix(k, n, 7, 1)
    C = oracle.fill_matrix(m, n, 7, 2)
    D, _ = run_sgemm(prog, cfg.tile_size, wi, A, B, None, 1.0, 0.0)
    k0, k1 = k_split_ranges(k, cfg.depth_k)
    S0, _ = run_sgemm(twin, tcfg.tile_size, tcfg.num_workitems, A[:, :k0], B[:k0, :], None, 1.0, 0.0)
    S1 = np.zeros((m, n), np.float32)
    if k1 < k:
        S1, _ = run_sgemm(twin, tcfg.tile_size, tcfg.num_workitems, A[:, k1:], B[k1:, :], None, 1.0, 0.0)
    assert np.array_equal(D, (S0 + S1).astype(np.float32))
    Dab, _ = run_sgemm(prog, cfg.tile_size, wi, A, B, C, 0.5, -1.25, preempt_seed=3)
    assert oracle.normwise_error(Dab, oracle.gemm_f64(A, B, C, 0.5, -1.25)) <= oracle.tolerance(k)
    Dab0, _ = run_sgemm(prog, cfg.tile_size, wi, A, B, C, 0.5, -1.25)
    assert np.array_equal(Dab, Dab0)


FLAG_PROTOCOL = """
generated_gemm:
    v_readfirstlane_b32 s4, v0
    s_cmp_ge_u32 s4, 64
    s_cbranch_scc1 .Lwriter
    v_mov_b32 v1, 0
.Lpoll:
    ds_read_b32 v2, v1
    s_waitcnt lgkmcnt(0)
    v_readfirstlane_b32 s5, v2
    s_cmp_eq_u32 s5, 1
    s_cbranch_scc1 .Lgot
    s_sleep 1
    s_branch .Lpoll
.Lgot:
    ds_read_b32 v3, v1 offset:4
    s_waitcnt lgkmcnt(0)
    ds_write_b32 v1, v3 offset:8
    s_endpgm
.Lwriter:
    v_mov_b32 v1, 0
    v_mov_b32 v2, 42
    v_mov_b32 v3, 1
    {first}
    {second}
    s_endpgm
.Lfunc_end0:
.amdhsa_kernel generated_gemm
    .amdhsa_group_segment_fixed_size 16
    .amdhsa_user_sgpr_count 2
    .amdhsa_user_sgpr_kernarg_segment_ptr 1
    .amdhsa_system_sgpr_workgroup_id_x 1
.end_amdhsa_kernel
"""


def _flag_protocol_result(data_first, seed):
    data, flag = "ds_write_b32 v1, v2 offset:4", "ds_write_b32 v1, v3"
    asm = FLAG_PROTOCOL.format(first=data if data_first else flag, second=flag if data_first else data)
    seen = []
    V.run_kernel(asm, (1, 1), 128, b"\0" * 8, V.Memory(64, "vmem"), preempt_seed=seed, preempt_rate=0.25,
                 on_workgroup=lambda x, y, waves: seen.append(int(waves[0].lds.read_u32(np.array([8]), 1, "")[0, 0])))
    return seen[0]


def test_vm_preemption_catches_a_flag_raised_before_its_data():
    """The checker behind the test above: wave 1 writes a value and raises a
    flag, wave 0 polls the flag and copies the value.  With the flag raised
    after the data every interleaving copies 42; raised before it, the turn
    order alone still copies 42 (the writer is never interrupted), but
    random preemption finds interleavings that copy the stale 0."""
    assert all(_flag_protocol_result(True, s) == 42 for s in [None] + list(range(200)))
    assert _flag_protocol_result(False, None) == 42
    stale = [s for s in range(200) if _flag_protocol_result(False, s) == 0]
    assert stale, "no interleaving put the reader between the writer's two writes"



SCRATCH_ROUND_TRIP = """
generated_gemm:
    s_mov_b32 s4, 1024
    s_mov_b32 s5, 0
    v_lshlrev_b32 v1, 2, v0
    v_add_u32 v2, 1000, v0
    v_add_u32 v3, 2000, v0
    scratch_store_dwordx2 off, v[2:3], off offset:8
    v_mov_b32 v2, 0
    v_mov_b32 v3, 0
    scratch_load_dwordx2 v[4:5], off, off offset:8
    s_waitcnt vmcnt(0)
    s_load_dword s2, s[0:1], 0x54
    s_waitcnt lgkmcnt(0)
    v_add_u32 v4, s2, v4
    global_store_dword v1, v4, s[4:5]
    global_store_dword v1, v5, s[4:5] offset:256
    s_endpgm
.Lfunc_end0:
.amdhsa_kernel generated_gemm
    .amdhsa_group_segment_fixed_size 0
    .amdhsa_kernarg_size 88
    .amdhsa_user_sgpr_count 2
    .amdhsa_user_sgpr_kernarg_segment_ptr 1
    .amdhsa_system_sgpr_workgroup_id_x 1
.end_amdhsa_kernel
"""


def test_vm_scratch_is_private_per_lane_and_kernargs_span_the_declared_segment():
    """Spilled registers (scratch_store / scratch_load with no address
    registers) come back per lane after the vmcnt wait, and the kernarg
    segment is as long as the kernel declares: bytes past the given 8-byte
    image (offset 0x54 here, inside the declared 88) read as zero, as the
    runtime's zero-filled segment does."""
    prog = V.parse_assembly(SCRATCH_ROUND_TRIP)
    assert prog.desc["amdhsa_kernarg_size"] == 88
    mem = V.Memory(4096, "vmem")
    mem.allocate_region(1024, 512, "out")
    V.run_kernel(prog, (1, 1), 64, b"\0" * 8, mem)
    out = np.frombuffer(mem.read_bytes(1024, 512), dtype=np.uint32)
    lanes = np.arange(64, dtype=np.uint32)
    assert np.array_equal(out[:64], 1000 + lanes) and np.array_equal(out[64:], 2000 + lanes)


def test_vm_scratch_bounds_are_checked():
    vm = GcnVirtualMachine()
    vm.v[1] = np.full(64, 1 << 20, dtype=np.uint32)
    with pytest.raises(MemoryError, match="scratch"):
        vm.run("generated_gemm:\n    scratch_store_dword v1, v2, off\n    s_endpgm\n")


def _with_layout(name, ta, tb):
    cfg, opt = copy.deepcopy(catalog.SOLUTIONS[name])
    c = g.GemmSolutionConfig(cfg.a_type, cfg.b_type, cfg.cd_type, cfg.scalar_type, cfg.mfma, cfg.wave_group,
                             cfg.wave_tiling, cfg.depth_k, ta, tb, vmem_stage=cfg.vmem_stage)
    ctx = g.GpuContext()
    g.gemm(ctx, "generated_gemm", "gfx950", c, opt, g.default_arguments())
    wg, _ = g.launch_geometry(c, opt)
    return V.parse_assembly(ctx.assembly(), "generated_gemm"), c, wg[0] * wg[1] * 64


@pytest.mark.parametrize("ta,tb", [(True, False), (False, True), (True, True)])
def test_ws_and_k_split_with_transposed_operands_in_vm(ta, tb):
    """The wave-specialised and the in-group K split instances rebuilt for
    TN, NT and TT: the first bit-identical to the barrier twin of its layout,
    the second to the sum of that twin's results on its two K ranges, on a
    ragged shape with a K remainder (alpha = 1, beta = 0)."""
    m, n, k = 100, 70, 77
    A = oracle.fill_matrix(m, k, 8, 0)
    B = oracle.fill_matrix(k, n, 8, 1)
    As = np.asfortranarray(A.T) if ta else A
    Bs = np.asfortranarray(B.T) if tb else B
    twin, tcfg, twi = _with_layout(KS_TWIN, ta, tb)

    def run_twin(k0, k1):
        a = np.asfortranarray(As[k0:k1, :] if ta else As[:, k0:k1])
        b = np.asfortranarray(Bs[:, k0:k1] if tb else Bs[k0:k1, :])
        return run_sgemm(twin, tcfg.tile_size, twi, a, b, None, 1.0, 0.0, mnk=(m, n, k1 - k0))[0]

    ws, wcfg, wwi = _with_layout(WS_NAME, ta, tb)
    Dw, _ = run_sgemm(ws, wcfg.tile_size, wwi, As, Bs, None, 1.0, 0.0, mnk=(m, n, k))
    assert np.array_equal(Dw, run_twin(0, k))
    ks, kcfg, kwi = _with_layout(KS_NAME, ta, tb)
    Dk, _ = run_sgemm(ks, kcfg.tile_size, kwi, As, Bs, None, 1.0, 0.0, mnk=(m, n, k))
    k0, k1 = k_split_ranges(k, kcfg.depth_k)
    S1 = run_twin(k1, k) if k1 < k else np.zeros((m, n), np.float32)
    assert np.array_equal(Dk, (run_twin(0, k0) + S1).astype(np.float32))
    assert oracle.normwise_error(Dk, oracle.gemm_f64(A, B, None, 1.0, 0.0)) <= oracle.tolerance(k)
