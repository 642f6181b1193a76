"""Kernel generator for the gfx950 FP32 column-major NN SGEMM.

This module keeps the reference generator's Python surface
(/root/reference/generator/generator.py) so that the tuner, the tests and any
caller written against it keep working:

* ``DataType`` / ``datatype_size``            (generator.py:816-824)
* ``GemmOptimizations(level, wgm, plr, gw, map_k_idx)``  (generator.py:827-854)
* ``GemmSolutionConfig(...)`` with ``tile_size``, ``num_workitems``,
  ``num_bytes_per_buffer_load``, ``lds_pad_bytes``, ``lds_usage_bytes``,
  ``to_dict`` / ``from_dict`` and ``RuntimeError`` on invalid geometry
  (generator.py:857-1055)
* ``FunctionArgument``                        (generator.py:94-103)
* ``gemm(context, name, arch, config, opt, args) -> str``  (generator.py:1056)
* ``compile(kern_name, kern_str, arch, output_folder, config) -> int``
  (generator.py:2534-2569): writes ``<out>/<name>.co`` and ``<out>/<name>.toml``
* the CLI ``generator.py --arch gfx950 <out>``  (generator.py:2571-2623)

What ``gemm`` produces is different by design: instead of GCN assembly text it
returns a self-contained HIP translation unit -- the hand-written gfx950
kernel template in ``csrc/sgemm_gfx950.hip`` specialised by ``#define`` lines --
and ``compile`` builds it with ``hipcc --cuda-device-only -c --offload-arch=gfx950``.  The
code object exports ``generated_gemm`` with the reference's 15-argument,
76-byte kernarg layout, so the reference runner can load it unchanged.
"""
from __future__ import annotations

import argparse
import functools
import math
import os
import shutil
import subprocess
import sys
import tempfile
from enum import IntEnum
from typing import Dict, List, Optional, Sequence, Tuple

_HERE = os.path.dirname(os.path.abspath(__file__))
PACKAGE_ROOT = os.path.dirname(_HERE)
KERNEL_TEMPLATE = os.path.join(PACKAGE_ROOT, "csrc", "sgemm_gfx950.hip")

DEFAULT_HIPCC_PATH = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
SUPPORTED_ARCHS = ("gfx950", "gfx950:xnack-")
# LDS of one gfx950 compute unit (CDNA4: 160 KiB), the largest static LDS a
# work-group may declare.
MAX_LDS_NUM_BYTES = 163840
# most K ranges one output tile may be split into (generated_gemm_splitk)
MAX_SPLIT_K = 16
# Work-items per work-group accepted by the hardware.
MAX_WORKITEMS = 1024
# How gfx950 serves one wave-wide LDS instruction, measured with
# profiler/lds_probe (962 patterns: lane-pair tests, strided lanes and this
# kernel's own accesses, every one reproduced by lds_access_cycles):
# (write, bytes per lane) -> (banks of 4 bytes, lanes served per cycle).
# Reads of 8 and 16 bytes see 64 banks (256 bytes a cycle), every other kind
# 32 banks (128 bytes a cycle).
LDS_SERVICE = {
    (False, 4): (32, 32), (False, 8): (64, 32), (False, 16): (64, 16),
    (True, 4): (32, 32), (True, 8): (32, 16), (True, 16): (32, 8),
}
LDS_BANK_BYTES = 4
# pads (floats) and B-chunk swizzles the layout search tries
LDS_PADS = (0, 4, 8, 12, 16)
# hipcc flags for every kernel: packed FP32 VALU ops stay off.
HIPCC_KERNEL_FLAGS = (
    "-O3",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
)

# MFMA atoms as (M, N, blocks, K), the reference's tuple convention
# (generator.py:796-801).
MFMA_32x32x2 = (32, 32, 1, 2)
MFMA_16x16x4 = (16, 16, 1, 4)
SUPPORTED_MFMAS = (MFMA_16x16x4, MFMA_32x32x2)


class DataType(IntEnum):
    FP32 = 0


def datatype_size(dtype: DataType) -> int:
    if dtype == DataType.FP32:
        return 4
    raise RuntimeError(f"unrecognized type {dtype!r}")


def _is_pow2(x: int) -> bool:
    return x > 0 and (x & (x - 1)) == 0


class GemmOptimizations:
    """Code-shape knobs that are baked into the code object.

    Same constructor and defaults as the reference (generator.py:827-854):
    level != 0 turns on ``plr = 1`` and ``gw = 1``.  Meaning on gfx950:

    * ``wgm``       -- group width (in tiles along M) of the work-group order.
    * ``plr``       -- K-loop schedule: 0 reads a k block's operands and then
                       multiplies; 1 reads block kb+1 while block kb multiplies
                       (register double buffering), refilling LDS after the
                       tile's last block; 2 also issues the next tile's LDS
                       writes and global loads right after the first block and,
                       with >= 3 LDS buffers, reads the next tile's first
                       operands before the barrier; 3 is 2 with the memory
                       instructions interleaved one by one between MFMAs.
    * ``gw``        -- epilogue (global write) flavour, as the reference's
                       ``gw_naive`` / ``gw_vgpr_minimized`` pair
                       (generator.py:2290-2508): 0 stores straight from the
                       accumulators (float4 per accumulator slot, 16 bytes in
                       each of atom_n columns per instruction, no LDS); 1
                       stages each MFMA column group through LDS and stores
                       whole column runs (falls back to 0 when the staging
                       chunks do not fit the kernel's LDS).
    * ``map_k_idx`` -- rotate the first K tile by ``tile_x & (map_k_idx - 1)``.
    * ``xcd``       -- (gfx950 only) number of XCDs to give contiguous tile
                       ranges to; 0 or 1 leaves the hardware order.
    * ``pd``        -- (gfx950 only) prefetch depth of the early-refill
                       schedules: a K tile's global loads are issued ``pd``
                       tiles before its LDS writes (1 or 2 register sets).
    * ``occ``       -- (gfx950 only) 0 lets the compiler size registers for
                       one wave per SIMD; n >= 2 caps them so that n waves
                       per SIMD (n work-groups of one wave per SIMD) fit.
    * ``split_k``   -- (gfx950 only) 1 builds the reference's single kernel
                       only; any other value also builds
                       ``generated_gemm_splitk``, which splits each output
                       tile's K into ranges and reduces them in the kernel.
                       The value is the launch's default split count: 0 lets
                       the host pick one per problem (split only when the
                       tiles cannot fill the GPU), 2..16 fixes it.
    * ``stream_k``  -- (gfx950 only) 1 also builds ``generated_gemm_streamk``,
                       which spreads the K iterations of the tiles past the
                       last whole round of work-groups over every resident
                       work-group (each tile cut at most once, fixed up by a
                       commutative two-partial sum); the host uses it when a
                       grid would leave a partial last round.
    * ``ws``        -- (gfx950 only) 1 doubles the work-group with loading
                       waves (wave specialisation): the configured waves only
                       read LDS and multiply, and as many more waves copy K
                       tiles from memory to LDS, the two roles ordered by LDS
                       counters instead of a work-group barrier per K tile.
                       The .toml then describes the launch: wave_group [2 *
                       WG0, WG1] and wave_tiling [WT0 / 2, WT1] (the same tile,
                       twice the work-items; WT0 must be even), with the
                       computing geometry under compute_wave_group /
                       compute_wave_tiling.  No split-K or stream-K kernel.
    * ``ws_pd``     -- (with ``ws``) K tiles each loading wave keeps in
                       flight in registers (2..4).
    * ``ksplit``    -- (gfx950 only) 1 doubles the work-group with a second
                       group of the configured waves: each group loads and
                       multiplies half of the tile's K tiles in an LDS ring
                       of its own (twice the LDS), one barrier per pair of K
                       tiles, and the groups' sums are added through LDS
                       before the epilogue.  The .toml describes the launch
                       as for ``ws``.  No split-K or stream-K kernel, no
                       ``map_k_idx``.
    * ``stream_k_rounds`` -- (host policy, written to the .toml) the most
                       whole-tile rounds of work-groups for which the host
                       still picks stream-K on its own (0: no limit); tiles
                       whose stream-K kernel loses on long grids set it.
    """

    def __init__(
        self,
        level: int,
        wgm: Optional[int] = None,
        plr: Optional[int] = None,
        gw: Optional[int] = None,
        map_k_idx: Optional[int] = None,
        xcd: Optional[int] = None,
        pd: Optional[int] = None,
        occ: Optional[int] = None,
        split_k: Optional[int] = None,
        stream_k: Optional[int] = None,
        stream_k_rounds: Optional[int] = None,
        ws: Optional[int] = None,
        ws_pd: Optional[int] = None,
        ksplit: Optional[int] = None,
    ):
        self.level = level
        self.wgm = 1
        self.plr = 0
        self.gw = 0
        self.map_k_idx = 0
        self.xcd = 0
        self.pd = 1
        self.occ = 0
        self.split_k = 1
        self.stream_k = 0
        self.stream_k_rounds = 0
        self.ws = 0
        self.ws_pd = 2
        self.ksplit = 0
        self._setup_optimizations()
        if wgm is not None:
            self.wgm = wgm
        if plr is not None:
            self.plr = plr
        if gw is not None:
            self.gw = gw
        if map_k_idx is not None:
            self.map_k_idx = map_k_idx
        if xcd is not None:
            self.xcd = xcd
        if pd is not None:
            self.pd = pd
        if occ is not None:
            self.occ = occ
        if split_k is not None:
            self.split_k = split_k
        if stream_k is not None:
            self.stream_k = stream_k
        if stream_k_rounds is not None:
            self.stream_k_rounds = stream_k_rounds
        if ws is not None:
            self.ws = ws
        if ws_pd is not None:
            self.ws_pd = ws_pd
        if ksplit is not None:
            self.ksplit = ksplit
        if self.wgm < 1:
            raise RuntimeError(f"Invalid wgm: {self.wgm}")
        if self.map_k_idx and not _is_pow2(self.map_k_idx):
            raise RuntimeError(f"map_k_idx must be 0 or a power of two: {self.map_k_idx}")
        if self.plr not in (0, 1, 2, 3) or self.gw not in (0, 1) or self.xcd < 0:
            raise RuntimeError(f"Invalid optimization knobs: plr={self.plr} gw={self.gw} xcd={self.xcd}")
        if self.pd not in (1, 2) or (self.pd == 2 and self.plr < 2):
            raise RuntimeError(f"Invalid prefetch depth {self.pd} (2 needs plr >= 2)")
        if self.occ not in (0, 1, 2, 3, 4, 8):
            raise RuntimeError(f"Invalid occupancy target {self.occ}")
        if not 0 <= self.split_k <= MAX_SPLIT_K:
            raise RuntimeError(f"Invalid split_k {self.split_k} (0 = auto, or 1..{MAX_SPLIT_K})")
        if self.stream_k not in (0, 1):
            raise RuntimeError(f"Invalid stream_k {self.stream_k} (0 or 1)")
        if self.stream_k_rounds < 0:
            raise RuntimeError(f"Invalid stream_k_rounds {self.stream_k_rounds} (0 = no limit)")
        if self.ws not in (0, 1) or self.ws_pd not in (2, 3, 4):
            raise RuntimeError(f"Invalid wave specialisation ws={self.ws} ws_pd={self.ws_pd}")
        if self.ws and (self.split_k != 1 or self.stream_k):
            raise RuntimeError("wave specialisation (ws=1) builds no split-K or stream-K kernel")
        if self.ksplit not in (0, 1):
            raise RuntimeError(f"Invalid in-group K split ksplit={self.ksplit}")
        if self.ksplit and (self.ws or self.split_k != 1 or self.stream_k or self.map_k_idx > 1):
            raise RuntimeError("the in-group K split (ksplit=1) excludes ws, split-K, stream-K and map_k_idx")

    def _setup_optimizations(self):
        if self.level != 0:
            self.plr = 1
            self.gw = 1

    def to_dict(self) -> Dict:
        return {
            "opt_level": int(self.level),
            "wgm": int(self.wgm),
            "plr": int(self.plr),
            "gw": int(self.gw),
            "map_k_idx": int(self.map_k_idx),
            "xcd": int(self.xcd),
            "pd": int(self.pd),
            "occ": int(self.occ),
            "split_k": int(self.split_k),
            "stream_k": int(self.stream_k),
            "stream_k_rounds": int(self.stream_k_rounds),
            "ws": int(self.ws),
            "ws_pd": int(self.ws_pd),
            "ksplit": int(self.ksplit),
        }

    def __repr__(self) -> str:
        return (f"GemmOptimizations(level={self.level}, wgm={self.wgm}, plr={self.plr}, "
                f"gw={self.gw}, map_k_idx={self.map_k_idx}, xcd={self.xcd}, pd={self.pd}, occ={self.occ}, "
                f"split_k={self.split_k}, stream_k={self.stream_k}, ws={self.ws}, ksplit={self.ksplit})")


def lds_lane_cycle(lane: int, access_bytes: int, write: bool = False) -> int:
    """Cycle of a wave-wide LDS instruction in which gfx950 serves ``lane``:
    consecutive groups of LDS_SERVICE's lanes per cycle, except ds_read_b128,
    which serves each half-wave in two cycles and splits its eight quads (4
    lanes each) by the parity of the quad index: {0, 3, 5, 6} then {1, 2, 4, 7}."""
    _, per = LDS_SERVICE[(bool(write), access_bytes)]
    if not write and access_bytes == 16:
        quad = (lane >> 2) & 7
        return (lane >> 5) * 2 + (bin(quad).count("1") & 1)
    return lane // per


def lds_access_cycles(byte_addrs: Sequence[int], access_bytes: int, write: bool = False) -> int:
    """Cycles one wave-wide LDS access takes: per cycle of lds_lane_cycle, as
    many as the most-used bank holds distinct dwords (lanes that read or write
    the same dword share its bank cycle).  Patterns that differ by a whole
    number of bank rows cost the same, so each is counted once."""
    banks, _ = LDS_SERVICE[(bool(write), access_bytes)]
    period = banks * LDS_BANK_BYTES
    base = min(byte_addrs) // period * period
    return _lds_access_cycles(tuple(a - base for a in byte_addrs), access_bytes, bool(write))


@functools.lru_cache(maxsize=1 << 16)
def _lds_access_cycles(byte_addrs: Tuple[int, ...], access_bytes: int, write: bool) -> int:
    banks, _ = LDS_SERVICE[(write, access_bytes)]
    groups: Dict[int, List[int]] = {}
    for lane, addr in enumerate(byte_addrs):
        groups.setdefault(lds_lane_cycle(lane, access_bytes, write), []).append(addr)
    cycles = 0
    for addrs in groups.values():
        words_per_bank: Dict[int, set] = {}
        for addr in addrs:
            for w in range(access_bytes // LDS_BANK_BYTES):
                word = addr // LDS_BANK_BYTES + w
                words_per_bank.setdefault(word % banks, set()).add(word)
        cycles += max(len(v) for v in words_per_bank.values())
    return cycles


def lds_tile_accesses(mfma: Sequence[int], wave_group: Sequence[int], wave_tiling: Sequence[int], depth_k: int,
                      trans_a: bool, trans_b: bool, operand: str, pad: int, b_swizzle: Tuple[int, int] = (0, 0),
                      row_swizzle: Tuple[int, int] = (0, 0)):
    """The wave-wide LDS instructions of one work-group per K tile for one
    operand ("a" or "b") and layout, as (kind, wave, byte addresses, bytes per
    lane, write, count) -- the address formulas of csrc/sgemm_gfx950.hip: the
    tile writes of every wave, and each wave's operand reads (the waves' reads
    differ by uniform offsets, so wave 0's pattern stands for all, counted
    once per wave).  ``b_swizzle`` is the chunk swizzle (shift, mask) of the
    operand's k-contiguous rows: B's, or A^T's (whose tile is [MT0][DK + pad],
    k contiguous, where A's is [DK][MT0 + pad]).  ``row_swizzle`` (shift,
    mask), A^T only, permutes the tile's rows: row m is stored at row
    m ^ ((m >> shift) & mask), a bijection when shift is at least the mask's
    bit width."""
    am, an, _, ak = mfma
    mt0 = am * wave_group[0] * wave_tiling[0]
    mt1 = an * wave_group[1] * wave_tiling[1]
    waves = wave_group[0] * wave_group[1]
    nt = waves * 64
    steps = depth_k // ak
    kpl = 4 if steps >= 4 else (2 if steps >= 2 else 1)
    kb_len = ak * kpl
    nkb = depth_k // kb_len
    shift, mask = b_swizzle
    out = []

    def writes(chunks, order, addr_of):
        for i in range(-(-chunks // nt)):
            for w in range(waves):
                lanes = [ch for ch in (64 * w + l + i * nt for l in range(64)) if ch < chunks]
                if lanes:
                    for addrs, width in addr_of([order(ch) for ch in lanes]):
                        out.append(("write", w, addrs, width, True, 1))

    def rows_first(per_row):  # chunk -> (position along the row, row): the along-row operands
        return lambda ch: (ch % per_row, ch // per_row)

    def chunk(row, c):  # the chunk swizzle of a k-contiguous row (B, A^T)
        return c ^ ((row >> shift) & mask)

    if operand == "a" and not trans_a:
        lda = mt0 + pad
        # float4 along m into row k
        writes(mt0 * depth_k // 4, rows_first(mt0 // 4), lambda cc: [([c1 * lda * 4 + c0 * 16 for c0, c1 in cc], 16)])
        width = 4 * wave_tiling[0]
        reads = [((l // am) * kpl * lda + (l % am) * wave_tiling[0]) * 4 for l in range(64)]
        for part in range(max(1, width // 16)):  # 8 floats: two 16-byte reads
            out.append(("read", 0, [x + 16 * part for x in reads], min(width, 16), False, waves * nkb * kpl))
        return out
    if operand == "a":
        # A^T: rows of m with k contiguous, chunk swizzled like B; a lane of
        # atom i reads row r * WT0 + i (the interleaved atoms), KPL k at once
        lda = depth_k + pad
        wt0 = wave_tiling[0]
        row_shift, row_mask = row_swizzle

        def prow(m):  # stored row of row m
            return m ^ ((m >> row_shift) & row_mask)

        # at depth 16 an 8-lane write cycle covers two rows: without a row
        # swizzle they are taken four rows apart (order 0, 4, 1, 5, 2, 6, 3, 7
        # in each group of eight)
        order = ((lambda ch: (ch & 3, ((ch >> 2) & ~7) | (((ch >> 2) & 1) << 2) | (((ch >> 2) >> 1) & 3)))
                 if depth_k // 4 == 4 and not row_mask else rows_first(depth_k // 4))
        writes(mt0 * depth_k // 4, order,
               lambda cc: [([(prow(c1) * lda + chunk(c1, c0) * 4) * 4 for c0, c1 in cc], 16)])
        for kb in range(nkb):
            for i in range(wt0):
                reads = []
                for l in range(64):
                    row, kc = (l % am) * wt0 + i, (l // am) * kpl + kb * kb_len
                    reads.append((prow(row) * lda + chunk(row, kc >> 2) * 4 + (kc & 3)) * 4)
                out.append(("read", 0, reads, 4 * kpl, False, waves))
        return out
    if trans_b:
        # B^T: rows of k with n contiguous (the mirror of A); a lane reads WT1
        # consecutive n, the B operands of the interleaved atoms
        ldb = mt1 + pad
        writes(mt1 * depth_k // 4, rows_first(mt1 // 4), lambda cc: [([c1 * ldb * 4 + c0 * 16 for c0, c1 in cc], 16)])
        width = 4 * wave_tiling[1]
        reads = [((l // an) * kpl * ldb + (l % an) * wave_tiling[1]) * 4 for l in range(64)]
        for part in range(max(1, width // 16)):
            out.append(("read", 0, [x + 16 * part for x in reads], min(width, 16), False, waves * nkb * kpl))
        return out
    ldb = depth_k + pad
    # float4 along k into row n, chunk swizzled
    writes(mt1 * depth_k // 4, rows_first(depth_k // 4),
           lambda cc: [([(c1 * ldb + chunk(c1, c0) * 4) * 4 for c0, c1 in cc], 16)])
    for kb in range(nkb):
        reads = []
        for l in range(64):
            n, kc = l % an, (l // an) * kpl + kb * kb_len
            reads.append((n * ldb + chunk(n, kc >> 2) * 4 + (kc & 3)) * 4)
        out.append(("read", 0, reads, 4 * kpl, False, waves * wave_tiling[1]))
    return out


def lds_epilogue_accesses(mfma: Sequence[int], wave_group: Sequence[int], wave_tiling: Sequence[int],
                          pad: int = 0, swizzle: bool = True, grouped: bool = True):
    """The staged epilogue's LDS instructions of one work-group, in the format
    of lds_tile_accesses -- the address formulas of csrc/sgemm_gfx950.hip: per
    column group of a wave's sub-tile, the accumulator scatter into the wave's
    column-major chunk (column stride SM + ``pad`` floats, SM the sub-tile's
    rows) and the read-back of float4 runs down each column.  A lane's rows
    come in groups of four: ``grouped`` writes 4 / WT0 slots with one 16-byte
    write when the wave tile is under four atoms tall (else one write per
    slot); ``swizzle`` stores float4 run r of column c at run r ^ (c mod
    SM / 4).  The defaults are the kernel's layout.  The waves' chunks differ
    by uniform offsets: wave 0's pattern, counted once per wave and column
    group."""
    am, an = mfma[0], mfma[1]
    wt0, wt1 = wave_tiling
    waves = wave_group[0] * wave_group[1]
    acc = am * an // 64
    sm = am * wt0
    e_ld = sm + pad
    e_runs = sm // 4
    qg = 1 if (wt0 >= 4 or not grouped) else 4 // wt0

    def row(q, lane):
        return (q & 3) + 8 * (q >> 2) + 4 * (lane >> 5) if am == 32 else q + 4 * (lane >> 4)

    def at(col, pos):  # byte address of float `pos` of column `col`
        run = pos // 4
        if swizzle:
            run ^= col % e_runs
        return (col * e_ld + run * 4 + pos % 4) * 4

    out = []
    for q in range(0, acc, qg):
        width = 4 * wt0 * qg
        for part in range(max(1, width // 16)):
            addrs = [at(lane % an, row(q, lane) * wt0 + 4 * part) for lane in range(64)]
            out.append(("epilogue write", 0, addrs, min(width, 16), True, waves * wt1))
    for p in range(an * e_runs // 64):
        idx = [p * 64 + lane for lane in range(64)]
        out.append(("epilogue read", 0, [at(i // e_runs, (i % e_runs) * 4) for i in idx], 16, False, waves * wt1))
    return out


def lds_tile_cycles(accesses) -> int:
    """LDS cycles of lds_tile_accesses' instructions."""
    return sum(count * lds_access_cycles(addrs, width, write) for _, _, addrs, width, write, count in accesses)


def lds_tile_min_cycles(accesses) -> int:
    """The least LDS cycles the same instructions can take: one cycle per
    group of lanes served together (lds_lane_cycle), that is, no bank
    conflicts."""
    return sum(count * len({lds_lane_cycle(lane, width, write) for lane in range(len(addrs))})
               for _, _, addrs, width, write, count in accesses)


@functools.lru_cache(maxsize=None)
def _lds_operand_layout(mfma: Tuple[int, ...], wave_group: Tuple[int, int], wave_tiling: Tuple[int, int],
                        depth_k: int, operand: str, trans: bool, rows: bool = False) -> Tuple[int, Tuple[int, ...]]:
    """(LDS cycles, (pad, swizzle shift, swizzle mask, row swizzle shift,
    row swizzle mask)) of one operand's tile with the fewest LDS cycles per
    K tile (lds_tile_cycles); ties go to the smaller pad, then to the smaller
    row swizzle, then to the smaller chunk swizzle.  Swizzles
    are tried where the operand's tile rows are k contiguous (B, A^T): masks
    whose XOR stays inside a row's depth_k / 4 chunks and shifts that give
    every row a lane reads one swizzle (B rows atom-N apart; A^T rows
    r * WT0 + i of the interleaved atoms, atom-M * WT0 apart).  With
    ``rows``, A^T also tries row swizzles (lds_tile_accesses' row_swizzle)
    in place of a pad: they move the rows that one instruction touches onto
    different banks.
    Candidates are tried in tie-break order and the search stops at the
    first that is conflict-free (lds_tile_min_cycles).  An operand's tile
    does not depend on the other operand's layout."""
    geo = (mfma, wave_group, wave_tiling, depth_k, trans, trans)
    swizzles = [(0, 0)]
    if operand == "a" and trans:
        wt0, sub_rows = wave_tiling[0], mfma[0] * wave_tiling[0]
        for mask in (1, 3, 7, 15):
            for shift in range(8):
                if (depth_k // 4) % (mask + 1) == 0 and (1 << shift) >= wt0 and sub_rows % ((mask + 1) << shift) == 0:
                    swizzles.append((shift, mask))
    if operand == "b" and not trans:
        for mask in (1, 3, 7, 15):
            for shift in range(5):
                if (depth_k // 4) % (mask + 1) == 0 and mfma[1] % ((mask + 1) << shift) == 0:
                    swizzles.append((shift, mask))

    row_swizzles = [(0, 0)]
    if operand == "a" and trans and rows:
        mt0 = mfma[0] * wave_group[0] * wave_tiling[0]
        row_swizzles += [(sh, rm) for rm in (1, 3, 7) for sh in range(rm.bit_length(), 8)
                         if (mt0 >> sh) > 1 and rm < mt0]
    # a row swizzle stands in for a pad: tried without one
    order = sorted(((p, sw, rs) for p in LDS_PADS for sw in swizzles for rs in row_swizzles if p == 0 or not rs[1]),
                   key=lambda x: (x[0], x[2][1], x[2][0], x[1][1], x[1][0]))
    best = None
    for p, sw, rs in order:
        acc = lds_tile_accesses(*geo, operand, p, sw, rs)
        c = lds_tile_cycles(acc)
        if best is None or c < best[0]:
            best = (c, p, sw, rs)
        if c == lds_tile_min_cycles(acc):
            break
    c, pad, swz, rsw = best
    return c, (pad, swz[0], swz[1], rsw[0], rsw[1])


def _lds_layout(mfma: Tuple[int, ...], wave_group: Tuple[int, int], wave_tiling: Tuple[int, int], depth_k: int,
                trans_a: bool, trans_b: bool, vmem_stage: int = 1) -> Tuple[int, int, int, int, int, int, int, int]:
    """(pad A, pad B, B swizzle shift, B swizzle mask, A^T swizzle shift,
    A^T swizzle mask, A^T row swizzle shift, A^T row swizzle mask): each
    operand's _lds_operand_layout.  An A^T row swizzle costs registers (a
    lane's rows are found one by one; at 256 x 256 depth 24 they spill), so
    it is taken only where its pad-free tile fits more work-groups in a CU's
    LDS than the best layout without one (vmem_stage + 1 stages of both
    tiles) and is as free of bank conflicts."""
    _, (pad_b, b_shift, b_mask, _, _) = _lds_operand_layout(mfma, wave_group, wave_tiling, depth_k, "b", trans_b)
    cyc, a = _lds_operand_layout(mfma, wave_group, wave_tiling, depth_k, "a", trans_a)
    if trans_a:
        cyc_r, a_r = _lds_operand_layout(mfma, wave_group, wave_tiling, depth_k, "a", trans_a, True)
        mt0 = mfma[0] * wave_group[0] * wave_tiling[0]
        mt1 = mfma[1] * wave_group[1] * wave_tiling[1]
        b_floats = depth_k * (mt1 + pad_b) if trans_b else mt1 * (depth_k + pad_b)

        def per_cu(pad_a):
            return MAX_LDS_NUM_BYTES // ((vmem_stage + 1) * (mt0 * (depth_k + pad_a) + b_floats) * 4)
        if cyc_r <= cyc and per_cu(a_r[0]) > per_cu(a[0]):
            a = a_r
    pad_a, a_shift, a_mask, r_shift, r_mask = a
    return pad_a, pad_b, b_shift, b_mask, a_shift, a_mask, r_shift, r_mask


class GemmSolutionConfig:
    """Geometry of one kernel instance (generator.py:857-1055).

    ``mfma`` is (M, N, blocks, K); MT0 = mfma[0] * wave_group[0] * wave_tiling[0]
    and MT1 = mfma[1] * wave_group[1] * wave_tiling[1]; the work-group has
    wave_group[0] * wave_group[1] waves of 64 lanes; ``vmem_stage + 1`` LDS
    buffers hold K tiles of depth ``depth_k``.  Invalid geometry raises
    ``RuntimeError`` at construction, as the reference does.
    """

    def __init__(
        self,
        a_type: DataType,
        b_type: DataType,
        cd_type: DataType,
        scalar_type: DataType,
        mfma: Tuple[int, int, int, int],
        wave_group: Tuple[int, int],
        wave_tiling: Tuple[int, int],
        depth_k: int,
        trans_a: bool,
        trans_b: bool,
        vmem_stage: int = 1,
    ):
        self.a_type = DataType(a_type)
        self.b_type = DataType(b_type)
        self.cd_type = DataType(cd_type)
        self.scalar_type = DataType(scalar_type)
        self.wave_group = tuple(int(x) for x in wave_group)
        self.trans_a = bool(trans_a)
        self.trans_b = bool(trans_b)
        self.mfma = tuple(int(x) for x in mfma)
        self.wave_tiling = tuple(int(x) for x in wave_tiling)
        self.depth_k = int(depth_k)
        self.vmem_stage = int(vmem_stage)
        self.wavefront_size = 64
        self.name = None
        self._validate()

    # ---------------------------------------------------------------- checks
    def _validate(self):
        if self.mfma not in SUPPORTED_MFMAS:
            raise RuntimeError(f"Unsupported MFMA atom: {self.mfma}")
        if any(t != DataType.FP32 for t in (self.a_type, self.b_type, self.cd_type, self.scalar_type)):
            raise RuntimeError("Only FP32 operands are supported")
        if not all(_is_pow2(w) for w in self.wave_group):
            raise RuntimeError(f"Invalid wave group: {self.wave_group}")
        if self.num_workitems > MAX_WORKITEMS:
            raise RuntimeError(f"Work-group of {self.num_workitems} work-items exceeds {MAX_WORKITEMS}")
        if self.wave_tiling[0] not in (1, 2, 4, 8):
            raise RuntimeError(f"Invalid wave tiling along M (1, 2, 4 or 8): {self.wave_tiling}")
        if not 1 <= self.wave_tiling[1] <= 8:
            raise RuntimeError(f"Invalid wave tiling along N (1..8): {self.wave_tiling}")
        if self.trans_b and self.wave_tiling[1] not in (1, 2, 4, 8):
            # B^T's tile is n contiguous: a lane reads its WT1 atoms' operands at once
            raise RuntimeError(f"Invalid wave tiling along N for B^T (1, 2, 4 or 8): {self.wave_tiling}")
        if self.depth_k < 4 or self.depth_k % 4:
            raise RuntimeError(f"depth_k must be a positive multiple of 4: {self.depth_k}")
        if self.depth_k % self.k_block:
            raise RuntimeError(f"depth_k {self.depth_k} is not a multiple of the k block {self.k_block}")
        if self.vmem_stage < 1:
            raise RuntimeError(f"vmem_stage must be >= 1: {self.vmem_stage}")
        if self.lds_usage_bytes > MAX_LDS_NUM_BYTES:
            raise RuntimeError(f"LDS usage exceeds {MAX_LDS_NUM_BYTES}: {self.lds_usage_bytes}")

    # -------------------------------------------------------------- geometry
    @property
    def tile_size(self) -> Tuple[int, int]:
        return (
            self.mfma[0] * self.wave_group[0] * self.wave_tiling[0],
            self.mfma[1] * self.wave_group[1] * self.wave_tiling[1],
        )

    @property
    def num_workitems(self) -> int:
        return self.wave_group[0] * self.wave_group[1] * self.wavefront_size

    @property
    def k_per_lane(self) -> int:
        """Consecutive k values one lane reads per LDS read (KPL)."""
        steps = self.depth_k // self.mfma[3]
        return 4 if steps >= 4 else (2 if steps >= 2 else 1)

    @property
    def k_block(self) -> int:
        """k values covered by one block of KPL MFMA steps."""
        return self.mfma[3] * self.k_per_lane

    @property
    def num_bytes_per_buffer_load(self) -> Tuple[int, int]:
        """Bytes per global load per work-item for A and B (always dwordx4 here)."""
        t0, t1 = self.tile_size
        per_a = t0 * self.depth_k * datatype_size(self.a_type) // self.num_workitems
        per_b = t1 * self.depth_k * datatype_size(self.b_type) // self.num_workitems
        return min(max(per_a, 0), 16), min(max(per_b, 0), 16)

    @property
    def num_dwords_per_buffer_load(self) -> Tuple[int, int]:
        b0, b1 = self.num_bytes_per_buffer_load
        return b0 // 4, b1 // 4

    @property
    def num_elements_per_ds_read(self) -> Tuple[int, int]:
        # A: the WT0 interleaved atoms' operands; B: KPL consecutive k values.
        return self.wave_tiling[0], self.k_per_lane

    @property
    def num_bytes_per_ds_read(self) -> Tuple[int, int]:
        return (
            self.num_elements_per_ds_read[0] * datatype_size(self.a_type),
            self.num_elements_per_ds_read[1] * datatype_size(self.b_type),
        )

    @property
    def num_unrolled_iters(self) -> int:
        return self.depth_k // self.mfma[3]

    # ------------------------------------------------------------------- LDS
    @property
    def lds_layout(self) -> Tuple[int, int, int, int, int, int, int, int]:
        """(pad A, pad B, B swizzle shift, B swizzle mask, A^T swizzle shift,
        A^T swizzle mask, A^T row swizzle shift, A^T row swizzle mask): see
        _lds_layout."""
        return _lds_layout(tuple(self.mfma), tuple(self.wave_group), tuple(self.wave_tiling), self.depth_k,
                           self.trans_a, self.trans_b, self.vmem_stage)

    @property
    def lds_pad_bytes(self) -> Tuple[int, int]:
        pad_a, pad_b = self.lds_layout[:2]
        return pad_a * datatype_size(self.a_type), pad_b * datatype_size(self.b_type)

    @property
    def lds_b_swizzle(self) -> Tuple[int, int]:
        """(shift, mask) of the B-tile chunk swizzle (mask 0: none)."""
        return self.lds_layout[2], self.lds_layout[3]

    @property
    def lds_a_swizzle(self) -> Tuple[int, int]:
        """(shift, mask) of the A^T-tile chunk swizzle (mask 0: none)."""
        return self.lds_layout[4], self.lds_layout[5]

    @property
    def lds_a_row_swizzle(self) -> Tuple[int, int]:
        """(shift, mask) of the A^T-tile row swizzle: row m is stored at row
        m ^ ((m >> shift) & mask) (mask 0: none)."""
        return self.lds_layout[6], self.lds_layout[7]

    def _lds_a_stage_bytes(self) -> int:
        pad_a = self.lds_pad_bytes[0] // datatype_size(self.a_type)
        if self.trans_a:  # [MT0][DK + padA]
            return self.tile_size[0] * (self.depth_k + pad_a) * datatype_size(self.a_type)
        return (self.tile_size[0] + pad_a) * self.depth_k * datatype_size(self.a_type)  # [DK][MT0 + padA]

    @property
    def lds_offset_bytes(self) -> Tuple[int, int]:
        return 0, self._lds_a_stage_bytes()

    @property
    def lds_swap_offset_bytes(self) -> int:
        """Bytes of one LDS stage: A [DK][MT0 + padA] (A^T: [MT0][DK + padA])
        then B [MT1][DK + padB] (B^T: [DK][MT1 + padB])."""
        pad_b = self.lds_pad_bytes[1] // datatype_size(self.b_type)
        if self.trans_b:
            b = self.depth_k * (self.tile_size[1] + pad_b)
        else:
            b = self.tile_size[1] * (self.depth_k + pad_b)
        return self._lds_a_stage_bytes() + b * datatype_size(self.b_type)

    @property
    def lds_usage_bytes(self) -> int:
        return (self.vmem_stage + 1) * self.lds_swap_offset_bytes

    # ----------------------------------------------------------- (de)serial
    def to_dict(self) -> Dict:
        return {
            "a_type": int(self.a_type),
            "b_type": int(self.b_type),
            "cd_type": int(self.cd_type),
            "scalar_type": int(self.scalar_type),
            "wave_group": list(self.wave_group),
            "trans_a": self.trans_a,
            "trans_b": self.trans_b,
            "mfma": list(self.mfma),
            "wave_tiling": list(self.wave_tiling),
            "depth_k": self.depth_k,
            "vmem_stage": self.vmem_stage,
            "wavefront_size": self.wavefront_size,
            "lds_usage_bytes": self.lds_usage_bytes,
            "name": self.name if self.name else "",
        }

    def from_dict(self, d: Dict):
        self.a_type = DataType(d["a_type"])
        self.b_type = DataType(d["b_type"])
        self.cd_type = DataType(d["cd_type"])
        self.scalar_type = DataType(d["scalar_type"])
        self.wave_group = tuple(d["wave_group"])
        self.trans_a = bool(d["trans_a"])
        self.trans_b = bool(d["trans_b"])
        self.mfma = tuple(d["mfma"])
        self.wave_tiling = tuple(d["wave_tiling"])
        self.depth_k = int(d["depth_k"])
        self.vmem_stage = int(d.get("vmem_stage", 1))
        self.wavefront_size = int(d["wavefront_size"])
        self.name = d.get("name", "") or None
        self._validate()
        want = static_lds_bytes(self, GemmOptimizations(1, ws=int(d.get("ws", 0)), ksplit=int(d.get("ksplit", 0))))
        if int(d["lds_usage_bytes"]) != want:
            raise RuntimeError(f"lds_usage_bytes {d['lds_usage_bytes']} does not match the geometry ({want})")
        return self

    @classmethod
    def from_toml(cls, path: str) -> "GemmSolutionConfig":
        d = read_toml(path)
        if d.get("ws") or d.get("ksplit"):  # the config is the computing geometry
            d = dict(d, wave_group=d["compute_wave_group"], wave_tiling=d["compute_wave_tiling"])
        cfg = cls(d["a_type"], d["b_type"], d["cd_type"], d["scalar_type"], d["mfma"], d["wave_group"],
                  d["wave_tiling"], d["depth_k"], d["trans_a"], d["trans_b"], d.get("vmem_stage", 1))
        return cfg.from_dict(d)

    def __repr__(self) -> str:
        return (f"GemmSolutionConfig(mfma={self.mfma}, wave_group={self.wave_group}, "
                f"wave_tiling={self.wave_tiling}, depth_k={self.depth_k}, vmem_stage={self.vmem_stage}, "
                f"tile={self.tile_size})")


class FunctionArgument:
    """One kernel argument (generator.py:94-103)."""

    def __init__(self, typename: str, name: str, offset: Optional[int], num_bytes: int):
        self.typename = typename
        self.name = name
        self.offset = offset
        self.num_bytes = num_bytes
        self.address_space = "global" if typename == "global_buffer" else None


FunctionArgumentList = List[FunctionArgument]

# The explicit kernel arguments of generated_gemm, in order (generator.py:2604-2620).
KERNEL_ARGUMENTS: Tuple[Tuple[str, str, int], ...] = (
    ("global_buffer", "a", 8), ("global_buffer", "b", 8), ("global_buffer", "c", 8), ("global_buffer", "d", 8),
    ("by_value", "m", 4), ("by_value", "n", 4), ("by_value", "k", 4),
    ("by_value", "lda", 4), ("by_value", "ldb", 4), ("by_value", "ldc", 4), ("by_value", "ldd", 4),
    ("by_value", "alpha", 4), ("by_value", "beta", 4),
    ("by_value", "numWorkgroupX", 4), ("by_value", "numWorkgroupY", 4),
)


def default_arguments() -> FunctionArgumentList:
    return [FunctionArgument(t, n, None, s) for t, n, s in KERNEL_ARGUMENTS]


def kernarg_layout(args: FunctionArgumentList) -> List[Tuple[str, int, int]]:
    """(name, offset, size) of each argument, naturally aligned, in order."""
    out, off = [], 0
    for arg in args:
        align = arg.num_bytes
        off = (off + align - 1) // align * align
        out.append((arg.name, off, arg.num_bytes))
        off += arg.num_bytes
    return out


def _check_arguments(args: FunctionArgumentList):
    got = [(a.typename, a.name, a.num_bytes) for a in args]
    if got != list(KERNEL_ARGUMENTS):
        raise RuntimeError(f"generated_gemm takes exactly the reference's 15 arguments, got {got}")


class GpuContext:
    """Holds what ``gemm`` generated: the HIP source and its compile flags.

    ``assembly()`` returns the gfx950 AMD assembly that hipcc produces for that
    source (a build of this project's own code), which the GPU-free virtual
    machine executes.
    """

    def __init__(self):
        self.source: Optional[str] = None
        self.arch: Optional[str] = None
        self.name: Optional[str] = None
        self.defines: Dict[str, int] = {}
        self._asm: Optional[str] = None

    def assembly(self) -> str:
        if self._asm is None:
            if self.source is None:
                raise RuntimeError("gemm() has not generated a kernel into this context")
            self._asm = compile_to_assembly(self.source, self.arch or "gfx950")
        return self._asm


def launch_geometry(config: GemmSolutionConfig, opt: GemmOptimizations) -> Tuple[Tuple[int, int], Tuple[int, int]]:
    """(wave_group, wave_tiling) the kernel is launched with: the config's,
    or with wave specialisation / the in-group K split twice the waves along
    M at half the atoms each (same tile; the loading waves, or the second K
    group, make up the second half)."""
    wg, wt = tuple(config.wave_group), tuple(config.wave_tiling)
    if not (opt.ws or opt.ksplit):
        return wg, wt
    what = "wave specialisation" if opt.ws else "the in-group K split"
    if wt[0] % 2:
        raise RuntimeError(f"{what} needs an even wave_tiling along M: {wt}")
    if opt.ksplit:
        tile_bytes = config.tile_size[0] * config.tile_size[1] * 4
        if tile_bytes > config.lds_usage_bytes:
            raise RuntimeError(f"the in-group K split passes group 1's sums ({tile_bytes} bytes for the "
                               f"{config.tile_size[0]} x {config.tile_size[1]} tile) through its LDS ring of "
                               f"{config.lds_usage_bytes} bytes: use more stages or a deeper K tile")
    if 2 * wg[0] * wg[1] * config.wavefront_size > MAX_WORKITEMS:
        raise RuntimeError(f"{what} doubles the work-group past {MAX_WORKITEMS} work-items")
    return (2 * wg[0], wg[1]), (wt[0] // 2, wt[1])


def ws_counter_bytes(config: GemmSolutionConfig) -> int:
    """Static LDS the wave-specialised K loop adds to the operand buffers: a
    ready and a done counter (uint32) per buffer."""
    return 2 * (config.vmem_stage + 1) * 4


def static_lds_bytes(config: GemmSolutionConfig, opt: GemmOptimizations) -> int:
    """The kernel's static LDS: the operand buffers (lds_usage_bytes), two
    rings of them with the in-group K split, plus the wave-specialised
    loop's counters."""
    n = config.lds_usage_bytes * (2 if opt.ksplit else 1)
    return n + (ws_counter_bytes(config) if opt.ws else 0)


def kernel_defines(config: GemmSolutionConfig, opt: GemmOptimizations, name: str = "generated_gemm") -> Dict[str, object]:
    pad_a = config.lds_pad_bytes[0] // 4
    pad_b = config.lds_pad_bytes[1] // 4
    wg, wt = launch_geometry(config, opt)
    return {
        "SG_ATOM_M": config.mfma[0],
        "SG_WG0": wg[0],
        "SG_WG1": wg[1],
        "SG_WT0": wt[0],
        "SG_WT1": wt[1],
        "SG_WS": int(opt.ws),
        "SG_WS_PD": int(opt.ws_pd),
        "SG_KSPLIT": int(opt.ksplit),
        "SG_DK": config.depth_k,
        "SG_NBUF": config.vmem_stage + 1,
        "SG_WGM": opt.wgm,
        "SG_XCD": opt.xcd,
        "SG_PD": opt.pd,
        "SG_OCC": opt.occ,
        "SG_SPLITK": int(opt.split_k != 1),
        "SG_STREAMK": int(opt.stream_k),
        "SG_MAPK": opt.map_k_idx,
        "SG_PLR": opt.plr,
        "SG_GW": opt.gw,
        "SG_TA": int(config.trans_a),
        "SG_TB": int(config.trans_b),
        "SG_PAD_A": pad_a,
        "SG_PAD_B": pad_b,
        "SG_BSWZ_SHIFT": config.lds_b_swizzle[0],
        "SG_BSWZ_MASK": config.lds_b_swizzle[1],
        "SG_ASWZ_SHIFT": config.lds_a_swizzle[0],
        "SG_ASWZ_MASK": config.lds_a_swizzle[1],
        "SG_ARSW_SHIFT": config.lds_a_row_swizzle[0],
        "SG_ARSW_MASK": config.lds_a_row_swizzle[1],
        "SG_KERNEL_NAME": name,
    }


def gemm(
    context: Optional[GpuContext],
    name: str,
    arch: str,
    config: GemmSolutionConfig,
    opt: GemmOptimizations,
    args: FunctionArgumentList,
) -> str:
    """Returns the HIP source of one specialised kernel (generator.py:1056).

    The text is the kernel template with the configuration prepended as
    ``#define`` lines, so it compiles on its own.  If ``context`` is given it
    also records the source there.
    """
    if arch not in SUPPORTED_ARCHS:
        raise RuntimeError(f"Unsupported arch {arch!r}; this generator targets {SUPPORTED_ARCHS}")
    _check_arguments(args)
    defines = kernel_defines(config, opt, name)
    with open(KERNEL_TEMPLATE, "r") as f:
        template = f.read()
    header = [f"// generated by generator.py for {arch}: {config!r} {opt!r}"]
    header += [f"#define {k} {v}" for k, v in defines.items()]
    src = "\n".join(header) + "\n" + template
    if context is not None:
        context.source = src
        context.arch = arch
        context.name = name
        context.defines = defines
        context._asm = None
    return src


def compile_to_assembly(kern_str: str, arch: str = "gfx950") -> str:
    """AMD assembly of a generated kernel (this project's own build)."""
    with tempfile.TemporaryDirectory() as tmp:
        src = os.path.join(tmp, "k.hip")
        out = os.path.join(tmp, "k.s")
        with open(src, "w") as f:
            f.write(kern_str)
        cmd = [DEFAULT_HIPCC_PATH, "-S", "--cuda-device-only", f"--offload-arch={arch}",
               *HIPCC_KERNEL_FLAGS, src, "-o", out]
        ret = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE)
        if ret.returncode:
            raise RuntimeError(f"hipcc -S failed:\n{ret.stderr.decode(errors='replace')}")
        with open(out) as f:
            return f.read()


def _toml_value(v) -> str:
    if isinstance(v, bool):
        return "true" if v else "false"
    if isinstance(v, int):
        return str(v)
    if isinstance(v, float):
        return repr(v)
    if isinstance(v, str):
        esc = v.replace("\\", "\\\\").replace('"', '\\"')
        return f'"{esc}"'
    if isinstance(v, (list, tuple)):
        return "[" + ", ".join(_toml_value(x) for x in v) + "]"
    raise TypeError(f"unsupported TOML value {v!r}")


def write_toml(d: Dict, path: str):
    """Flat TOML writer (the subset tomli_w produced for the reference)."""
    with open(path, "w") as f:
        for k, v in d.items():
            f.write(f"{k} = {_toml_value(v)}\n")


def read_toml(path: str) -> Dict:
    try:
        import tomllib  # Python >= 3.11
    except ImportError:  # pragma: no cover - depends on the interpreter
        import tomli as tomllib
    with open(path, "rb") as f:
        return tomllib.load(f)


def compile(kern_name: str, kern_str: str, arch: str, output_folder: str, gemm_config: GemmSolutionConfig,
            opt: Optional[GemmOptimizations] = None, extra_keys: Optional[Dict] = None,
            verbose: bool = False) -> int:
    """Builds ``<out>/<name>.co`` and writes ``<out>/<name>.toml`` (generator.py:2534-2569).

    Returns 0 on success and the failing step's non-zero code otherwise; on
    failure no ``.toml`` is written, so a stale pair is never left behind.
    """
    os.makedirs(output_folder, exist_ok=True)
    src_path = os.path.join(output_folder, f"{kern_name}.hip")
    co_path = os.path.join(output_folder, f"{kern_name}.co")
    toml_path = os.path.join(output_folder, f"{kern_name}.toml")
    with open(src_path, "w") as f:
        f.write(kern_str)
    tmp_co = co_path + ".tmp"
    # a plain amdhsa ELF code object (no offload bundle), like the reference's .co
    cmd = [DEFAULT_HIPCC_PATH, "--cuda-device-only", "-c", "--no-gpu-bundle-output",
           f"--offload-arch={arch}", *HIPCC_KERNEL_FLAGS,
           "-Rpass-analysis=kernel-resource-usage", src_path, "-o", tmp_co]
    ret = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE)
    if ret.returncode:
        if verbose:
            sys.stderr.write(ret.stderr.decode(errors="replace"))
        if os.path.exists(tmp_co):
            os.remove(tmp_co)
        return ret.returncode
    os.replace(tmp_co, co_path)
    d = gemm_config.to_dict()
    if not d["name"]:
        d["name"] = kern_name
    if opt is not None and (opt.ws or opt.ksplit):
        # the launch geometry for every runner (the reference's included);
        # the computing waves' own geometry beside it
        wg, wt = launch_geometry(gemm_config, opt)
        d["compute_wave_group"], d["compute_wave_tiling"] = d["wave_group"], d["wave_tiling"]
        d["wave_group"], d["wave_tiling"] = list(wg), list(wt)
        d["lds_usage_bytes"] = static_lds_bytes(gemm_config, opt)  # the code object's whole static LDS
    d["arch"] = arch
    if opt is not None:
        d.update(opt.to_dict())
    remarks = ret.stderr.decode(errors="replace")
    d.update(parse_resource_usage(remarks))
    if opt is not None and opt.split_k != 1:
        d.update({f"splitk_{k}": v for k, v in parse_resource_usage(remarks, "generated_gemm_splitk").items()})
    if opt is not None and opt.stream_k:
        d.update({f"streamk_{k}": v for k, v in parse_resource_usage(remarks, "generated_gemm_streamk").items()})
    if extra_keys:
        d.update(extra_keys)
    write_toml(d, toml_path)
    return 0


_RESOURCE_KEYS = {
    "VGPRs": "vgprs",
    "AGPRs": "agprs",
    "TotalSGPRs": "sgprs",
    "ScratchSize [bytes/lane]": "scratch_bytes_per_lane",
    "Occupancy [waves/SIMD]": "occupancy_waves_per_simd",
    "LDS Size [bytes/block]": "lds_bytes_compiled",
}


def parse_resource_usage(remarks: str, kernel: str = "generated_gemm") -> Dict[str, int]:
    """The compiler's kernel-resource-usage remark for ``kernel`` as integer
    TOML keys (a code object may hold several kernels)."""
    out: Dict[str, int] = {}
    current = None
    for line in remarks.splitlines():
        if "remark:" not in line:
            continue
        body = line.split("remark:", 1)[1].strip()
        if body.startswith("Function Name:"):
            current = body[len("Function Name:"):].split("[")[0].strip()
            continue
        if current is not None and current != kernel:
            continue
        for label, key in _RESOURCE_KEYS.items():
            if body.startswith(label + ":"):
                val = body[len(label) + 1:].split("[")[0].strip()
                try:
                    out[key] = int(val)
                except ValueError:
                    pass
    return out


def build_kernel(output_folder: str, config: GemmSolutionConfig, opt: GemmOptimizations,
                 kern_name: str = "generated_gemm", arch: str = "gfx950", verbose: bool = True) -> Tuple[str, str]:
    """gemm + compile; returns the (.co, .toml) paths or raises RuntimeError."""
    # the exported symbol stays generated_gemm whatever the files are called
    src = gemm(None, "generated_gemm", arch, config, opt, default_arguments())
    rc = compile(kern_name, src, arch, output_folder, config, opt, verbose=verbose)
    if rc:
        raise RuntimeError(f"compile of {kern_name} failed with code {rc}")
    return os.path.join(output_folder, f"{kern_name}.co"), os.path.join(output_folder, f"{kern_name}.toml")


# Default instance of the CLI: the catalog's instance for the 4096^3 headline
# problem, one 256 x 256 work-group of eight waves per CU (in the layout
# trans_a / trans_b ask for).
def default_config(trans_a: bool = False, trans_b: bool = False) -> Tuple[GemmSolutionConfig, GemmOptimizations]:
    cfg = GemmSolutionConfig(DataType.FP32, DataType.FP32, DataType.FP32, DataType.FP32,
                             MFMA_32x32x2, (4, 2), (2, 4), 16, trans_a, trans_b, vmem_stage=2)
    opt = GemmOptimizations(1, wgm=8, plr=3, gw=1, map_k_idx=0, xcd=8)
    return cfg, opt


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="Generate the gfx950 SGEMM code object and its .toml")
    ap.add_argument(dest="output_folder", action="store", type=str, help="Output folder")
    ap.add_argument("--arch", dest="arch", action="store", choices=list(SUPPORTED_ARCHS), default="gfx950")
    ap.add_argument("--trans-a", action="store_true", help="op(A) = A^T: A stored k x m (lda >= k)")
    ap.add_argument("--trans-b", action="store_true", help="op(B) = B^T: B stored n x k (ldb >= n)")
    args = ap.parse_args(argv)
    cfg, opt = default_config(args.trans_a, args.trans_b)
    src = gemm(None, "generated_gemm", args.arch, cfg, opt, default_arguments())
    rc = compile("generated_gemm", src, args.arch, args.output_folder, cfg, opt, verbose=True)
    if rc == 0:
        print(f"wrote {args.output_folder}/generated_gemm.co and {args.output_folder}/generated_gemm.toml")
    return rc


if __name__ == "__main__":
    sys.exit(main())
