// FP32 column-major NN SGEMM for CDNA4 (gfx950): D = alpha * A * B + beta * C.
//
// One translation unit per tuned configuration.  The generator compiles this
// file with `hipcc --cuda-device-only -c --offload-arch=gfx950 -DSG_...=<value>` and the
// resulting code object exports one kernel, `generated_gemm`, whose explicit
// kernel arguments are laid out byte-for-byte like the reference emitter's
// (generator.py:2604-2620, packed by generator_runner.cpp:132-148):
//
//   offset  0 a   8 b   16 c   24 d          (global float pointers)
//   offset 32 m  36 n   40 k   44 lda  48 ldb  52 ldc  56 ldd   (uint32)
//   offset 60 alpha     64 beta                 (float)
//   offset 68 numWorkgroupX  72 numWorkgroupY   (int32)      -> 76 B, padded to 80
//
// Launch: grid = (numWorkgroupX, numWorkgroupY) workgroups of
// SG_WG0 * SG_WG1 * 64 work-items; all LDS is static (the runner passes 0 B of
// dynamic LDS, generator_runner.cpp:189).  numWorkgroupX = ceil(m / MT0),
// numWorkgroupY = ceil(n / MT1) with MT0 = atom_m * WG0 * WT0 and
// MT1 = atom_n * WG1 * WT1 (generator.py:898-903).  Any m, n, k, any leading
// dimensions and any 4-byte aligned pointers take the vector path: buffer
// loads and stores of float4 chunks need dword alignment only, and their
// range check is per dword.  Chunks wholly past m or n load a chunk inside
// the tile instead; a chunk straddling the end of an operand reads 0 past it;
// the epilogue stores only elements inside D.  A K remainder shifts the K
// origin so that the first K tile is the partial one, its missing values
// loaded as zeros (element by element for chunks along k that straddle it).
// Only a K remainder with a single K tile (per K group under the in-group K
// split, SG_KSPLIT), or with a rotated first K tile (SG_MAPK > 1), takes the
// element-wise path.  The host side (shim, runner)
// checks that lda >= m, ldb >= k, ldc >= m, ldd >= m before every launch.
//
// Data path per K tile of depth DK:
//   HBM --buffer_load_dwordx4--> VGPR --ds_write_b128--> LDS (NBUF buffers)
//   LDS --ds_read_b{32,64,128}--> VGPR --v_mfma_f32_{32x32x2,16x16x4}_f32--> accumulators
// and after the K loop accumulators --(alpha)--> LDS column chunk --(beta * C)-->
// buffer_store_dwordx4 down whole columns of D.
//
// LDS layouts (floats):
//   A tile: [DK][MT0 + PAD_A]  -- one k per row, m contiguous; written straight
//           from the column-major global rows (coalesced, conflict-free).
//   B tile: [MT1][DK + PAD_B]  -- one n per row, k contiguous; written straight
//           from the column-major global columns.  In the NN/TN layouts the
//           16-byte chunks of a row may be XOR-swizzled: chunk c of row n sits
//           at chunk c ^ ((n >> SG_BSWZ_SHIFT) & SG_BSWZ_MASK) of that row, so
//           that the ds_write_b128 of two rows per 8 lanes and the
//           ds_read_b128 of 16 rows per cycle both hit distinct banks without
//           a pad (gfx950 serves b128 writes 8 lanes x 32 banks per cycle,
//           b128 reads 16 lanes x 64 banks, measured by profiler/lds_probe).
//
// K permutation.  An MFMA atom with atom_k = 2 (32x32x2) or 4 (16x16x4) feeds
// lane group g = lane / atom_m one k value.  Any bijection between the k values
// of a block and (MFMA step j, lane group g) gives the same sum as long as A and
// B use the same one, so within a block of KB = atom_k * KPL values lane group g
// takes k = block + g * KPL + j at step j (j < KPL).  A lane then reads KPL
// consecutive k of one B column with a single ds_read_b128 (KPL = 4).
//
// M interleave.  Atom i of a wave's WT0 atoms along M owns the rows
// wave_row + r * WT0 + i (r < atom_m), so one lane's A operands for the WT0
// atoms at one k are WT0 consecutive floats in an LDS row: one ds_read_b128
// for WT0 = 4.  The same interleave makes the epilogue's WT0 values per
// accumulator slot consecutive rows of D, stored with one dwordx4 per slot.
//
// Work-group order.  Tiles are first spread so that each of the 8 XCDs (which
// receive work-groups round-robin by linear id) owns a contiguous range of
// logical tiles (SG_XCD), then grouped SG_WGM tiles wide along M
// (generator.py:1437-1464 semantics, extended to a partial last group), and
// the starting K tile can be rotated by (tile_x & (SG_MAPK - 1))
// (generator.py:1506-1514, :1724-1744).

#include <hip/hip_runtime.h>
#include <stdint.h>

#ifndef SG_ATOM_M
#define SG_ATOM_M 32
#endif
#ifndef SG_WG0
#define SG_WG0 2
#endif
#ifndef SG_WG1
#define SG_WG1 2
#endif
#ifndef SG_WT0
#define SG_WT0 4
#endif
#ifndef SG_WT1
#define SG_WT1 4
#endif
#ifndef SG_DK
#define SG_DK 16
#endif
#ifndef SG_NBUF
#define SG_NBUF 2
#endif
#ifndef SG_WGM
#define SG_WGM 1
#endif
#ifndef SG_XCD
#define SG_XCD 0
#endif
#ifndef SG_MAPK
#define SG_MAPK 0
#endif
#ifndef SG_PLR
#define SG_PLR 1
#endif
#ifndef SG_PD
#define SG_PD 1
#endif
#ifndef SG_OCC
#define SG_OCC 0
#endif
#ifndef SG_GW
#define SG_GW 1
#endif
#ifndef SG_PAD_A
#define SG_PAD_A 0
#endif
#ifndef SG_BSWZ_SHIFT
#define SG_BSWZ_SHIFT 0
#endif
#ifndef SG_BSWZ_MASK
#define SG_BSWZ_MASK 0
#endif
#ifndef SG_PAD_B
#define SG_PAD_B 4
#endif
#ifndef SG_ASWZ_SHIFT
#define SG_ASWZ_SHIFT 0
#endif
#ifndef SG_ASWZ_MASK
#define SG_ASWZ_MASK 0
#endif
#ifndef SG_ARSW_SHIFT
#define SG_ARSW_SHIFT 0
#endif
#ifndef SG_ARSW_MASK
#define SG_ARSW_MASK 0
#endif
#ifndef SG_TA
#define SG_TA 0
#endif
#ifndef SG_TB
#define SG_TB 0
#endif
#ifndef SG_WS
#define SG_WS 0
#endif
#ifndef SG_WS_PD
#define SG_WS_PD 2
#endif
#ifndef SG_KSPLIT
#define SG_KSPLIT 0
#endif
#ifndef SG_KERNEL_NAME
#define SG_KERNEL_NAME generated_gemm
#endif
#ifndef SG_SPLITK
#define SG_SPLITK 0
#endif
#ifndef SG_KERNEL_NAME_SPLITK
#define SG_KERNEL_NAME_SPLITK generated_gemm_splitk
#endif
#ifndef SG_STREAMK
#define SG_STREAMK 0
#endif
#ifndef SG_KERNEL_NAME_STREAMK
#define SG_KERNEL_NAME_STREAMK generated_gemm_streamk
#endif

namespace sg {

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Word 3 of a raw (untyped, stride 0) buffer resource on gfx9-family GPUs.
constexpr int BUFFER_RSRC_WORD3 = 0x00020000;
// Cache-policy operand of the buffer intrinsics on gfx94x/gfx950: bit 0 sc0,
// bit 1 nt, bit 4 sc1; sc1 alone is device scope (coherent across XCDs).
constexpr int CPOL_SC1 = 0x10;
constexpr int CPOL_NT = 0x2;

template <int N> struct Vec;
template <> struct Vec<1> { typedef float type; };
template <> struct Vec<2> { typedef f32x2 type; };
template <> struct Vec<4> { typedef f32x4 type; };

template <int AM> struct Atom;

// v_mfma_f32_32x32x2_f32: lane l supplies A[l % 32][l / 32] and B[l / 32][l % 32];
// accumulator slot q of lane l holds D[(q % 4) + 8 * (q / 4) + 4 * (l / 32)][l % 32].
template <> struct Atom<32> {
    static constexpr int M = 32, N = 32, K = 2, ACC = 16;
    typedef f32x16 acc_t;
    __device__ static __forceinline__ acc_t mfma(float a, float b, acc_t c) {
        return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
    }
    __device__ static __forceinline__ int row(int q, int lane) {
        return (q & 3) + 8 * (q >> 2) + 4 * (lane >> 5);
    }
};

// v_mfma_f32_16x16x4_f32: lane l supplies A[l % 16][l / 16] and B[l / 16][l % 16];
// accumulator slot q of lane l holds D[q + 4 * (l / 16)][l % 16].
template <> struct Atom<16> {
    static constexpr int M = 16, N = 16, K = 4, ACC = 4;
    typedef f32x4 acc_t;
    __device__ static __forceinline__ acc_t mfma(float a, float b, acc_t c) {
        return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
    }
    __device__ static __forceinline__ int row(int q, int lane) { return q + 4 * (lane >> 4); }
};

// WG0 x WG1 waves of WT0 x WT1 atoms describe the launch (the .toml's
// wave_group / wave_tiling: NT work-items, an MT0 x MT1 tile).  With WS (wave
// specialisation) the first half of the waves along M computes the whole tile
// -- WG0 / 2 x WG1 waves of 2 * WT0 x WT1 atoms -- and the other half only
// moves K tiles from memory to LDS.  With KS (K split inside the work-group)
// each half is a group of that shape that loads and multiplies half of the K
// tiles of the whole tile in an LDS ring of its own; the groups' sums meet in
// LDS.  Otherwise every wave does both jobs for the whole K range.
template <int AM, int WG0, int WG1, int WT0, int WT1, int DK, int NBUF, int PAD_A, int PAD_B, bool TA, bool TB,
          bool WS, bool KS>
struct Geometry {
    typedef Atom<AM> atom;
    static constexpr int NT = WG0 * WG1 * 64;
    static constexpr int MT0 = atom::M * WG0 * WT0;
    static constexpr int MT1 = atom::N * WG1 * WT1;
    static constexpr bool HALVES = WS || KS;            // the waves split into two halves along M
    static constexpr int CWG0 = HALVES ? WG0 / 2 : WG0;  // computing waves along M (of one group)
    static constexpr int CWT0 = HALVES ? WT0 * 2 : WT0;  // their atoms along M
    static constexpr int CWAVES = CWG0 * WG1;            // computing waves (of one group)
    static constexpr int CNT = CWAVES * 64;              // their work-items
    // work-items that load one LDS ring's K tiles: every one, the loading
    // half (WS) or one group's (KS)
    static constexpr int LT = WS ? NT - CNT : (KS ? CNT : NT);
    // k values a lane reads per LDS read of B (and MFMA steps per k block)
    static constexpr int KPL = (DK / atom::K >= 4) ? 4 : ((DK / atom::K >= 2) ? 2 : 1);
    static constexpr int KB = atom::K * KPL;
    // A tile: [DK][MT0 + PAD_A] (m contiguous), or for A^T [MT0][DK + PAD_A]
    // (k contiguous, like B); B tile: [MT1][DK + PAD_B] (k contiguous), or
    // for B^T [DK][MT1 + PAD_B] (n contiguous, like A): the tile keeps the
    // operand's contiguous dimension, so every LDS write is a 16-byte row piece
    static constexpr int A_LD = TA ? DK + PAD_A : MT0 + PAD_A;  // LDS row stride of the A tile (floats)
    static constexpr int B_LD = TB ? MT1 + PAD_B : DK + PAD_B;  // LDS row stride of the B tile (floats)
    static constexpr int A_STAGE = TA ? MT0 * A_LD : DK * A_LD;
    static constexpr int B_STAGE = TB ? DK * B_LD : MT1 * B_LD;
    static constexpr int STAGE = A_STAGE + B_STAGE;
    static constexpr int LDS_FLOATS = NBUF * STAGE;
    // float4 chunks each thread moves per K tile
    static constexpr int A_CHUNKS = MT0 * DK / 4;
    static constexpr int B_CHUNKS = MT1 * DK / 4;
    static constexpr int LA = (A_CHUNKS + LT - 1) / LT;
    static constexpr int LB = (B_CHUNKS + LT - 1) / LT;

    static_assert(DK % 4 == 0, "DK must be a multiple of 4");
    static_assert(DK % KB == 0, "DK must be a multiple of the k block");
    static_assert(MT0 % 4 == 0, "MT0 must be a multiple of 4");
    static_assert(CWT0 == 1 || CWT0 == 2 || CWT0 == 4 || CWT0 == 8, "WT0 must be 1, 2, 4 or 8");
    static_assert(!HALVES || (WG0 % 2 == 0), "wave specialisation / the K split halve an even wave group along M");
    static_assert(!(WS && KS), "wave specialisation and the in-group K split exclude each other");
    static_assert(WT1 >= 1 && WT1 <= 8, "WT1 must be in [1, 8]");
    static_assert(!TB || WT1 == 1 || WT1 == 2 || WT1 == 4 || WT1 == 8, "B^T reads WT1 consecutive floats");
    static_assert(PAD_A % 4 == 0 && PAD_B % 4 == 0, "LDS pads keep 16-byte rows");
    static_assert(NBUF >= 2, "at least two LDS buffers");
    static_assert(LDS_FLOATS * 4 <= 163840, "LDS tile exceeds the 160 KiB of a gfx950 CU");
};

typedef Geometry<SG_ATOM_M, SG_WG0, SG_WG1, SG_WT0, SG_WT1, SG_DK, SG_NBUF, SG_PAD_A, SG_PAD_B, SG_TA != 0, SG_TB != 0,
                 SG_WS != 0, SG_KSPLIT != 0> G;
static_assert(!SG_WS || (!SG_SPLITK && !SG_STREAMK), "the wave-specialised K loop has no split-K / stream-K variant");
static_assert(!SG_KSPLIT || (!SG_SPLITK && !SG_STREAMK && SG_MAPK <= 1),
              "the in-group K split has no split-K / stream-K variant and no K rotation");

// B-tile chunk swizzle of row n (0: rows stored straight).  The XOR stays
// inside a row when its chunk count is a multiple of MASK + 1, and a lane's
// rows differ by multiples of the atom's N, which leave the swizzle alone
// when atom N is a multiple of (MASK + 1) << SHIFT.
__device__ __forceinline__ constexpr int bswz(int n) { return (n >> SG_BSWZ_SHIFT) & SG_BSWZ_MASK; }
static_assert(SG_BSWZ_MASK == 0 || (SG_BSWZ_MASK & (SG_BSWZ_MASK + 1)) == 0, "swizzle mask is 2^b - 1");
static_assert((SG_DK / 4) % (SG_BSWZ_MASK + 1) == 0, "swizzle leaves the B row");
static_assert(G::atom::N % ((SG_BSWZ_MASK + 1) << SG_BSWZ_SHIFT) == 0, "swizzle varies across a lane's rows");
static_assert(SG_BSWZ_MASK == 0 || !SG_TB, "the B swizzle is for the layouts with k contiguous in B");

// A^T-tile chunk swizzle of row m, the same scheme: a lane reads rows
// wm * SM + r * WT0 + i (SM = atom M * WT0, i < WT0 the atom), which share
// one swizzle when SHIFT >= log2(WT0) and SM is a multiple of
// (MASK + 1) << SHIFT.
__device__ __forceinline__ constexpr int aswz(int m) { return (m >> SG_ASWZ_SHIFT) & SG_ASWZ_MASK; }
static_assert(SG_ASWZ_MASK == 0 || (SG_ASWZ_MASK & (SG_ASWZ_MASK + 1)) == 0, "swizzle mask is 2^b - 1");
static_assert((SG_DK / 4) % (SG_ASWZ_MASK + 1) == 0, "swizzle leaves the A^T row");
static_assert(SG_ASWZ_MASK == 0 || ((1 << SG_ASWZ_SHIFT) >= G::CWT0 &&
                                    (G::atom::M * G::CWT0) % ((SG_ASWZ_MASK + 1) << SG_ASWZ_SHIFT) == 0),
              "swizzle varies across a lane's rows");
static_assert(SG_ASWZ_MASK == 0 || SG_TA, "the A swizzle is for the layout with k contiguous in A^T");

// A^T-tile row swizzle: row m is stored at row arow(m).  The XOR touches
// only bits below SHIFT, so it is a bijection on [0, MT0).  It moves the
// rows one LDS instruction touches (rows r * WT0 + i of the lanes of one
// atom i, or the rows of one write cycle) onto different banks where a
// pad would otherwise do it.  Rows a lane reads are found one by one.
__device__ __forceinline__ constexpr int arow(int m) { return m ^ ((m >> SG_ARSW_SHIFT) & SG_ARSW_MASK); }
static_assert(SG_ARSW_MASK == 0 || ((SG_ARSW_MASK & (SG_ARSW_MASK + 1)) == 0 && (1 << SG_ARSW_SHIFT) > SG_ARSW_MASK &&
                                    SG_ARSW_MASK < G::MT0),
              "the row swizzle is a bijection on the tile's rows");
static_assert(SG_ARSW_MASK == 0 || SG_TA, "the row swizzle is for the layout with k contiguous in A^T");

// Reads WT0 consecutive floats (the A operands of the WT0 interleaved atoms).
template <int W> __device__ __forceinline__ void lds_read_row(const float* p, float (&out)[W]) {
    if constexpr (W == 1) {
        out[0] = p[0];
    } else if constexpr (W == 2) {
        f32x2 v = *reinterpret_cast<const f32x2*>(p);
        out[0] = v.x; out[1] = v.y;
    } else {
#pragma unroll
        for (int h = 0; h < W / 4; ++h) {
            f32x4 v = *reinterpret_cast<const f32x4*>(p + 4 * h);
            out[4 * h + 0] = v.x; out[4 * h + 1] = v.y; out[4 * h + 2] = v.z; out[4 * h + 3] = v.w;
        }
    }
}

template <int W> __device__ __forceinline__ void store_row(float* p, const float (&v)[W]) {
    if constexpr (W == 1) {
        p[0] = v[0];
    } else if constexpr (W == 2) {
        f32x2 t; t.x = v[0]; t.y = v[1];
        *reinterpret_cast<f32x2*>(p) = t;
    } else {
#pragma unroll
        for (int h = 0; h < W / 4; ++h) {
            f32x4 t; t.x = v[4 * h]; t.y = v[4 * h + 1]; t.z = v[4 * h + 2]; t.w = v[4 * h + 3];
            *reinterpret_cast<f32x4*>(p + 4 * h) = t;
        }
    }
}

template <int W> __device__ __forceinline__ void global_load_row(const float* p, float (&v)[W]) {
    if constexpr (W == 1) {
        v[0] = p[0];
    } else if constexpr (W == 2) {
        f32x2 t = *reinterpret_cast<const f32x2*>(p);
        v[0] = t.x; v[1] = t.y;
    } else {
#pragma unroll
        for (int h = 0; h < W / 4; ++h) {
            f32x4 t = *reinterpret_cast<const f32x4*>(p + 4 * h);
            v[4 * h] = t.x; v[4 * h + 1] = t.y; v[4 * h + 2] = t.z; v[4 * h + 3] = t.w;
        }
    }
}

// Tags selecting the vector (float4 chunk) or element-wise K loop.
struct FastPath { static constexpr bool slow = false; };
struct SlowPath { static constexpr bool slow = true; };
// Tags marking the load of a partial first K tile (shifted K origin) or any other.
struct Head { static constexpr bool on = true; };
struct NoHead { static constexpr bool on = false; };

// Scheduling masks of __builtin_amdgcn_sched_group_barrier.
constexpr int SCHED_MFMA = 0x008;
constexpr int SCHED_VMEM_READ = 0x020;
constexpr int SCHED_DS_READ = 0x100;
constexpr int SCHED_DS_WRITE = 0x200;

// Orders one k block's instructions as MFMA, memory op, MFMA, memory op, ...:
// first the NREAD LDS reads (operands of the next block), then the NWRITE LDS
// writes and NLOAD global loads of the refill, alternating.  Memory ops beyond
// the MFMA count are left to the scheduler.
template <int NMFMA, int NREAD, int NWRITE, int NLOAD>
__device__ __forceinline__ void interleave_block() {
#pragma unroll
    for (int i = 0; i < NMFMA; ++i) {
        __builtin_amdgcn_sched_group_barrier(SCHED_MFMA, 1, 0);
        if (i < NREAD) {
            __builtin_amdgcn_sched_group_barrier(SCHED_DS_READ, 1, 0);
        } else {
            const int j = i - NREAD;
            if (j < 2 * NWRITE && j < 2 * NLOAD) {
                if (j % 2 == 0) __builtin_amdgcn_sched_group_barrier(SCHED_DS_WRITE, 1, 0);
                else __builtin_amdgcn_sched_group_barrier(SCHED_VMEM_READ, 1, 0);
            } else if (j < NWRITE + NLOAD) {
                if (NWRITE > NLOAD) __builtin_amdgcn_sched_group_barrier(SCHED_DS_WRITE, 1, 0);
                else __builtin_amdgcn_sched_group_barrier(SCHED_VMEM_READ, 1, 0);
            }
        }
    }
}

// Work-group `lin` (of `total`, dispatched round-robin) runs on XCD
// lin % SG_XCD; renumber so that each XCD owns one contiguous range of the
// logical order (XCD x gets total / SG_XCD work-groups, one more for the first
// total % SG_XCD XCDs).  A bijection on [0, total).
__device__ __forceinline__ int xcd_order(int lin, int total) {
    if constexpr (SG_XCD > 1) {
        const int x = lin % SG_XCD, q = total / SG_XCD, r = total % SG_XCD;
        return x * q + (x < r ? x : r) + lin / SG_XCD;
    }
    return lin;
}

// Maps a logical tile index to (tile_x, tile_y): groups SG_WGM tiles wide
// along M, column by column inside a group.
__device__ __forceinline__ void tile_coords(int z, int nwgx, int nwgy, int& tx, int& ty) {
    if constexpr (SG_WGM > 1) {
        const int span = SG_WGM * nwgy;
        const int group = z / span;
        const int first_x = group * SG_WGM;
        const int rem = nwgx - first_x;
        const int width = rem < SG_WGM ? rem : SG_WGM;
        const int in_group = z - group * span;
        tx = first_x + in_group % width;
        ty = in_group / width;
    } else {
        tx = z % nwgx;
        ty = z / nwgx;
    }
}

}  // namespace sg

// SG_OCC > 0 asks the compiler for at least SG_OCC waves per SIMD (registers
// capped at 512 / SG_OCC per lane), so that SG_OCC work-groups of one wave
// per SIMD can share a CU and hide each other's barrier waits.
#if SG_OCC > 0
#define SG_OCC_ATTR __attribute__((amdgpu_waves_per_eu(SG_OCC, SG_OCC)))
#else
#define SG_OCC_ATTR
#endif

// How a work-group's accumulators leave the K loop.  FIX_NONE: straight to
// the epilogue.  Otherwise the work-group covered part of the tile's K range:
// it stores its raw accumulators as partial `slot` of the `parts` partials at
// `ws`, takes a ticket, and the last of the `parts` arrivals combines the
// partials and runs the epilogue.  FIX_SPLIT re-reads partials 0, 1, ...,
// parts - 1 (its own included) and sums them in that order; FIX_STREAM
// (parts == 2) adds the other partial to its own accumulators -- a two-term
// sum, the same bits whichever work-group arrives last.  Either way the result
// does not depend on timing.
constexpr int FIX_NONE = 0, FIX_SPLIT = 1, FIX_STREAM = 2;
struct Fixup {
    int kind;
    float* ws;          // partial 0 of this tile (FIX_SPLIT) or of this stream-K boundary (FIX_STREAM)
    uint32_t* ticket;   // zero before the first arrival; re-armed to zero by the last one
    uint32_t parts;
    uint32_t slot;
};

// One output tile (tx, ty): the K loop over [k_first, k_first + k) of the
// operands, the fix-up, then the epilogue.  c and d may be one matrix (an
// in-place update of C): an element of C is read only by the lane that then
// writes that element of D, in the one epilogue that finishes its tile, so
// neither pointer is declared restrict.
__device__ __forceinline__ void gemm_tile(const float* __restrict__ a, const float* __restrict__ b,
                                          const float* c, float* d,
                                          uint32_t m, uint32_t n, uint32_t k_total,
                                          uint32_t lda, uint32_t ldb, uint32_t ldc, uint32_t ldd,
                                          float alpha, float beta, int tx, int ty, uint32_t k_first, uint32_t k,
                                          const Fixup fx, const int tid) {
    using namespace sg;
    typedef G::atom AT;
    typedef AT::acc_t acc_t;
    constexpr int NT = G::NT, MT0 = G::MT0, MT1 = G::MT1, DK = SG_DK, NBUF = SG_NBUF;
    constexpr int WT0 = G::CWT0, WT1 = SG_WT1, KPL = G::KPL, KB = G::KB;
    // K-tile loads: work-item ltid of LT (every work-item, or with wave
    // specialisation those of the loading waves; the computing waves' ltid
    // is a valid index they never use)
    constexpr int LT = G::LT;
    constexpr bool TA = SG_TA != 0, TB = SG_TB != 0;

    const int lane = tid & 63;
    // wave-uniform (a scalar register): the epilogue's buffer descriptors
    // derived from it then need no per-lane waterfall loop
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // with the in-group K split, group 1's waves repeat group 0's layout
    const int kgrp = SG_KSPLIT ? wave / G::CWAVES : 0;
    const int cwave = SG_KSPLIT ? wave % G::CWAVES : wave;
    const int wm = cwave % G::CWG0;
    const int wn = cwave / G::CWG0;
    const bool loader_wave = SG_WS && wave >= G::CWAVES;
    const int ltid = SG_WS ? (tid >= G::CNT ? tid - G::CNT : tid % LT) : (SG_KSPLIT ? tid % G::CNT : tid);
#if SG_KSPLIT
    // one LDS ring per K group; this wave's group's ring
    __shared__ __attribute__((aligned(16))) float lds_rings[2 * G::LDS_FLOATS];
    float* const lds = lds_rings + kgrp * G::LDS_FLOATS;
#else
    __shared__ __attribute__((aligned(16))) float lds[G::LDS_FLOATS];
#endif
    const uint32_t row0 = (uint32_t)tx * MT0;
    const uint32_t col0 = (uint32_t)ty * MT1;

    // Bytes from each operand's first element to just past the last one the
    // caller guarantees (column-major with its leading dimension): the loads'
    // buffer descriptors never reach past them.
    auto extent = [](uint32_t cols, uint32_t ld, uint32_t rows) -> uint64_t {
        return (cols && rows) ? ((uint64_t)(cols - 1) * ld + rows) * 4u : 0u;
    };
    const char* const a_lim = reinterpret_cast<const char*>(a) + (TA ? extent(m, lda, k_total) : extent(k_total, lda, m));
    const char* const b_lim = reinterpret_cast<const char*>(b) + (TB ? extent(k_total, ldb, n) : extent(n, ldb, k_total));
    // the K range [k_first, k_first + k): a range of whole K tiles, the last
    // one possibly cut at k_total
    a += TA ? (size_t)k_first : (size_t)k_first * lda;
    b += TB ? (size_t)k_first * ldb : (size_t)k_first;
    const int ktiles = (int)((k + DK - 1) / DK);
    // Uniform per work-group: every tile takes the vector path (float4 chunks
    // through buffer loads, dword alignment is enough) except for the K
    // remainders it cannot take below; those load and store element by
    // element with bounds checks.
    //
    // K remainder: the K origin moves back by kshift, so K tile t covers k in
    // [t*DK - kshift, (t+1)*DK - kshift).  Only tile 0 is then partial; its
    // first kshift values load as zeros, and every later tile -- including the
    // one the branch-free refill repeats past the end -- is whole and in
    // bounds.  This needs at least two K tiles and no rotation of the first.
    //
    // Edges in M and N: values of A past row m and of B past column n only
    // reach rows and columns of D past the edge, which the epilogue does not
    // store.  So a chunk wholly past the edge loads a chunk of the tile's first
    // row (A) or column (B) instead, always in bounds, and a chunk straddling
    // the edge loads as it is: its dwords past the operand's last element are
    // outside the buffer descriptor's range and read as 0 (the range check is
    // per dword), the others are in memory.
    const bool edge = row0 + MT0 > m || col0 + MT1 > n;
    const uint32_t kshift = (k % DK) ? DK - k % DK : 0u;
    // the fast path's head tile needs a second K tile in the wave's range: the
    // clamped prefetch past the range's end reloads its last tile, which must
    // not be the head (with the in-group K split: per group)
    const int kt_half = (ktiles + 1) / 2;
    const bool slow = kshift != 0u && (SG_MAPK > 1 || (SG_KSPLIT ? kt_half : ktiles) < 2);
    // The K tiles this wave's K loop runs: all ktiles from tile 0, or with the
    // in-group K split h = ceil(ktiles / 2) each -- group 0 tiles [0, h),
    // group 1 tiles [ktiles - h, ktiles), so both run the same number of
    // iterations (and barriers).  For an odd count group 1's first tile is
    // group 0's last: group 1 loads it as zeros (a head tile whose shift is
    // the whole tile: its descriptor starts at that tile's first k and every
    // lane reads there and discards the value).  kshift_h is the head tile's
    // shift: values of its first kshift_h k load as zeros.  Without the split
    // kt_count and kshift_h are ktiles and kshift themselves (references), so
    // the K loop's code is exactly that of a kernel without the knob.
    const bool upper = SG_KSPLIT && kgrp == 1;
    const int& kt_count = SG_KSPLIT ? kt_half : ktiles;
    const int kt_base = upper ? ktiles - kt_half : 0;
    const bool zero_head = upper && (ktiles & 1) != 0;
    const uint32_t kshift_up = zero_head ? (uint32_t)DK : 0u;
    const uint32_t& kshift_h = upper ? kshift_up : kshift;

    // ---- global -> VGPR staging (byte offsets inside a K tile) ----
    // Every thread moves float4 chunks.  A chunk runs along the operand's
    // contiguous dimension: m for A (NN) or k for A^T, k for B (NN) or n for
    // B^T.  Chunks along the LDS row direction are written with one
    // ds_write_b128; chunks across it (the transposed operands) are scattered
    // with four ds_write_b32, so the LDS layouts and reads never change:
    //   A: [DK][MT0 + PAD_A] (m contiguous), B: [MT1][DK + PAD_B] (k contiguous).
    // per chunk: (i0, i1) = position along (contiguous dim / 4, other dim)
    constexpr int A_C0 = TA ? DK / 4 : MT0 / 4;   // chunks along the contiguous dim of A
    constexpr int B_C0 = TB ? MT1 / 4 : DK / 4;   // chunks along the contiguous dim of B
    // element (row, kk) of op(A) is a[row + kk*lda] (NN) or a[kk + row*lda] (T)
    const float* a_tile = TA ? a + (size_t)row0 * lda : a + row0;
    const float* b_tile = TB ? b + col0 : b + (size_t)col0 * ldb;
    // Chunk ch of a K tile -> (c0, c1), its float4 position along the
    // operand's contiguous dimension and across it; every chunk lies along an
    // LDS row, contiguous dimension first (A^T at depth 16 with its rows
    // reordered, below).
    auto a_chunk = [&](int ch, int& c0, int& c1) __attribute__((always_inline)) {
        if constexpr (TA && A_C0 == 4 && SG_ARSW_MASK == 0) {
            // an 8-lane write cycle covers two A^T rows: take them four rows
            // apart (row order 0, 4, 1, 5, 2, 6, 3, 7 in each group of eight),
            // whose banks a 4- or 12-float pad keeps apart (a row swizzle
            // keeps consecutive rows apart instead)
            const int j = ch >> 2;
            c0 = ch & 3;
            c1 = (j & ~7) | ((j & 1) << 2) | ((j >> 1) & 3);
        } else {
            c0 = ch % A_C0;
            c1 = ch / A_C0;
        }
    };
    auto b_chunk = [&](int ch, int& c0, int& c1) __attribute__((always_inline)) {
        c0 = ch % B_C0;
        c1 = ch / B_C0;
    };
    uint32_t a_off[G::LA], b_off[G::LB];  // bytes from the K tile's first element
    int a_lds[G::LA], b_lds[G::LB];
#pragma unroll
    for (int i = 0; i < G::LA; ++i) {
        const int ch = ltid + i * LT;
        int c0, c1;
        a_chunk(ch, c0, c1);
        // a chunk of rows wholly past m reads the tile's first row instead
        if constexpr (!TA) {  // c0: m / 4, c1: k
            const uint32_t r = row0 + (uint32_t)(c0 * 4) < m ? (uint32_t)(c0 * 4) : 0u;
            a_off[i] = (r + (uint32_t)c1 * lda) * 4u;
            a_lds[i] = c1 * G::A_LD + c0 * 4;
        } else {              // c0: k / 4, c1: m
            const uint32_t r = row0 + (uint32_t)c1 < m ? (uint32_t)c1 : 0u;
            a_off[i] = ((uint32_t)(c0 * 4) + r * lda) * 4u;
            a_lds[i] = sg::arow(c1) * G::A_LD + (c0 ^ sg::aswz(c1)) * 4;
        }
    }
#pragma unroll
    for (int i = 0; i < G::LB; ++i) {
        const int ch = ltid + i * LT;
        int c0, c1;
        b_chunk(ch, c0, c1);
        // a chunk of columns wholly past n reads the tile's first column instead
        if constexpr (!TB) {  // c0: k / 4, c1: n
            const uint32_t cc = col0 + (uint32_t)c1 < n ? (uint32_t)c1 : 0u;
            b_off[i] = ((uint32_t)(c0 * 4) + cc * ldb) * 4u;
            b_lds[i] = G::A_STAGE + c1 * G::B_LD + (c0 ^ sg::bswz(c1)) * 4;
        } else {              // c0: n / 4, c1: k
            const uint32_t cc = col0 + (uint32_t)(c0 * 4) < n ? (uint32_t)(c0 * 4) : 0u;
            b_off[i] = (cc + (uint32_t)c1 * ldb) * 4u;
            b_lds[i] = G::A_STAGE + c1 * G::B_LD + c0 * 4;
        }
    }
    // Bytes one K tile of each operand spans from its first element: DK
    // columns of A (or MT0 rows of A^T) and MT1 columns of B (or DK rows of
    // B^T).  The host keeps them below 2^31, so the byte offsets above fit
    // 32 bits; they are the buffer descriptors' num_records.
    const uint32_t a_bytes = ((TA ? (uint32_t)(MT0 - 1) : (uint32_t)(DK - 1)) * lda + (uint32_t)(TA ? DK : MT0)) * 4u;
    const uint32_t b_bytes = ((TB ? (uint32_t)(DK - 1) : (uint32_t)(MT1 - 1)) * ldb + (uint32_t)(TB ? MT1 : DK)) * 4u;
    // Which loads can reach past an operand's last element: chunks wholly
    // past m or n are redirected, and every K tile but the first lies inside
    // [0, k), so only a chunk straddling m (A) or n (B^T) in the operand's
    // last column (row) reads past it, by at most 3 dwords -- at a column
    // (row) within 3 of the last, inside the last K tile since DK >= 4 and
    // that tile is whole.  So only the last K tile's descriptors are cut at
    // the operand's end; a cut never removes an element inside the operand.
    auto cut = [](const char* lim, const float* base, uint32_t bytes) -> int {
        const int64_t left = lim - reinterpret_cast<const char*>(base);
        return (int)(left < 0 ? 0 : (left < (int64_t)bytes ? left : (int64_t)bytes));
    };
    int a_rec_last = 0, b_rec_last = 0;
    if (ktiles > 0) {
        const int64_t kb = (int64_t)(ktiles - 1) * DK - (int64_t)kshift;
        a_rec_last = cut(a_lim, a_tile + (TA ? kb : kb * (int64_t)lda), a_bytes);
        b_rec_last = cut(b_lim, b_tile + (TB ? kb * (int64_t)ldb : kb), b_bytes);
    }
    // PD register staging sets: with the early-refill schedules a K tile's
    // global loads are issued PD tiles before its LDS writes.
    constexpr int PD = (SG_PLR >= 2) ? SG_PD : 1;
    static_assert(PD == 1 || PD == 2, "prefetch depth must be 1 or 2");
    f32x4 ra[PD][G::LA], rb[PD][G::LB];

    int kt_first = kt_base;
    if constexpr (SG_MAPK > 1) kt_first = (tx & (SG_MAPK - 1)) % (ktiles > 0 ? ktiles : 1);

    // gload_to(tag, t, da, db, head): global -> VGPR copy of K tile t into
    // da (A) and db (B); gload(tag, t, set, head) into register set `set`.  On the fast
    // path every chunk is one buffer_load_dwordx4: a wave-uniform descriptor
    // per operand and K tile (scalar arithmetic only; num_records is the K
    // tile's footprint) and the chunk's 32-bit byte offset -- no 64-bit vector
    // address per load.  A Head tag (tile 0 of a shifted K origin) keeps only
    // the values at k >= kshift and zeros the rest.  With a
    // SlowPath tag every element is
    // loaded from a clamped (always valid) address and replaced by 0 when it
    // lies outside A or B, so the code stays branch-free.
    auto gload_to = [&](auto path, int t, f32x4 (&da)[G::LA], f32x4 (&db)[G::LB], auto head)
        __attribute__((always_inline)) {
        int kt = kt_first + t;
        if (kt >= ktiles) kt -= ktiles;
        if constexpr (!decltype(path)::slow) {
            // descriptors start at the K tile's first k, or for a Head tile at
            // its first k inside the operand (tile k = kshift): no base ever
            // lies before the matrix
            const int64_t kb = (int64_t)kt * DK - (int64_t)kshift + (decltype(head)::on ? (int64_t)kshift : 0);
            const float* pa = a_tile + (TA ? kb : kb * (int64_t)lda);
            const float* pb = b_tile + (TB ? kb * (int64_t)ldb : kb);
            // num_records: the K tile's footprint, cut at the operand's last
            // element in the last K tile (32-bit scalar select, no 64-bit compare)
            const bool last = kt == ktiles - 1;
            const int a_rec = last ? a_rec_last : (int)a_bytes;
            const int b_rec = last ? b_rec_last : (int)b_bytes;
            const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc((void*)pa, (short)0, a_rec, BUFFER_RSRC_WORD3);
            const __amdgpu_buffer_rsrc_t rsb = __builtin_amdgcn_make_buffer_rsrc((void*)pb, (short)0, b_rec, BUFFER_RSRC_WORD3);
            const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
            // A Head chunk keeps the values at k >= kshift (inside the tile) and
            // zeros the rest; a value below kshift loads the one at k = kshift of
            // its row or column instead, so every load stays in bounds.  The
            // descriptor starts kshift k steps (k_bytes each) into the tile:
            // offsets move back by that much.  Chunks along k (A^T, B; k_bytes
            // = 4) straddle kshift unless it is a multiple of 4: then they load
            // element by element.
            auto head_load = [&](const __amdgpu_buffer_rsrc_t& rs, uint32_t off, int kk, bool along_k,
                                 uint32_t k_bytes) __attribute__((always_inline)) -> f32x4 {
                if (!along_k || (kshift_h & 3u) == 0u) {
                    const bool live = kk >= (int)kshift_h;
                    const uint32_t o = off - (live ? kshift_h : (uint32_t)kk) * k_bytes;
                    const f32x4 v = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)o, 0, 0));
                    return live ? v : z;
                }
                f32x4 v;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    // the element's k clamped up to kshift, as a byte step from
                    // the descriptor's first k; written as one max so that no
                    // constant splits off into the instruction's offset field
                    // (the register part alone could be negative)
                    const int ke = max(kk + e, (int)kshift_h);
                    const uint32_t o = off + (uint32_t)(ke - kk - (int)kshift_h) * 4u;
                    const float x = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, (int)o, 0, 0));
                    v[e] = kk + e >= (int)kshift_h ? x : 0.0f;
                }
                return v;
            };
#pragma unroll
            for (int i = 0; i < G::LA; ++i) {
                const int ch = ltid + i * LT;
                if (G::A_CHUNKS % LT == 0 || ch < G::A_CHUNKS) {
                    if constexpr (decltype(head)::on) {
                        // k inside the tile of the chunk's first element: c1 (A), 4 * c0 (A^T)
                        int c0, c1;
                        a_chunk(ch, c0, c1);
                        const int kk = TA ? c0 * 4 : c1;
                        da[i] = head_load(rsa, a_off[i], kk, TA, TA ? 4u : lda * 4u);
                    } else {
                        da[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rsa, (int)a_off[i], 0, 0));
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < G::LB; ++i) {
                const int ch = ltid + i * LT;
                if (G::B_CHUNKS % LT == 0 || ch < G::B_CHUNKS) {
                    if constexpr (decltype(head)::on) {
                        // k inside the tile of the chunk's first element: 4 * c0 (B), c1 (B^T)
                        int c0, c1;
                        b_chunk(ch, c0, c1);
                        const int kk = TB ? c1 : c0 * 4;
                        db[i] = head_load(rsb, b_off[i], kk, !TB, TB ? ldb * 4u : 4u);
                    } else {
                        db[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rsb, (int)b_off[i], 0, 0));
                    }
                }
            }
        } else {
            const uint32_t k0 = (uint32_t)kt * DK;
            // group 1's zero head tile of the in-group K split loads nothing
            const bool zt = zero_head && kt == kt_base;
#pragma unroll
            for (int i = 0; i < G::LA; ++i) {
                const int ch = ltid + i * LT;
                if (G::A_CHUNKS % LT == 0 || ch < G::A_CHUNKS) {
                    int c0, c1;
                    a_chunk(ch, c0, c1);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const uint32_t row = row0 + (TA ? (uint32_t)c1 : (uint32_t)(c0 * 4 + e));
                        const uint32_t kk = k0 + (TA ? (uint32_t)(c0 * 4 + e) : (uint32_t)c1);
                        const uint32_t rc = row < m ? row : m - 1;
                        const uint32_t kc = kk < k ? kk : k - 1;
                        const float x = TA ? a[(size_t)rc * lda + kc] : a[(size_t)kc * lda + rc];
                        da[i][e] = (row < m && kk < k && !zt) ? x : 0.0f;
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < G::LB; ++i) {
                const int ch = ltid + i * LT;
                if (G::B_CHUNKS % LT == 0 || ch < G::B_CHUNKS) {
                    int c0, c1;
                    b_chunk(ch, c0, c1);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const uint32_t col = col0 + (TB ? (uint32_t)(c0 * 4 + e) : (uint32_t)c1);
                        const uint32_t kk = k0 + (TB ? (uint32_t)c1 : (uint32_t)(c0 * 4 + e));
                        const uint32_t cc = col < n ? col : n - 1;
                        const uint32_t kc = kk < k ? kk : k - 1;
                        const float x = TB ? b[(size_t)kc * ldb + cc] : b[(size_t)cc * ldb + kc];
                        db[i][e] = (col < n && kk < k && !zt) ? x : 0.0f;
                    }
                }
            }
        }
    };
    auto gload = [&](auto path, int t, int set, auto head) __attribute__((always_inline)) {
        gload_to(path, t, ra[set], rb[set], head);
    };
    auto swrite_from = [&](int buf, const f32x4 (&da)[G::LA], const f32x4 (&db)[G::LB])
        __attribute__((always_inline)) {
        float* s = lds + buf * G::STAGE;
#pragma unroll
        for (int i = 0; i < G::LA; ++i)
            if (G::A_CHUNKS % LT == 0 || ltid + i * LT < G::A_CHUNKS) {
                *reinterpret_cast<f32x4*>(s + a_lds[i]) = da[i];  // a row of A or of A^T
            }
#pragma unroll
        for (int i = 0; i < G::LB; ++i)
            if (G::B_CHUNKS % LT == 0 || ltid + i * LT < G::B_CHUNKS) {
                *reinterpret_cast<f32x4*>(s + b_lds[i]) = db[i];  // a row of B or of B^T
            }
    };
    auto swrite = [&](int buf, int set) __attribute__((always_inline)) { swrite_from(buf, ra[set], rb[set]); };

    // ---- LDS -> MFMA operand addresses ----
    const int r = lane % AT::M;  // row (A) / column (B) inside the atom
    const int g = lane / AT::M;  // k group
    // A: row k = g * KPL + ..., WT0 consecutive m (the interleaved atoms);
    // A^T: rows m = wm * SM + r * WT0 + i, KPL consecutive k each, stored at
    // rows arow(m): a_ri[i] is atom i's row offset from a_rd
    const int a_row0 = wm * (AT::M * WT0) + r * WT0;
    const int a_rd = TA ? a_row0 * G::A_LD + (SG_ASWZ_MASK ? 0 : g * KPL)
                        : g * KPL * G::A_LD + wm * (AT::M * WT0) + r * WT0;
    const int a_fr = sg::aswz(a_row0);  // the swizzle of every A^T row this lane reads
    int a_ri[WT0];
#pragma unroll
    for (int i = 0; i < WT0; ++i) a_ri[i] = (sg::arow(a_row0 + i) - a_row0) * G::A_LD;
    // B: rows n = wn * SN + jn * AN + r, KPL consecutive k each; B^T: row k =
    // g * KPL + ..., WT1 consecutive n (the interleaved atoms: column r of
    // atom jn is tile column r * WT1 + jn, which the epilogue follows)
    const int b_rd = TB ? G::A_STAGE + g * KPL * G::B_LD + wn * (AT::N * WT1) + r * WT1
                        : G::A_STAGE + (wn * (AT::N * WT1) + r) * G::B_LD + (SG_BSWZ_MASK ? 0 : g * KPL);
    const int b_fr = sg::bswz(r);  // the swizzle of every B row this lane reads

    acc_t acc[WT0][WT1];
#pragma unroll
    for (int i = 0; i < WT0; ++i)
#pragma unroll
        for (int j = 0; j < WT1; ++j)
#pragma unroll
            for (int q = 0; q < AT::ACC; ++q) acc[i][j][q] = 0.0f;

    constexpr int NKB = DK / KB;
    // operand registers for one k block
    struct Frag {
        float a[KPL][WT0];
        float b[WT1][KPL];
    };
    auto load_frag = [&](const float* s, int kb, Frag& f) __attribute__((always_inline)) {
        if constexpr (!TA) {
#pragma unroll
            for (int j = 0; j < KPL; ++j) lds_read_row<WT0>(s + a_rd + (kb * KB + j) * G::A_LD, f.a[j]);
        } else {
#pragma unroll
            for (int i = 0; i < WT0; ++i) {
                const float* p;
                if constexpr (SG_ASWZ_MASK == 0) {
                    p = s + a_rd + a_ri[i] + kb * KB;
                } else {
                    const int kc = g * KPL + kb * KB;  // first k of the read, inside one chunk
                    p = s + a_rd + a_ri[i] + ((((kc >> 2) ^ a_fr) << 2) | (kc & 3));
                }
                float tmp[KPL];
                lds_read_row<KPL>(p, tmp);
#pragma unroll
                for (int j = 0; j < KPL; ++j) f.a[j][i] = tmp[j];
            }
        }
        if constexpr (TB) {
#pragma unroll
            for (int j = 0; j < KPL; ++j) {
                float tmp[WT1];
                lds_read_row<WT1>(s + b_rd + (kb * KB + j) * G::B_LD, tmp);
#pragma unroll
                for (int jn = 0; jn < WT1; ++jn) f.b[jn][j] = tmp[jn];
            }
        } else {
#pragma unroll
            for (int jn = 0; jn < WT1; ++jn) {
                const float* p;
                if constexpr (SG_BSWZ_MASK == 0) {
                    p = s + b_rd + jn * AT::N * G::B_LD + kb * KB;
                } else {
                    const int kc = g * KPL + kb * KB;  // first k of the read, inside one chunk
                    p = s + b_rd + jn * AT::N * G::B_LD + ((((kc >> 2) ^ b_fr) << 2) | (kc & 3));
                }
                float tmp[KPL];
                lds_read_row<KPL>(p, tmp);
#pragma unroll
                for (int j = 0; j < KPL; ++j) f.b[jn][j] = tmp[j];
            }
        }
    };
    auto mfma_frag = [&](const Frag& f) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < KPL; ++j)
#pragma unroll
            for (int i = 0; i < WT0; ++i)
#pragma unroll
                for (int jn = 0; jn < WT1; ++jn) acc[i][jn] = AT::mfma(f.a[j][i], f.b[jn][j], acc[i][jn]);
    };
    // the k steps [j0, j1) of mfma_frag
    auto mfma_frag_part = [&](const Frag& f, int j0, int j1) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < KPL; ++j)
            if (j >= j0 && j < j1) {
#pragma unroll
                for (int i = 0; i < WT0; ++i)
#pragma unroll
                    for (int jn = 0; jn < WT1; ++jn) acc[i][jn] = AT::mfma(f.a[j][i], f.b[jn][j], acc[i][jn]);
            }
    };
    auto compute = [&](int buf) __attribute__((always_inline)) {
        const float* s = lds + buf * G::STAGE;
        if constexpr (SG_PLR > 0 && NKB > 1) {
            // software pipeline: operands of block kb+1 are read while block kb multiplies
            Frag f[2];
            load_frag(s, 0, f[0]);
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) {
                if (kb + 1 < NKB) load_frag(s, kb + 1, f[(kb + 1) & 1]);
                mfma_frag(f[kb & 1]);
            }
        } else {
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) {
                Frag f;
                load_frag(s, kb, f);
                mfma_frag(f);
            }
        }
    };

    // ---- K loop: NBUF LDS buffers, one barrier per tile ----
    // One instantiation of the K loop per load path; the choice is uniform
    // per work-group, so neither loop carries a branch on it.
    auto kloop = [&](auto path) __attribute__((always_inline)) {
        // Tile t lives in buffer t % NBUF.  Buffer (t + NBUF - 1) % NBUF was last
        // read in iteration t - 1, so after the barrier that ends iteration t - 1
        // any point of iteration t may refill it.
    #pragma unroll
        for (int s = 0; s < NBUF - 1; ++s) {
            if (s < kt_count) {
                if (s == 0 && kshift_h != 0u) gload(path, 0, 0, Head{});
                else gload(path, s, 0, NoHead{});
                swrite(s, 0);
            }
        }
        // tiles NBUF - 1 .. NBUF + PD - 2 go to the register sets
    #pragma unroll
        for (int j = 0; j < PD; ++j)
            if (NBUF - 1 + j < kt_count) gload(path, NBUF - 1 + j, (NBUF - 1 + j) % PD, NoHead{});
        __syncthreads();

        if constexpr (SG_PLR >= 2) {
            // Early refill: the next tile's LDS writes and the global loads after it
            // are issued right after the first k block's MFMAs, so they overlap MFMA
            // execution instead of sitting between the last MFMA and the barrier.
            // With NBUF >= 3 the first operands of tile t + 1 (written in iteration
            // t - 1) are read before the barrier too, so nothing but the barrier
            // separates the last MFMA of one tile from the first of the next.
            // Iteration t writes tile t + NBUF - 1 from register set
            // (t + NBUF - 1) % PD and refills that set with tile t + NBUF - 1 + PD,
            // so a tile's global loads have PD iterations to arrive.
            constexpr int U = (PD == 2 && NBUF % 2) ? 2 * NBUF : NBUF;  // lcm(NBUF, PD)
            Frag cur, nxt;
            if (kt_count > 0) load_frag(lds, 0, cur);
            for (int t0 = 0; t0 < kt_count; t0 += U) {
    #pragma unroll
                for (int uu = 0; uu < U; ++uu) {
                    const int t = t0 + uu;
                    const int u = uu % NBUF;
                    const int set = (uu + NBUF - 1) % PD;
                    if (t < kt_count) {
                        const float* s = lds + u * G::STAGE;
    #pragma unroll
                        for (int kb = 0; kb < NKB; ++kb) {
                            const bool last = kb + 1 == NKB;
                            // Branch-free refill: past the last tile the loads repeat the
                            // last tile and the writes land in the buffer of tile t - 1,
                            // which no later iteration reads; the prefetch past the end
                            // reads a valid buffer whose values go unused.
                            if (!last) load_frag(s, kb + 1, nxt);
                            else if (NBUF >= 3) load_frag(lds + ((u + 1) % NBUF) * G::STAGE, 0, nxt);
                            mfma_frag(cur);
                            if (kb == 0) {
                                swrite((u + NBUF - 1) % NBUF, set);
                                gload(path, min(t + NBUF - 1 + PD, kt_count - 1), set, NoHead{});
                            }
                            if constexpr (SG_PLR >= 3) {
                                constexpr int NMFMA = KPL * WT0 * WT1;
                                // LDS read instructions of one block: float4 reads of
                                // rows; rows of one or two floats pair up into one
                                // ds_read2 (KPL rows of A or of B^T, A_LD or B_LD apart)
                                constexpr int NREAD_A = TA ? WT0 * (KPL >= 4 ? KPL / 4 : 1)
                                                           : (WT0 >= 4 ? KPL * (WT0 / 4) : (KPL + 1) / 2);
                                constexpr int NREAD_B = TB ? (WT1 >= 4 ? KPL * (WT1 / 4) : (KPL + 1) / 2)
                                                           : WT1 * (KPL >= 4 ? KPL / 4 : 1);
                                constexpr int NREAD = NREAD_A + NREAD_B;
                                constexpr int NREAD_NEXT = (NKB > 1 || NBUF >= 3) ? NREAD : 0;
                                if (kb == 0) interleave_block<NMFMA, NREAD_NEXT, G::LA + G::LB, G::LA + G::LB>();
                                else if (!last || NBUF >= 3) interleave_block<NMFMA, NREAD, 0, 0>();
                                else interleave_block<NMFMA, 0, 0, 0>();
                            }
                            if (!last || NBUF >= 3) cur = nxt;
                        }
                        __syncthreads();
                        if (NBUF == 2 && t + 1 < kt_count) load_frag(lds + ((u + 1) % NBUF) * G::STAGE, 0, cur);
                    }
                }
            }
        } else {
            for (int t0 = 0; t0 < kt_count; t0 += NBUF) {
    #pragma unroll
                for (int u = 0; u < NBUF; ++u) {
                    const int t = t0 + u;
                    if (t < kt_count) {
                        compute(u);
                        if (t + NBUF - 1 < kt_count) swrite((u + NBUF - 1) % NBUF, 0);
                        if (t + NBUF < kt_count) gload(path, t + NBUF, 0, NoHead{});
                        __syncthreads();
                    }
                }
            }
        }
    };
#if SG_WS
    // ---- wave-specialised K loop ----
    // The loading waves copy K tiles into the NBUF LDS buffers; the computing
    // waves only read LDS and multiply.  No work-group barrier inside the
    // loop: two LDS counters per buffer order the roles.  ready[b] counts the
    // loading waves that have written buffer b's current tile (NLW per tile),
    // done[b] the computing waves that have finished reading it (CWAVES per
    // tile).  Tile t -- round r = t / NBUF of buffer b = t % NBUF -- may be
    // read once ready[b] >= NLW * (r + 1), and buffer b may take tile t +
    // NBUF once done[b] >= CWAVES * (r + 1).  LDS serves one wave's accesses
    // in issue order, so a count raised after a wave's writes (or reads) is
    // seen by another wave only after them; compiler barriers keep that
    // order in the code.  A wait gives up after a bounded number of polls:
    // a broken count would end the loop with wrong values, never hang.
    {
        constexpr int NLW = G::NT / 64 - G::CWAVES;
        static_assert(NLW > 0, "wave specialisation needs loading waves");
        __shared__ uint32_t ws_count[2 * NBUF];
        uint32_t* const ready = ws_count;
        uint32_t* const done = ws_count + NBUF;
        if (tid < 2 * NBUF) ws_count[tid] = 0u;
        __syncthreads();
        auto wait_at_least = [&](uint32_t* cnt, uint32_t target) __attribute__((always_inline)) {
            for (uint32_t poll = 0; poll < (1u << 22); ++poll) {
                const uint32_t v = __builtin_amdgcn_readfirstlane(
                    __hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
                if (v >= target) break;
                __builtin_amdgcn_s_sleep(1);
            }
            asm volatile("" ::: "memory");
        };
        // One LDS add per wave, by lane 0 alone, without a branch: EXEC is
        // narrowed to lane 0 around the ds_add_u32 (the low 32 bits of a
        // pointer into LDS are its LDS address).  The asm is also a compiler
        // barrier: the wave's LDS accesses before it stay before it.
        auto raise = [&](uint32_t* cnt) __attribute__((always_inline)) {
            const uint32_t addr = (uint32_t)reinterpret_cast<uintptr_t>(cnt);
            uint64_t saved;
            asm volatile(
                "s_mov_b64 %0, exec\n\t"
                "s_mov_b64 exec, 1\n\t"
                "s_nop 1\n\t"
                "ds_add_u32 %1, %2\n\t"
                "s_mov_b64 exec, %0"
                : "=&s"(saved)
                : "v"(addr), "v"(1u)
                : "memory");
        };
        if (loader_wave) {
            // P register sets: the loads of tiles t + 1 .. t + P - 1 are in
            // flight while tile t waits for its buffer and is written
            constexpr int P = SG_WS_PD;
            static_assert(P >= 2 && P <= 4, "2 to 4 register sets per loading wave");
            f32x4 wa[P][G::LA], wb[P][G::LB];
            auto produce = [&](auto path) __attribute__((always_inline)) {
                // lcm(NBUF, P): buffer and register set are compile-time per step
                constexpr int U = (NBUF % P == 0) ? NBUF : ((P % NBUF == 0) ? P : NBUF * P);
                if (ktiles > 0) {
                    if (kshift != 0u) gload_to(path, 0, wa[0], wb[0], Head{});
                    else gload_to(path, 0, wa[0], wb[0], NoHead{});
                }
#pragma unroll
                for (int j = 1; j < P; ++j)
                    if (j < ktiles) gload_to(path, j, wa[j], wb[j], NoHead{});
                for (int t0 = 0; t0 < ktiles; t0 += U) {
#pragma unroll
                    for (int uu = 0; uu < U; ++uu) {
                        const int t = t0 + uu;
                        if (t < ktiles) {
                            const int u = uu % NBUF, set = uu % P;
                            if (t >= NBUF) wait_at_least(&done[u], (uint32_t)(G::CWAVES * (t / NBUF)));
                            swrite_from(u, wa[set], wb[set]);
                            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                            raise(&ready[u]);
                            if (t + P < ktiles) gload_to(path, t + P, wa[set], wb[set], NoHead{});
                        }
                    }
                }
            };
            if (slow) produce(SlowPath{});
            else produce(FastPath{});
            __syncthreads();  // pairs with the computing waves' barrier below
            return;
        }
        constexpr int NMFMA = KPL * WT0 * WT1;
        constexpr int NREAD_A = TA ? WT0 * (KPL >= 4 ? KPL / 4 : 1) : (WT0 >= 4 ? KPL * (WT0 / 4) : (KPL + 1) / 2);
        constexpr int NREAD_B = TB ? (WT1 >= 4 ? KPL * (WT1 / 4) : (KPL + 1) / 2) : WT1 * (KPL >= 4 ? KPL / 4 : 1);
        constexpr int NREAD = NREAD_A + NREAD_B;
        Frag cur, nxt;
        if (ktiles > 0) {
            wait_at_least(&ready[0], (uint32_t)NLW);
            load_frag(lds, 0, cur);
        }
        for (int t0 = 0; t0 < ktiles; t0 += NBUF) {
#pragma unroll
            for (int u = 0; u < NBUF; ++u) {
                const int t = t0 + u;
                if (t < ktiles) {
                    const float* sb = lds + u * G::STAGE;
                    const int un = (u + 1) % NBUF;
                    const uint32_t need = (uint32_t)(NLW * ((t + 1) / NBUF + 1));
                    // the next buffer's count, read a tile ahead of its use
                    const uint32_t seen = __hip_atomic_load(&ready[un], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
#pragma unroll
                    for (int kb = 0; kb < NKB; ++kb) {
                        if (kb + 1 < NKB) {
                            load_frag(sb, kb + 1, nxt);
                        } else {
                            // the next tile's first operands; branch-free past
                            // the last tile (a valid buffer whose values go
                            // unused), only the rare wait is conditional
                            if (__builtin_expect(t + 1 < ktiles && __builtin_amdgcn_readfirstlane(seen) < need, 0))
                                wait_at_least(&ready[un], need);
                            asm volatile("" ::: "memory");
                            load_frag(lds + un * G::STAGE, 0, nxt);
                        }
                        if (kb + 1 < NKB) {
                            mfma_frag(cur);
                        } else {
                            // the last block's operands are in registers: buffer u is
                            // free once half its MFMAs are issued (the signal then
                            // sits between MFMAs, not at the tile boundary)
                            mfma_frag_part(cur, 0, KPL / 2);
                            raise(&done[u]);
                            mfma_frag_part(cur, KPL / 2, KPL);
                        }
                        // the first block also carries the early read of the next count
                        if constexpr (SG_PLR >= 3) {
                            if (kb == 0) interleave_block<NMFMA, NREAD + 1, 0, 0>();
                            else interleave_block<NMFMA, NREAD, 0, 0>();
                        }
                        cur = nxt;
                    }
                }
            }
        }
        __syncthreads();  // every computing wave is past the K buffers: the epilogue reuses them
    }
#else
    if (slow) kloop(SlowPath{});
    else kloop(FastPath{});
#endif
    // The epilogue stages the tile through LDS when its chunks fit (SG_GW).
    constexpr bool STAGED = SG_GW != 0 && G::CWAVES * AT::N * AT::M * WT0 <= G::LDS_FLOATS;
    if constexpr (SG_KSPLIT != 0) {
        // ---- the two K halves meet in LDS: group 0 += group 1 ----
        // Wave w of group 1 holds the same sub-tile as wave w of group 0; its
        // accumulators go to group 1's ring (the ring after group 0's) as
        // float4 chunk ch of work-item ctid at float4 (ch * CNT + ctid), read
        // back by the same work-item of group 0 and added after group 0's own
        // (a fixed order: the result does not depend on timing).  Group 1
        // then leaves, after the barrier that opens the staged epilogue.
        constexpr int HC = AT::ACC / 4;
        constexpr int CH = WT0 * WT1 * HC;
        static_assert(!SG_KSPLIT || CH * G::CNT * 4 <= G::LDS_FLOATS, "group 1's sums fit its LDS ring");
        float* const part = kgrp == 1 ? lds : lds + G::LDS_FLOATS;
        const int ctid = tid % G::CNT;
        __syncthreads();  // both groups are past their last K-tile read
        if (kgrp == 1) {
#pragma unroll
            for (int i = 0; i < WT0; ++i)
#pragma unroll
                for (int j = 0; j < WT1; ++j)
#pragma unroll
                    for (int h = 0; h < HC; ++h) {
                        f32x4 v;
                        v.x = acc[i][j][4 * h]; v.y = acc[i][j][4 * h + 1];
                        v.z = acc[i][j][4 * h + 2]; v.w = acc[i][j][4 * h + 3];
                        *reinterpret_cast<f32x4*>(part + (((i * WT1 + j) * HC + h) * G::CNT + ctid) * 4) = v;
                    }
        }
        __syncthreads();
        if (kgrp == 1) {
            if constexpr (STAGED) __syncthreads();  // pairs with the staged epilogue's barrier
            return;
        }
#pragma unroll
        for (int i = 0; i < WT0; ++i)
#pragma unroll
            for (int j = 0; j < WT1; ++j)
#pragma unroll
                for (int h = 0; h < HC; ++h) {
                    const f32x4 v = *reinterpret_cast<const f32x4*>(part + (((i * WT1 + j) * HC + h) * G::CNT + ctid) * 4);
                    acc[i][j][4 * h] += v.x; acc[i][j][4 * h + 1] += v.y;
                    acc[i][j][4 * h + 2] += v.z; acc[i][j][4 * h + 3] += v.w;
                }
    }

    if (fx.kind != FIX_NONE) {
        // ---- publish the partial; the last arrival combines ----
        // Partial s: float4 chunk ch of thread tid (slots 4h..4h+3 of atom
        // (i, j), ch = (i * WT1 + j) * ACC / 4 + h) is float4 number
        // (s * CH + ch) * NT + tid from fx.ws.
        //
        // Partials are written and read with device-scope (sc1) buffer
        // accesses, coherent across the XCDs' L2 caches by themselves, and the
        // ticket is an agent-scope relaxed atomic: no device-scope fence, which
        // would write back and invalidate a whole L2 per use.  Ordering: each
        // wave waits for its partial stores to be acknowledged (vmcnt(0))
        // before the barrier after which one thread takes the ticket, and the
        // last arrival issues its partial loads only after its ticket returned.
        constexpr int HC = AT::ACC / 4;
        constexpr int CH = WT0 * WT1 * HC;
        constexpr uint32_t PART_BYTES = (uint32_t)CH * NT * 16;
        const __amdgpu_buffer_rsrc_t rs =
            __builtin_amdgcn_make_buffer_rsrc(fx.ws, (short)0, (int)(fx.parts * PART_BYTES), BUFFER_RSRC_WORD3);
#pragma unroll
        for (int i = 0; i < WT0; ++i)
#pragma unroll
            for (int j = 0; j < WT1; ++j)
#pragma unroll
                for (int h = 0; h < HC; ++h) {
                    const int ch = (i * WT1 + j) * HC + h;
                    f32x4 v;
                    v.x = acc[i][j][4 * h]; v.y = acc[i][j][4 * h + 1];
                    v.z = acc[i][j][4 * h + 2]; v.w = acc[i][j][4 * h + 3];
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rs, tid * 16,
                                                           (int)(fx.slot * PART_BYTES) + ch * NT * 16, CPOL_SC1);
                }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __shared__ uint32_t arrived;
        __syncthreads();
        if (tid == 0) arrived = __hip_atomic_fetch_add(fx.ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        if (arrived + 1 != fx.parts) return;
        auto read_part = [&](uint32_t sp, int ch) __attribute__((always_inline)) {
            return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                 rs, tid * 16, (int)(sp * PART_BYTES) + ch * NT * 16, CPOL_SC1));
        };
        if (fx.kind == FIX_SPLIT) {
            // Sum partials 0, 1, ..., parts - 1 in that order (the own one is
            // re-read too), so the result does not depend on the arrival order.
#pragma unroll
            for (int i = 0; i < WT0; ++i)
#pragma unroll
                for (int j = 0; j < WT1; ++j)
#pragma unroll
                    for (int h = 0; h < HC; ++h) {
                        const f32x4 v = read_part(0, (i * WT1 + j) * HC + h);
                        acc[i][j][4 * h] = v.x; acc[i][j][4 * h + 1] = v.y;
                        acc[i][j][4 * h + 2] = v.z; acc[i][j][4 * h + 3] = v.w;
                    }
            for (uint32_t sp = 1; sp < fx.parts; ++sp) {
#pragma unroll
                for (int i = 0; i < WT0; ++i)
#pragma unroll
                    for (int j = 0; j < WT1; ++j)
#pragma unroll
                        for (int h = 0; h < HC; ++h) {
                            const f32x4 v = read_part(sp, (i * WT1 + j) * HC + h);
                            acc[i][j][4 * h] += v.x; acc[i][j][4 * h + 1] += v.y;
                            acc[i][j][4 * h + 2] += v.z; acc[i][j][4 * h + 3] += v.w;
                        }
            }
        } else {
            // two partials: own + other, commutative.  Read in batches of one
            // atom's chunks so the loads never hold more than ACC extra
            // registers (all of them at once would spill the largest tiles).
#pragma unroll
            for (int i = 0; i < WT0; ++i)
#pragma unroll
                for (int j = 0; j < WT1; ++j) {
#pragma unroll
                    for (int h = 0; h < HC; ++h) {
                        const f32x4 v = read_part(1u - fx.slot, (i * WT1 + j) * HC + h);
                        acc[i][j][4 * h] += v.x; acc[i][j][4 * h + 1] += v.y;
                        acc[i][j][4 * h + 2] += v.z; acc[i][j][4 * h + 3] += v.w;
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
        }
        // every arrival of this launch has been counted: re-arm for the next one
        if (tid == 0) __hip_atomic_store(fx.ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    // ---- epilogue: D = alpha * acc + beta * C ----
    const int wrow = row0 + wm * (AT::M * WT0);
    const int wcol = col0 + wn * (AT::N * WT1);
    // column (inside the wave's sub-tile) of column c of atom group jn: the
    // groups side by side, or for B^T interleaved (the order of its reads)
    auto sub_col = [](int jn, int c) __attribute__((always_inline)) {
        return TB ? c * WT1 + jn : jn * AT::N + c;
    };
    // Whole tiles go through LDS: the accumulators of one MFMA column group
    // (atom_n columns of the wave's SM-row sub-tile) are scattered into a
    // column-major LDS chunk, then read back as float4 runs down each column,
    // so one store instruction writes whole columns (SM * 4 bytes each, full
    // 128-byte lines) instead of 16 bytes in each of atom_n columns.  Columns
    // are unpadded and float4 run r of column c sits at run r ^ (c mod
    // E_RUNS): the scatter's 16-byte writes (8 lanes a cycle, 8 columns at
    // one row) and the read-back's 16-byte reads (a half-wave's quads
    // {0,3,5,6} and {1,2,4,7} a cycle, down one to eight columns) then reach
    // distinct banks.  A 4-float pad instead serves the writes but not the
    // reads when a half-wave spans two or more columns (SM <= 64).
    constexpr int SM = AT::M * WT0;           // rows of a wave's sub-tile
    constexpr int E_LD = SM;                  // LDS column stride
    constexpr int E_CHUNK = AT::N * E_LD;     // floats of LDS per wave
    constexpr int E_RUNS = SM / 4;            // float4 runs per column
    constexpr int E_PER_LANE = AT::N * E_RUNS / 64;
    static_assert(AT::N * E_RUNS % 64 == 0, "a column group is a whole number of float4s per lane");
    static_assert((E_RUNS & (E_RUNS - 1)) == 0, "the run swizzle stays inside a column");
    // SG_GW (the reference's global-write flavour, generator.py:2290-2508):
    // 1 stages through LDS as above when the chunks fit, 0 always stores
    // straight from the accumulators (no LDS, fewer live registers)
    static_assert(STAGED == (SG_GW != 0 && G::CWAVES * E_CHUNK <= G::LDS_FLOATS), "one staging rule");
    if constexpr (STAGED) {
        {
            // every wave's last K-loop access to LDS is behind this barrier
            // (the wave-specialised loop ends with that barrier itself)
            if constexpr (!SG_WS) __syncthreads();
            float* e = lds + wave * E_CHUNK;
            // Buffer descriptors over the wave's sub-tile of D and of C (SN
            // columns of SM rows from (wrow, wcol)), cut at the matrix's last
            // element; dword alignment is enough, so any ldc / ldd works.
            constexpr int SN = AT::N * WT1;
            auto sub_rsrc = [&](const float* base, uint32_t ld) __attribute__((always_inline)) {
                const uintptr_t first = reinterpret_cast<uintptr_t>(base) + ((uint64_t)wcol * ld + (uint32_t)wrow) * 4u;
                const uintptr_t last = reinterpret_cast<uintptr_t>(base) + ((uint64_t)(n - 1) * ld + m) * 4u;
                const uint64_t foot = ((uint64_t)(SN - 1) * ld + SM) * 4u;
                const uint64_t left = last > first ? (uint64_t)(last - first) : 0u;
                return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(first), (short)0,
                                                         (int)(left < foot ? left : foot), BUFFER_RSRC_WORD3);
            };
            const __amdgpu_buffer_rsrc_t rsd = sub_rsrc(d, ldd);
            const __amdgpu_buffer_rsrc_t rsc = sub_rsrc(beta != 0.0f ? c : d, beta != 0.0f ? ldc : ldd);
#pragma unroll
            for (int jn = 0; jn < WT1; ++jn) {
                // A lane's slots q..q+3 (q a multiple of 4) hold four
                // consecutive rows of its column in both atoms, so below four
                // rows per slot (WT0 < 4) QG slots share one 16-byte write:
                // every write is whole float4 runs (8- and 4-byte writes
                // would serve 16 and 32 lanes a cycle, more than the 8
                // distinct runs a row of 8 columns offers).
                constexpr int QG = WT0 >= 4 ? 1 : 4 / WT0;
                static_assert(4 % QG == 0 && AT::ACC % QG == 0, "slot groups stay inside a run of four rows");
                static_assert((WT0 * QG) % 4 == 0, "whole float4 runs per write");
                const int ecol = lane % AT::N;
                const int eswz = ecol & (E_RUNS - 1);
#pragma unroll
                for (int q = 0; q < AT::ACC; q += QG) {
                    float v[WT0 * QG];
#pragma unroll
                    for (int g = 0; g < QG; ++g)
#pragma unroll
                        for (int i = 0; i < WT0; ++i) v[g * WT0 + i] = alpha * acc[i][jn][q + g];
                    const int run0 = AT::row(q, lane) * WT0 / 4;
#pragma unroll
                    for (int h = 0; h < WT0 * QG / 4; ++h) {
                        f32x4 t;
                        t.x = v[4 * h]; t.y = v[4 * h + 1]; t.z = v[4 * h + 2]; t.w = v[4 * h + 3];
                        *reinterpret_cast<f32x4*>(e + ecol * E_LD + ((run0 + h) ^ eswz) * 4) = t;
                    }
                }
                // the wave's scattered writes are complete before any lane reads them back
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                // Lane run p: column cc, rows r4..r4+3 of the group, in batches
                // of EB runs: the batch's LDS reads, then its C loads (a run
                // reaching past C's last element reads 0 there, the others
                // stay inside C's allocation), then its stores.
                constexpr int EB = E_PER_LANE < 4 ? E_PER_LANE : 4;
                static_assert(E_PER_LANE % EB == 0, "whole batches of runs");
                auto run_off = [&](int p, uint32_t ld) __attribute__((always_inline)) {
                    const int idx = p * 64 + lane;
                    return ((uint32_t)sub_col(jn, idx / E_RUNS) * ld + (uint32_t)((idx % E_RUNS) * 4)) * 4u;
                };
#pragma unroll
                for (int p0 = 0; p0 < E_PER_LANE; p0 += EB) {
                    f32x4 v[EB];
#pragma unroll
                    for (int b = 0; b < EB; ++b) {
                        const int idx = (p0 + b) * 64 + lane;
                        const int ec = idx / E_RUNS;
                        v[b] = *reinterpret_cast<const f32x4*>(e + ec * E_LD + ((idx % E_RUNS) ^ (ec & (E_RUNS - 1))) * 4);
                    }
                    if (beta != 0.0f) {
                        f32x4 cv[EB];
#pragma unroll
                        for (int b = 0; b < EB; ++b)
                            cv[b] = __builtin_bit_cast(
                                f32x4, __builtin_amdgcn_raw_buffer_load_b128(rsc, (int)run_off(p0 + b, ldc), 0, 0));
#pragma unroll
                        for (int b = 0; b < EB; ++b) {
                            v[b].x = __builtin_fmaf(beta, cv[b].x, v[b].x); v[b].y = __builtin_fmaf(beta, cv[b].y, v[b].y);
                            v[b].z = __builtin_fmaf(beta, cv[b].z, v[b].z); v[b].w = __builtin_fmaf(beta, cv[b].w, v[b].w);
                        }
                    }
                    // streaming (nt) stores: D is not read again by this launch
                    if (!edge) {
#pragma unroll
                        for (int b = 0; b < EB; ++b)
                            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v[b]), rsd,
                                                                   (int)run_off(p0 + b, ldd), 0, CPOL_NT);
                    } else {
                        // only elements inside D are stored: a run reaching past m
                        // (possible when m % 4 != 0) is stored element by element
#pragma unroll
                        for (int b = 0; b < EB; ++b) {
                            const int idx = (p0 + b) * 64 + lane;
                            const uint32_t row = (uint32_t)wrow + (uint32_t)((idx % E_RUNS) * 4);
                            const uint32_t col = (uint32_t)wcol + (uint32_t)sub_col(jn, idx / E_RUNS);
                            const uint32_t off = run_off(p0 + b, ldd);
                            if (col < n && row < m) {
                                if (row + 4u <= m) {
                                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v[b]), rsd, (int)off,
                                                                           0, CPOL_NT);
                                } else {
#pragma unroll
                                    for (int q = 0; q < 3; ++q) {
                                        // the element is copied out first: hipcc's
                                        // bit_cast of a vector element with a loop
                                        // index read element 0 for every q
                                        const float x = v[b][q];
                                        if (row + (uint32_t)q < m)
                                            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, x), rsd,
                                                                                  (int)(off + 4u * q), 0, CPOL_NT);
                                    }
                                }
                            }
                        }
                    }
                }
                // this group's reads are done before the next group overwrites the chunk
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            }
            return;
        }
    }
    // Direct stores (when the LDS chunk does not fit): vector stores for an
    // interior tile with 16-byte aligned columns of C and D, else element by
    // element with bounds checks.
    const bool d_vec = !edge && ((ldc | ldd) & 3u) == 0 &&
                       ((reinterpret_cast<uintptr_t>(c) | reinterpret_cast<uintptr_t>(d)) & 15u) == 0;
#pragma unroll
    for (int jn = 0; jn < WT1; ++jn) {
        const size_t colo = (size_t)(wcol + sub_col(jn, lane % AT::N));
#pragma unroll
        for (int q = 0; q < AT::ACC; ++q) {
            const int rr = wrow + AT::row(q, lane) * WT0;
            float v[WT0];
#pragma unroll
            for (int i = 0; i < WT0; ++i) v[i] = alpha * acc[i][jn][q];
            if (d_vec) {
                if (beta != 0.0f) {
                    float cv[WT0];
                    global_load_row<WT0>(c + colo * ldc + rr, cv);
#pragma unroll
                    for (int i = 0; i < WT0; ++i) v[i] = __builtin_fmaf(beta, cv[i], v[i]);
                }
                store_row<WT0>(d + colo * ldd + rr, v);
            } else if (colo < n) {
#pragma unroll
                for (int i = 0; i < WT0; ++i) {
                    const uint32_t row = (uint32_t)rr + i;
                    if (row < m) {
                        float x = v[i];
                        if (beta != 0.0f) x = __builtin_fmaf(beta, c[colo * ldc + row], x);
                        d[colo * ldd + row] = x;
                    }
                }
            }
        }
    }
}

// Tile of work-group (bx, by) of a 2-D tile grid: the XCD renumbering and
// the grouping act on the 2-D grid.  (Both orderings of a split launch's whole
// (tile, range) grid tried -- range by range, and tile by tile -- measured
// slower on MI355X than this per-slice order.)
__device__ __forceinline__ void grid_tile(int bx, int by, int nwgx, int nwgy, int& tx, int& ty) {
    sg::tile_coords(sg::xcd_order(bx + nwgx * by, nwgx * nwgy), nwgx, nwgy, tx, ty);
}

extern "C" __global__ void __launch_bounds__(sg::G::NT) SG_OCC_ATTR
SG_KERNEL_NAME(const float* __restrict__ a, const float* __restrict__ b,
               const float* c, float* d,
               uint32_t m, uint32_t n, uint32_t k,
               uint32_t lda, uint32_t ldb, uint32_t ldc, uint32_t ldd,
               float alpha, float beta, int32_t numWorkgroupX, int32_t numWorkgroupY) {
    int tx, ty;
    grid_tile((int)blockIdx.x, (int)blockIdx.y, numWorkgroupX, numWorkgroupY, tx, ty);
    gemm_tile(a, b, c, d, m, n, k, lda, ldb, ldc, ldd, alpha, beta, tx, ty, 0u, k,
              Fixup{FIX_NONE, nullptr, nullptr, 1u, 0u}, (int)threadIdx.x);
}

#if SG_SPLITK
// Split-K variant: the reference's 15 arguments, then
//   offset 80 ws (float*)   88 tickets (uint32_t*)   96 splits (uint32_t) -> 100 B, padded to 104
// Launch: grid = (numWorkgroupX, numWorkgroupY, splits), splits >= 1.
// Work-group (x, y, z) takes tile (x, y) and K range z: the K tiles are split
// into `splits` ranges of ceil(K tiles / splits) (the last takes the
// remainder; ranges past the end are empty and contribute a zero partial).
// ws holds numWorkgroupX * numWorkgroupY * splits * MT0 * MT1 floats;
// tickets holds numWorkgroupX * numWorkgroupY zeros before the first launch
// and is left zeroed by every launch.  Launches sharing ws/tickets must not
// overlap.
extern "C" __global__ void __launch_bounds__(sg::G::NT) SG_OCC_ATTR
SG_KERNEL_NAME_SPLITK(const float* __restrict__ a, const float* __restrict__ b,
                      const float* c, float* d,
                      uint32_t m, uint32_t n, uint32_t k,
                      uint32_t lda, uint32_t ldb, uint32_t ldc, uint32_t ldd,
                      float alpha, float beta, int32_t numWorkgroupX, int32_t numWorkgroupY,
                      float* ws, uint32_t* tickets, uint32_t splits) {
    constexpr uint32_t DK = SG_DK;
    int tx, ty;
    grid_tile((int)blockIdx.x, (int)blockIdx.y, numWorkgroupX, numWorkgroupY, tx, ty);
    const uint32_t split = blockIdx.z;
    const uint32_t kt_all = (k + DK - 1) / DK;
    const uint32_t per = (kt_all + splits - 1) / splits;
    const uint32_t k_first = min(split * per, kt_all) * DK;
    const uint32_t k_end = min(k_first + per * DK, k);
    const uint32_t tile = (uint32_t)tx + (uint32_t)ty * (uint32_t)numWorkgroupX;
    gemm_tile(a, b, c, d, m, n, k, lda, ldb, ldc, ldd, alpha, beta, tx, ty, k_first,
              k_end > k_first ? k_end - k_first : 0u,
              Fixup{FIX_SPLIT, ws + (size_t)tile * splits * (sg::G::MT0 * sg::G::MT1), tickets + tile, splits, split},
              (int)threadIdx.x);
}
#endif

#if SG_STREAMK
// Stream-K variant for tile grids that leave a partial last round of
// work-groups: the reference's 15 arguments, then
//   offset 80 ws (float*)   88 tickets (uint32_t*)   96 sk_tiles (uint32_t)   100 groups (uint32_t) -> 104 B
// Launch: grid = (G, 1, 1), G = groups (passed explicitly: the kernel reads no
// hidden argument; for speed at most the work-groups resident at once, though
// no work-group ever waits for another), with
// T = numWorkgroupX * numWorkgroupY tiles, G <= sk_tiles <= T, and T - sk_tiles
// a multiple of G, and sk_tiles * ceil(k / DK) * G below 2^32.  The K tiles of
// the first sk_tiles logical tiles form one
// sequence of sk_tiles * ceil(k / DK) iterations; work-group w (after the XCD
// renumbering) takes iterations [S w / G, S (w + 1) / G), at least one tile's
// worth, so every tile of the sequence is cut at most once, at a work-group
// boundary: the two work-groups either side of boundary w store partials 0
// (head) and 1 (tail) of ws[w], and the later one adds them and runs the
// epilogue.  Then the work-group runs the remaining (data-parallel) tiles
// sk_tiles + w, + G, ... whole.  ws holds G * 2 * MT0 * MT1 floats and tickets
// G zeros, left zero by the launch; launches sharing them must not overlap.
extern "C" __global__ void __launch_bounds__(sg::G::NT) SG_OCC_ATTR
SG_KERNEL_NAME_STREAMK(const float* __restrict__ a, const float* __restrict__ b,
                       const float* c, float* d,
                       uint32_t m, uint32_t n, uint32_t k,
                       uint32_t lda, uint32_t ldb, uint32_t ldc, uint32_t ldd,
                       float alpha, float beta, int32_t numWorkgroupX, int32_t numWorkgroupY,
                       float* ws, uint32_t* tickets, uint32_t sk_tiles, uint32_t groups) {
    constexpr uint32_t DK = SG_DK;
    constexpr size_t PART_FLOATS = (size_t)sg::G::MT0 * sg::G::MT1;
    const uint32_t w = (uint32_t)sg::xcd_order((int)blockIdx.x, (int)groups);
    const uint32_t tiles = (uint32_t)numWorkgroupX * (uint32_t)numWorkgroupY;
    const uint32_t kt = (k + DK - 1) / DK;
    // 32-bit iteration arithmetic: the host keeps sk_tiles * kt * groups below 2^32
    const uint32_t total = sk_tiles * kt;
    const uint32_t it_end = total * (w + 1) / groups;
    uint32_t it = total * w / groups;
    uint32_t dp = sk_tiles + w;
    // one call site for both phases: the stream-K iterations first, then the
    // data-parallel tiles (a second inlined copy of the tile would double the
    // kernel's registers)
    for (;;) {
        uint32_t t, k0, k1;
        if (it < it_end) {
            t = it / kt;
            k0 = it - t * kt;
            k1 = min(kt, it_end - t * kt);
            it = t * kt + k1;
        } else if (dp < tiles) {
            t = dp;
            k0 = 0;
            k1 = kt;
            dp += groups;
        } else {
            break;
        }
        Fixup fx{FIX_NONE, nullptr, nullptr, 1u, 0u};
        if (k0 > 0 || k1 < kt) {
            // cut at boundary w (this work-group has the tail, from k0) or
            // w + 1 (the head, up to k1)
            const uint32_t bnd = k0 > 0 ? w : w + 1;
            fx = Fixup{FIX_STREAM, ws + (size_t)bnd * 2 * PART_FLOATS, tickets + bnd, 2u, k0 > 0 ? 1u : 0u};
        }
        int tx, ty;
        sg::tile_coords((int)t, numWorkgroupX, numWorkgroupY, tx, ty);
        const uint32_t kf = k0 * DK, ke = min(k1 * DK, k);
        // the thread index made opaque per tile: nothing derived from it is
        // hoisted out of this loop to stay live through the K loop
        int tid = (int)threadIdx.x;
        asm volatile("" : "+v"(tid));
        __syncthreads();  // every wave is done with the previous tile's LDS
        gemm_tile(a, b, c, d, m, n, k, lda, ldb, ldc, ldd, alpha, beta, tx, ty, kf, ke - kf, fx, tid);
    }
}
#endif
