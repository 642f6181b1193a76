// Library-internal interface between the host library's translation units
// (sgemm_shim.cpp and sgemm_noalloc.hip).  Nothing here is part of the C-ABI:
// the symbols have hidden visibility and C++ linkage.
#pragma once

#include "sgemm_shim.h"

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>

#define SGEMM_INTERNAL __attribute__((visibility("hidden")))

namespace sgemm_internal {

// Device memory a split-K launch works in: the tile partials and one ticket
// per output tile (zero before the launch; the kernel leaves them zero).
struct Workspace {
    float* partials;
    size_t partial_bytes;
    uint32_t* tickets;
    size_t ticket_count;
};

// How an m x n x k launch runs with the handle's current settings: plain
// (splits == 1, sk_tiles == 0), split-K (splits > 1) or stream-K (sk_tiles >
// 0 over sk_groups work-groups), and the workspace it needs.
struct Plan {
    uint32_t splits = 1;
    uint32_t sk_tiles = 0;
    uint32_t sk_groups = 0;
    size_t tiles = 0;
    size_t partial_bytes = 0;
    size_t ticket_count = 0;
};
SGEMM_INTERNAL Plan plan(const sgemm_handle* h, uint32_t m, uint32_t n, uint32_t k);

// Shape, pointer and alignment checks of sgemm_launch.
SGEMM_INTERNAL int check_launch(const sgemm_handle* h, const float* dA, const float* dB, const float* dC, float* dD,
                                uint32_t m, uint32_t n, uint32_t k, uint32_t lda, uint32_t ldb, uint32_t ldc,
                                uint32_t ldd, float beta);

// Enqueues one checked launch of h's kernels on `stream`.  A split-K or
// stream-K launch uses `ws` (its sizes must cover plan()'s needs); a plain one
// ignores it.
SGEMM_INTERNAL int launch(sgemm_handle* h, const float* dA, const float* dB, const float* dC, float* dD, uint32_t m,
                          uint32_t n, uint32_t k, uint32_t lda, uint32_t ldb, uint32_t ldc, uint32_t ldd, float alpha,
                          float beta, const Workspace* ws, hipStream_t stream);

// One part of a launch: kernel handle `kh` on an m x n block whose A, B, C,
// D start `*_off` floats into the caller's matrices.
struct Part {
    sgemm_handle* kh;
    uint32_t m, n;
    size_t a_off, b_off, c_off, d_off;
};
// The parts of an m x n x k launch of h (sgemm_set_edge_kernels), in launch
// order on h's stream: the whole problem on h, or h on the tile-aligned
// interior plus the row-strip kernel on a thin bottom strip (rows past the
// last whole tile row, every column) and the column-strip kernel on a thin
// right strip (columns past the last whole tile column, interior rows).  A
// strip is thin when it is at most a quarter of h's tile, and is split off
// only when that takes a round of work-groups off h's grid.  Returns 1..3.
SGEMM_INTERNAL int decompose(const sgemm_handle* h, uint32_t m, uint32_t n, uint32_t k, uint32_t lda, uint32_t ldb,
                             uint32_t ldc, uint32_t ldd, Part out[3]);

// Looks up the device address of sgemm_launch_noalloc's static scratch on
// device `dev` (once per device; later calls return at once).  sgemm_open
// calls it for the handle's device, so launches never do.
SGEMM_INTERNAL int noalloc_prepare(int dev);

SGEMM_INTERNAL hipStream_t stream(const sgemm_handle* h);
SGEMM_INTERNAL int device(const sgemm_handle* h);
// Records `message` as the calling thread's sgemm_last_error and returns `code`.
SGEMM_INTERNAL int set_error(int code, const char* message);

}  // namespace sgemm_internal
