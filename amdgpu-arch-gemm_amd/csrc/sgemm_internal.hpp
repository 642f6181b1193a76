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

// K ranges, partial bytes and output tiles of an m x n x k launch with the
// handle's current split setting (no device work).
SGEMM_INTERNAL int plan(const sgemm_handle* h, uint32_t m, uint32_t n, uint32_t k, uint32_t* splits,
                        size_t* ws_bytes, size_t* tiles);

// Shape, pointer and alignment checks of sgemm_launch.
SGEMM_INTERNAL int check_launch(const sgemm_handle* h, const float* dA, const float* dB, const float* dC, float* dD,
                                uint32_t m, uint32_t n, uint32_t k, uint32_t lda, uint32_t ldb, uint32_t ldc,
                                uint32_t ldd, float beta);

// Enqueues one checked launch on the handle's stream.  A split launch uses
// `ws` (its sizes must cover plan()'s needs); an unsplit one ignores it.
SGEMM_INTERNAL int launch(sgemm_handle* h, const float* dA, const float* dB, const float* dC, float* dD, uint32_t m,
                          uint32_t n, uint32_t k, uint32_t lda, uint32_t ldb, uint32_t ldc, uint32_t ldd, float alpha,
                          float beta, const Workspace* ws);

SGEMM_INTERNAL hipStream_t stream(const sgemm_handle* h);
SGEMM_INTERNAL int device(const sgemm_handle* h);
// Records `message` as the calling thread's sgemm_last_error and returns `code`.
SGEMM_INTERNAL int set_error(int code, const char* message);

}  // namespace sgemm_internal
