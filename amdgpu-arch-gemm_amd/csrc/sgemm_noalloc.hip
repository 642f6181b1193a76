// sgemm_launch_noalloc: sgemm_launch for callers that cannot allocate device
// memory (code under HIP graph capture, serving loops, harnesses that forbid
// hipMalloc).  A split-K or stream-K launch needs a workspace -- partial tiles
// and their tickets -- which sgemm_launch allocates on the handle's first
// launch that needs it; here it lives in a fixed device array, `scratch`,
// compiled into this library, one copy per device, held until the process
// ends.  Nothing on this path calls hipMalloc, hipFree or any allocating
// routine.
//
// Host code never uses the array's name as a device address: the address of
// each device's copy is looked up once, with that device current, through
// hipGetSymbolAddress, and that pointer is what the kernels receive.  The
// lookup runs in sgemm_open (noalloc_prepare) for the handle's device, so a
// launch -- even the first one on a device, even under graph capture -- only
// reads the stored pointer.

#include "sgemm_internal.hpp"

#include <hip/hip_runtime.h>

#include <cstdio>
#include <mutex>

namespace {

constexpr size_t kTicketBytes = (size_t)SGEMM_NOALLOC_MAX_TILES * 4u;
constexpr size_t kScratchBytes = (size_t)SGEMM_NOALLOC_PARTIAL_BYTES + kTicketBytes;

// Split-K partials (the first SGEMM_NOALLOC_PARTIAL_BYTES bytes), then the
// tickets.  Every call on a device shares that device's copy and leaves its
// contents behind; tickets are cleared by every call that uses them.
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

// Zeroes the tickets of one launch (a kernel rather than a memset, so that a
// caller may capture the call in a HIP graph).
__global__ void __launch_bounds__(256) clear_tickets(uint32_t* __restrict__ t, uint32_t count) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i < count) t[i] = 0u;
}

constexpr int kMaxDevices = 64;
std::mutex g_mutex;
void* g_scratch[kMaxDevices];  // device address of each device's `scratch`, null until looked up

// Address of `scratch` on device `dev`, looked up once per device with that
// device current (the calling thread's current device is restored).
int scratch_address(int dev, void** out) {
    if (dev < 0 || dev >= kMaxDevices) return sgemm_internal::set_error(SGEMM_E_INVALID, "device id out of range");
    std::lock_guard<std::mutex> lock(g_mutex);
    if (!g_scratch[dev]) {
        int cur = 0;
        hipError_t e = hipGetDevice(&cur);
        if (e == hipSuccess && cur != dev) e = hipSetDevice(dev);
        void* p = nullptr;
        if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (cur != dev) (void)hipSetDevice(cur);
        if (e != hipSuccess || !p) {
            char msg[256];
            snprintf(msg, sizeof(msg), "hipGetSymbolAddress(scratch) on device %d failed: %s (%d)", dev,
                     hipGetErrorString(e), (int)e);
            return sgemm_internal::set_error(e != hipSuccess ? (int)e : SGEMM_E_NO_DEVICE, msg);
        }
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    return SGEMM_OK;
}

}  // namespace

int sgemm_internal::noalloc_prepare(int dev) {
    void* p = nullptr;
    return scratch_address(dev, &p);
}

extern "C" int sgemm_launch_noalloc(sgemm_handle* h, const float* dA, const float* dB, const float* dC, float* dD,
                                    uint32_t m, uint32_t n, uint32_t k, uint32_t lda, uint32_t ldb, uint32_t ldc,
                                    uint32_t ldd, float alpha, float beta) {
    if (!h) return sgemm_internal::set_error(SGEMM_E_INVALID, "sgemm_launch_noalloc: null handle");
    int r = sgemm_internal::check_launch(h, dA, dB, dC, dD, m, n, k, lda, ldb, ldc, ldd, beta);
    if (r != SGEMM_OK || m == 0 || n == 0) return r;
    hipStream_t s = sgemm_internal::stream(h);
    sgemm_internal::Part parts[3];
    const int count = sgemm_internal::decompose(h, m, n, k, lda, ldb, ldc, ldd, parts);
    // every part's needs are checked before anything is launched
    for (int q = 0; q < count; ++q) {
        const sgemm_internal::Part& pt = parts[q];
        if (pt.kh != h && (r = sgemm_check_shape(pt.kh, pt.m, pt.n, k, lda, ldb, ldc, ldd)) != SGEMM_OK) return r;
        const sgemm_internal::Plan p = sgemm_internal::plan(pt.kh, pt.m, pt.n, k);
        if (p.partial_bytes > (size_t)SGEMM_NOALLOC_PARTIAL_BYTES || p.ticket_count > (size_t)SGEMM_NOALLOC_MAX_TILES) {
            char msg[256];
            snprintf(msg, sizeof(msg),
                     "sgemm_launch_noalloc: a %ux%ux%u launch (%u K ranges, %u stream-K tiles) needs %zu bytes of "
                     "partials and %zu tickets; the static scratch holds %u bytes and %u tickets", pt.m, pt.n, k,
                     p.splits, p.sk_tiles, p.partial_bytes, p.ticket_count, (unsigned)SGEMM_NOALLOC_PARTIAL_BYTES,
                     (unsigned)SGEMM_NOALLOC_MAX_TILES);
            return sgemm_internal::set_error(SGEMM_E_SHAPE, msg);
        }
    }
    for (int q = 0; q < count; ++q) {
        const sgemm_internal::Part& pt = parts[q];
        const float* a = dA ? dA + pt.a_off : dA;
        const float* b = dB ? dB + pt.b_off : dB;
        const float* c = dC ? dC + pt.c_off : dC;
        float* d = dD + pt.d_off;
        const sgemm_internal::Plan p = sgemm_internal::plan(pt.kh, pt.m, pt.n, k);
        if (!p.partial_bytes) {  // generated_gemm uses no workspace
            r = sgemm_internal::launch(pt.kh, a, b, c, d, pt.m, pt.n, k, lda, ldb, ldc, ldd, alpha, beta, nullptr, s);
            if (r != SGEMM_OK) return r;
            continue;
        }
        void* base = nullptr;
        if ((r = scratch_address(sgemm_internal::device(h), &base)) != SGEMM_OK) return r;
        float* partials = static_cast<float*>(base);
        uint32_t* tickets =
            reinterpret_cast<uint32_t*>(static_cast<unsigned char*>(base) + SGEMM_NOALLOC_PARTIAL_BYTES);
        // the parts run in order on one stream, so they share the scratch
        hipLaunchKernelGGL(clear_tickets, dim3((unsigned)((p.ticket_count + 255) / 256)), dim3(256), 0, s, tickets,
                           (uint32_t)p.ticket_count);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) {
            char msg[256];
            snprintf(msg, sizeof(msg), "clear_tickets launch failed: %s (%d)", hipGetErrorString(e), (int)e);
            return sgemm_internal::set_error((int)e, msg);
        }
        const sgemm_internal::Workspace ws{partials, (size_t)SGEMM_NOALLOC_PARTIAL_BYTES, tickets,
                                           (size_t)SGEMM_NOALLOC_MAX_TILES};
        r = sgemm_internal::launch(pt.kh, a, b, c, d, pt.m, pt.n, k, lda, ldb, ldc, ldd, alpha, beta, &ws, s);
        if (r != SGEMM_OK) return r;
    }
    return SGEMM_OK;
}
