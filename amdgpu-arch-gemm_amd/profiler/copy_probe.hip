// copy_probe: a plain device-to-device copy of a known number of bytes, used to
// calibrate rocprofv3's FETCH_SIZE / WRITE_SIZE counters on this GPU.
//
//   copy_probe <bytes> <launches>
//
// Each launch reads exactly <bytes> and writes exactly <bytes> with 16-byte
// vector accesses (grid-stride loop, every element touched once).  The buffers
// are far larger than the caches when <bytes> is large, so the counters of one
// launch should read <bytes> / 1024 KiB each; the ratio actual/expected is the
// scale factor applied to the SGEMM kernel's counter values.

#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

__global__ void __launch_bounds__(256) copy_probe_kernel(const float4* __restrict__ src, float4* __restrict__ dst,
                                                         size_t n) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) dst[i] = src[i];
}

#define CHECK(call)                                                                      \
    do {                                                                                 \
        hipError_t e_ = (call);                                                          \
        if (e_ != hipSuccess) {                                                          \
            fprintf(stderr, "%s failed: %s\n", #call, hipGetErrorString(e_));           \
            return 1;                                                                    \
        }                                                                                \
    } while (0)

int main(int argc, char** argv) {
    if (argc < 3) {
        fprintf(stderr, "usage: %s <bytes> <launches>\n", argv[0]);
        return 2;
    }
    const size_t bytes = strtoull(argv[1], nullptr, 10) / 16 * 16;
    const int launches = atoi(argv[2]);
    if (bytes == 0 || launches <= 0) {
        fprintf(stderr, "bytes and launches must be positive\n");
        return 2;
    }
    float4 *src = nullptr, *dst = nullptr;
    CHECK(hipMalloc(&src, bytes));
    CHECK(hipMalloc(&dst, bytes));
    CHECK(hipMemset(src, 0, bytes));
    const size_t n = bytes / 16;
    const unsigned blocks = 256 * 8;
    hipEvent_t a, b;
    CHECK(hipEventCreate(&a));
    CHECK(hipEventCreate(&b));
    CHECK(hipEventRecord(a, nullptr));
    for (int i = 0; i < launches; ++i) copy_probe_kernel<<<blocks, 256>>>(src, dst, n);
    CHECK(hipGetLastError());
    CHECK(hipEventRecord(b, nullptr));
    CHECK(hipEventSynchronize(b));
    float ms = 0.0f;
    CHECK(hipEventElapsedTime(&ms, a, b));
    printf("copy_probe: %zu bytes x %d launches, %.4f ms/launch, %.1f GB/s (read+write)\n", bytes, launches,
           ms / launches, 2.0 * bytes / (ms / launches * 1e-3) / 1e9);
    CHECK(hipFree(src));
    CHECK(hipFree(dst));
    return 0;
}
