// mfma_probe: the FP32 MFMA ceiling the SGEMM kernels are measured against.
//
//   mfma_probe [iterations] [launches]
//
// The headline instance's MFMA stream with no memory traffic: 256 work-groups
// of 4 waves (one per SIMD, one work-group per CU on a 256-CU MI355X), each
// wave issuing v_mfma_f32_32x32x2_f32 into 16 independent 32x32 accumulators,
// 8 k-steps per iteration (one K tile of depth 16).  Prints the launch time
// and TFLOP/s (2 * 32 * 32 * 2 FLOP per MFMA) against the 157.3 TFLOP/s
// nominal peak (256 CU x 256 FLOP/clk x 2.4 GHz).

#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

typedef float f32x16 __attribute__((ext_vector_type(16)));

__global__ void __launch_bounds__(256) mfma_probe_kernel(float* __restrict__ out, int iters) {
    f32x16 acc[4][4];
    for (int i = 0; i < 4; ++i)
        for (int j = 0; j < 4; ++j)
            for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.0f;
    float a[4], b[4];
    for (int i = 0; i < 4; ++i) {
        a[i] = 1e-3f * (float)(threadIdx.x + i);
        b[i] = 1e-3f * (float)(threadIdx.x - i);
    }
    for (int t = 0; t < iters; ++t) {
#pragma unroll
        for (int kk = 0; kk < 8; ++kk)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    // keep every accumulator live: one float per work-item
    float s = 0.0f;
    for (int i = 0; i < 4; ++i)
        for (int j = 0; j < 4; ++j)
            for (int q = 0; q < 16; ++q) s += acc[i][j][q];
    out[blockIdx.x * 256 + threadIdx.x] = s;
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
    const int iters = argc > 1 ? atoi(argv[1]) : 2048;
    const int runs = argc > 2 ? atoi(argv[2]) : 20;
    const int groups = 256;
    if (iters <= 0 || runs <= 0) {
        fprintf(stderr, "usage: %s [iterations > 0] [launches > 0]\n", argv[0]);
        return 1;
    }
    float* out = nullptr;
    CHECK(hipMalloc(&out, (size_t)groups * 256 * sizeof(float)));
    hipEvent_t e0, e1;
    CHECK(hipEventCreate(&e0));
    CHECK(hipEventCreate(&e1));
    for (int w = 0; w < 5; ++w) mfma_probe_kernel<<<groups, 256>>>(out, iters);
    CHECK(hipGetLastError());
    CHECK(hipDeviceSynchronize());
    CHECK(hipEventRecord(e0));
    for (int r = 0; r < runs; ++r) mfma_probe_kernel<<<groups, 256>>>(out, iters);
    CHECK(hipEventRecord(e1));
    CHECK(hipEventSynchronize(e1));
    float ms = 0.0f;
    CHECK(hipEventElapsedTime(&ms, e0, e1));
    ms /= (float)runs;
    const double flops = (double)groups * 4 * iters * 8 * 16 * (2.0 * 32 * 32 * 2);
    const double tflops = flops / ms * 1e-9;
    printf("mfma_probe: %d work-groups x 4 waves, %d iterations: %.4f ms per launch, %.2f TFLOP/s "
           "(%.1f%% of 157.3)\n", groups, iters, ms, tflops, 100.0 * tflops / 157.3);
    CHECK(hipFree(out));
    return 0;
}
