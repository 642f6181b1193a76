// GeneratorRunner: benchmark and validate one generated gfx950 SGEMM code object.
//
//   GeneratorRunner <co> <toml> M N K <num_warmup_runs> <num_benchmark_runs> <validation_flag>
//                   [seed] [dist] [alpha] [beta]
//
// The first eight arguments and the last three stdout lines
// ("ASM gemm: <ms> ms", "Gflops: <x>", "GiB/s: <x>") are those of the reference
// runner (README.md:84, generator_runner.cpp:192-283), which the tuner parses
// (sgemm_tuner.py:115).  Differences, all deliberate:
//   * inputs are seeded (sgemm_fill): A = matrix 0, B = matrix 1, C = matrix 2,
//     with the optional [seed] (default 0) and [dist] (0 = U[-1,1), 1 = N(0,1));
//     the reference's randomize() is unseeded (BufferUtils.hpp:6-16);
//   * alpha = beta = 1 by default, as in the reference (generator_runner.cpp:219-220);
//     [alpha] [beta] override them;
//   * every HIP error is checked and reported; usage errors exit with -1 before
//     any argument is touched (the reference reads argv first, :193-201);
//   * "cpuGemm func" is the reference's single-threaded loop, timed once (the
//     reference divides the single run by numRuns, :229); past a 3 s budget it
//     runs on a column slice and the scaled figure says so.  The whole-matrix
//     reference comes from a blocked, multithreaded loop that is bitwise the
//     same (checked on the slice), on a line of its own, next to the host CPU
//     model and hardware_concurrency;
//   * validation needs both the normwise
//     criterion max|D - D_ref| / max|D_ref| <= 1e-5 * sqrt(K) and the
//     reference's elementwise |gpu - cpu| < 1e-3 (its mismatch count is printed
//     in the reference's "# of mismatches: N/(m*n)" form);
//   * the naive HIP comparison kernel (:35-67, :246-265) is not run.
// Exit code 0 = pass, -1 (255) = usage error, HIP error or validation failure.

#include "sgemm_shim.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <exception>
#include <iostream>
#include <string>
#include <thread>
#include <vector>

#include "cpu_reference.hpp"

namespace {

// single-thread time the reference-loop cpuGemm may take in a validation run;
// beyond it the loop runs on a column slice and the figure is scaled
constexpr double kCpuBudgetMs = 3000.0;

double gflops(uint32_t m, uint32_t n, uint32_t k, double ms) {  // generator_runner.cpp:75-77
    return 2.0 * m * n * k / ms * 1e-6;
}

double mem_bw_gib(size_t m, size_t n, size_t k, double ms) {  // generator_runner.cpp:79-83
    return (double)(m * k + n * k + 2 * m * n) * sizeof(float) / ms / 1024.0 / 1024.0;
}

bool parse_u32(const char* s, uint32_t* out) {
    char* end = nullptr;
    unsigned long long v = strtoull(s, &end, 10);
    if (!s[0] || *end || v > 0xffffffffull) return false;
    *out = (uint32_t)v;
    return true;
}

int usage(const char* prog) {
    std::cerr << "usage: " << prog
              << " <co> <toml> M N K <num_warmup_runs> <num_benchmark_runs> <validation_flag>"
                 " [seed] [dist] [alpha] [beta]\n";
    return -1;
}

int shim_error(const char* what, int code) {
    std::cerr << what << " failed (" << code << "): " << sgemm_last_error() << "\n";
    return -1;
}

}  // namespace

int run(int argc, char** argv);

int main(int argc, char** argv) {
    try {
        return run(argc, argv);
    } catch (const std::exception& e) {  // host buffers of a shape this host cannot hold
        std::cerr << "GeneratorRunner: " << e.what() << "\n";
        return -1;
    }
}

int run(int argc, char** argv) {
    if (argc < 9) return usage(argv[0]);
    uint32_t m, n, k, warmup, runs, validate, seed = 0, dist = SGEMM_DIST_UNIFORM;
    if (!parse_u32(argv[3], &m) || !parse_u32(argv[4], &n) || !parse_u32(argv[5], &k) ||
        !parse_u32(argv[6], &warmup) || !parse_u32(argv[7], &runs) || !parse_u32(argv[8], &validate) ||
        (argc > 9 && !parse_u32(argv[9], &seed)) || (argc > 10 && !parse_u32(argv[10], &dist)))
        return usage(argv[0]);
    float alpha = 1.0f, beta = 1.0f;
    if (argc > 11) alpha = strtof(argv[11], nullptr);
    if (argc > 12) beta = strtof(argv[12], nullptr);
    if (runs == 0) runs = 1;

    sgemm_handle* h = nullptr;
    int r = sgemm_open(argv[1], argv[2], &h);
    if (r != SGEMM_OK) return shim_error("sgemm_open", r);
    sgemm_kernel_info info{};
    if ((r = sgemm_get_info(h, &info)) != SGEMM_OK) {
        sgemm_close(h);
        return shim_error("sgemm_get_info", r);
    }
    r = sgemm_check_shape(h, m, n, k, info.trans_a ? k : m, info.trans_b ? n : k, m, m);
    if (r != SGEMM_OK) {
        std::cerr << sgemm_last_error() << "\n";
        sgemm_close(h);
        return -1;
    }

    int splits = 1;
    if ((r = sgemm_launch_splits(h, m, n, k, &splits)) != SGEMM_OK) {
        sgemm_close(h);
        return shim_error("sgemm_launch_splits", r);
    }
    std::cout << "K ranges per output tile: " << splits << (splits > 1 ? " (generated_gemm_splitk)" : "") << "\n";

    std::vector<float> A((size_t)m * k), B((size_t)k * n), C((size_t)m * n), D((size_t)m * n, 0.0f);
    if ((r = sgemm_fill(A.data(), A.size(), seed, 0, (int)dist)) != SGEMM_OK ||
        (r = sgemm_fill(B.data(), B.size(), seed, 1, (int)dist)) != SGEMM_OK ||
        (r = sgemm_fill(C.data(), C.size(), seed, 2, (int)dist)) != SGEMM_OK) {
        sgemm_close(h);
        return shim_error("sgemm_fill", r);
    }

    std::vector<float> ref;
    std::vector<double> ref64;
    if (validate) {
        ref.assign((size_t)m * n, 0.0f);
        // The stored A is k x m and B is n x k for transposed kernels; the CPU
        // reference multiplies the column-major op(A) (m x k) and op(B) (k x n).
        std::vector<float> opA, opB;
        const float* pa = A.data();
        const float* pb = B.data();
        if (info.trans_a) {
            opA.resize(A.size());
            for (uint32_t l = 0; l < k; ++l)
                for (uint32_t i = 0; i < m; ++i) opA[i + (size_t)l * m] = A[l + (size_t)i * k];
            pa = opA.data();
        }
        if (info.trans_b) {
            opB.resize(B.size());
            for (uint32_t j = 0; j < n; ++j)
                for (uint32_t l = 0; l < k; ++l) opB[l + (size_t)j * k] = B[j + (size_t)l * n];
            pb = opB.data();
        }
        const unsigned threads = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
        if (!runner_cpu_reference(pa, pb, C.data(), ref.data(), alpha, beta, m, n, k, threads, kCpuBudgetMs,
                                  std::cout)) {
            std::cerr << "the blocked CPU reference differs from the reference loop\n";
            sgemm_close(h);
            return -1;
        }
        ref64.assign((size_t)m * n, 0.0);
        runner_gemm_f64(pa, pb, C.data(), ref64.data(), alpha, beta, m, n, k, threads);
    }

    double ms = 0.0;
    r = sgemm_run(h, A.data(), B.data(), C.data(), D.data(), m, n, k, alpha, beta, (int)warmup, (int)runs, &ms);
    if (r != SGEMM_OK) {
        sgemm_close(h);
        return shim_error("sgemm_run", r);
    }
    sgemm_close(h);

    int status = 0;
    if (validate) {
        double max_err = 0.0, max_ref = 0.0;
        size_t worst = 0, bad = 0;
        for (size_t i = 0; i < D.size(); ++i) {
            const double e = std::fabs((double)D[i] - (double)ref[i]);
            if (!(e <= max_err)) {  // also catches NaN
                max_err = std::isnan(e) ? INFINITY : e;
                worst = i;
            }
            max_ref = std::max(max_ref, std::fabs((double)ref[i]));
            if (std::isnan(D[i]) != std::isnan(ref[i])) ++bad;
        }
        const double rel = max_ref > 0 ? max_err / max_ref : max_err;
        const double tol = 1e-5 * std::sqrt((double)std::max<uint32_t>(k, 1));
        const bool normwise_pass = rel <= tol && bad == 0;
        // the reference's elementwise rule as well: almostEqual(gpu, cpu, 1e-3),
        // i.e. |gpu - cpu| < 1e-3 (Math.hpp:5-8), first 10 mismatches printed
        // and counted over all m * n outputs (generator_runner.cpp:292-303)
        size_t mismatches = 0;
        for (size_t i = 0; i < D.size(); ++i) {
            if (!(std::fabs(D[i] - ref[i]) < 1e-3f)) {
                if (mismatches < 10)
                    std::cout << "gpu & cpu results mismatched at index: " << i << "\n"
                              << D[i] << " != " << ref[i] << "\n";
                ++mismatches;
            }
        }
        const bool pass = normwise_pass && mismatches == 0;
        std::cout << "max |D - D_ref| = " << max_err << " at index " << worst << " (gpu " << D[worst] << ", cpu "
                  << ref[worst] << ")\n"
                  << "normwise relative error = " << rel << " (tolerance 1e-5*sqrt(K) = " << tol << "): "
                  << (normwise_pass ? "pass" : "FAIL") << "\n"
                  << "float64 reference: normwise error of the GPU result "
                  << runner_normwise_error(D.data(), ref64.data(), D.size()) << ", of cpuGemm "
                  << runner_normwise_error(ref.data(), ref64.data(), ref.size()) << "\n"
                  << "# of mismatches: " << mismatches << "/" << D.size() << "\n"
                  << "validation: " << (pass ? "PASS" : "FAIL") << "\n";
        status = pass ? 0 : -1;
    }
    const double tflops = gflops(m, n, k, ms) * 1e-3;
    std::cout << "TFLOP/s: " << tflops << " (" << 100.0 * tflops / 157.3 << "% of the 157.3 TFLOP/s FP32 MFMA peak)\n";
    std::cout << "ASM gemm: " << ms << " ms\n"
              << "Gflops: " << gflops(m, n, k, ms) << '\n'
              << "GiB/s: " << mem_bw_gib(m, n, k, ms) << '\n';
    return status;
}
