// CPU GEMM the GeneratorRunner validates against when validation_flag = 1.
//
// Same arithmetic as the reference runner's cpuGemm (generator_runner.cpp:16-33):
// for every output (i, j) a float accumulator sums a[i + l*m] * b[l + j*k] for
// l = 0..k-1 in order, then d = beta * c + alpha * acc.  Columns j are split
// over threads; every output keeps its summation order, so the result does not
// depend on the thread count.  This file must be compiled without FP
// contraction (-ffp-contract=off) so that products and sums round separately.
#pragma once

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <thread>
#include <vector>

inline void runner_cpu_gemm_cols(const float* a, const float* b, const float* c, float* d, float alpha, float beta,
                                 uint32_t m, uint32_t k, uint32_t j0, uint32_t j1) {
    for (uint32_t i = 0; i < m; ++i) {
        for (uint32_t j = j0; j < j1; ++j) {
            float acc = 0.0f;
            for (uint32_t l = 0; l < k; ++l) acc += a[i + (size_t)l * m] * b[l + (size_t)j * k];
            const size_t idx = i + (size_t)j * m;
            d[idx] = beta * c[idx] + alpha * acc;
        }
    }
}

inline void runner_cpu_gemm(const float* a, const float* b, const float* c, float* d, float alpha, float beta,
                            uint32_t m, uint32_t n, uint32_t k, unsigned threads) {
    threads = std::max(1u, std::min<unsigned>(threads, n ? n : 1));
    if (threads == 1) {
        runner_cpu_gemm_cols(a, b, c, d, alpha, beta, m, k, 0, n);
        return;
    }
    std::vector<std::thread> pool;
    const uint32_t chunk = (n + threads - 1) / threads;
    for (unsigned t = 0; t < threads; ++t) {
        const uint32_t j0 = t * chunk, j1 = std::min(n, j0 + chunk);
        if (j0 < j1) pool.emplace_back(runner_cpu_gemm_cols, a, b, c, d, alpha, beta, m, k, j0, j1);
    }
    for (auto& th : pool) th.join();
}

// float64 reference for the error report: for each column j, acc[i] += a[i + l*m] * b[l + j*k]
// in double (column-major friendly order), then d = beta * c + alpha * acc.  The
// rounding of this sum is ~1e-16 relative, so it measures the error of both the
// GPU result and the float cpuGemm above.
inline void runner_gemm_f64_cols(const float* a, const float* b, const float* c, double* d, double alpha,
                                 double beta, uint32_t m, uint32_t k, uint32_t j0, uint32_t j1) {
    std::vector<double> acc(m);
    for (uint32_t j = j0; j < j1; ++j) {
        std::fill(acc.begin(), acc.end(), 0.0);
        for (uint32_t l = 0; l < k; ++l) {
            const double bl = b[l + (size_t)j * k];
            const float* al = a + (size_t)l * m;
            for (uint32_t i = 0; i < m; ++i) acc[i] += (double)al[i] * bl;
        }
        for (uint32_t i = 0; i < m; ++i) d[i + (size_t)j * m] = beta * (double)c[i + (size_t)j * m] + alpha * acc[i];
    }
}

inline void runner_gemm_f64(const float* a, const float* b, const float* c, double* d, double alpha, double beta,
                            uint32_t m, uint32_t n, uint32_t k, unsigned threads) {
    threads = std::max(1u, std::min<unsigned>(threads, n ? n : 1));
    std::vector<std::thread> pool;
    const uint32_t chunk = (n + threads - 1) / threads;
    for (unsigned t = 0; t < threads; ++t) {
        const uint32_t j0 = t * chunk, j1 = std::min(n, j0 + chunk);
        if (j0 < j1) pool.emplace_back(runner_gemm_f64_cols, a, b, c, d, alpha, beta, m, k, j0, j1);
    }
    for (auto& th : pool) th.join();
}

// max |x - ref| / max |ref| over all elements (NaN in x counts as infinite error)
inline double runner_normwise_error(const float* x, const double* ref, size_t count) {
    double max_err = 0.0, max_ref = 0.0;
    for (size_t i = 0; i < count; ++i) {
        const double e = std::fabs((double)x[i] - ref[i]);
        max_err = std::isnan(e) ? INFINITY : std::max(max_err, e);
        max_ref = std::max(max_ref, std::fabs(ref[i]));
    }
    return max_ref > 0 ? max_err / max_ref : max_err;
}
