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
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <fstream>
#include <ostream>
#include <string>
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

// The same arithmetic in a cache- and register-blocked loop nest, for
// whole-matrix validation at sizes where the loop above takes minutes: a block
// of kRows x kCols outputs keeps one float accumulator per output and adds the
// rounded products for l = 0..k-1 in order; vector lanes run over rows (other
// outputs).  Only the loop nest differs, never the operations one output sees,
// so the result is bitwise that of runner_cpu_gemm (-ffp-contract=off).
namespace runner_blocked {
constexpr uint32_t kRows = 32, kCols = 4;

// a partial block at the bottom or right edge: rows <= kRows, cols <= kCols
inline void edge_block(const float* a, const float* b, const float* c, float* d, float alpha, float beta,
                       uint32_t m, uint32_t k, uint32_t i0, uint32_t j0, uint32_t rows, uint32_t cols) {
    float acc[kCols][kRows];
    for (uint32_t jj = 0; jj < cols; ++jj)
        for (uint32_t ii = 0; ii < rows; ++ii) acc[jj][ii] = 0.0f;
    for (uint32_t l = 0; l < k; ++l) {
        const float* al = a + (size_t)l * m + i0;
        for (uint32_t jj = 0; jj < cols; ++jj) {
            const float bl = b[l + (size_t)(j0 + jj) * k];
            for (uint32_t ii = 0; ii < rows; ++ii) acc[jj][ii] += al[ii] * bl;
        }
    }
    for (uint32_t jj = 0; jj < cols; ++jj)
        for (uint32_t ii = 0; ii < rows; ++ii) {
            const size_t idx = (size_t)(i0 + ii) + (size_t)(j0 + jj) * m;
            d[idx] = beta * c[idx] + alpha * acc[jj][ii];
        }
}

// AVX2 and baseline clones of the block, picked at load time by an ifunc
// resolver.  A ThreadSanitizer build keeps the baseline body only: the
// resolver runs before that sanitizer's runtime starts and would crash it.
#if defined(__SANITIZE_THREAD__)
#define RUNNER_BLOCK_CLONES
#else
#define RUNNER_BLOCK_CLONES __attribute__((target_clones("avx2", "default")))
#endif

// a whole block, with constant trip counts the compiler vectorises over rows
// (its own body: a callee built without these options would not inline)
RUNNER_BLOCK_CLONES __attribute__((optimize("O3"))) inline void full_block(
    const float* a, const float* b, const float* c, float* d, float alpha, float beta, uint32_t m, uint32_t k,
    uint32_t i0, uint32_t j0) {
    float acc[kCols][kRows];
    for (uint32_t jj = 0; jj < kCols; ++jj)
        for (uint32_t ii = 0; ii < kRows; ++ii) acc[jj][ii] = 0.0f;
    const float* bj0 = b + (size_t)j0 * k;
    for (uint32_t l = 0; l < k; ++l) {
        const float* al = a + (size_t)l * m + i0;
        for (uint32_t jj = 0; jj < kCols; ++jj) {
            const float bl = bj0[l + (size_t)jj * k];
            for (uint32_t ii = 0; ii < kRows; ++ii) acc[jj][ii] += al[ii] * bl;
        }
    }
    for (uint32_t jj = 0; jj < kCols; ++jj)
        for (uint32_t ii = 0; ii < kRows; ++ii) {
            const size_t idx = (size_t)(i0 + ii) + (size_t)(j0 + jj) * m;
            d[idx] = beta * c[idx] + alpha * acc[jj][ii];
        }
}

// columns [j0, j1): row blocks outside, so one block's A rows are reused from
// cache by every column block of the range
inline void cols(const float* a, const float* b, const float* c, float* d, float alpha, float beta, uint32_t m,
                 uint32_t k, uint32_t j0, uint32_t j1) {
    for (uint32_t i0 = 0; i0 < m; i0 += kRows) {
        const uint32_t rows = std::min(kRows, m - i0);
        for (uint32_t j = j0; j < j1; j += kCols) {
            const uint32_t nc = std::min(kCols, j1 - j);
            if (rows == kRows && nc == kCols)
                full_block(a, b, c, d, alpha, beta, m, k, i0, j);
            else
                edge_block(a, b, c, d, alpha, beta, m, k, i0, j, rows, nc);
        }
    }
}
}  // namespace runner_blocked

inline void runner_cpu_gemm_blocked(const float* a, const float* b, const float* c, float* d, float alpha,
                                    float beta, uint32_t m, uint32_t n, uint32_t k, unsigned threads) {
    using runner_blocked::kCols;
    const uint32_t col_blocks = (n + kCols - 1) / kCols;
    threads = std::max(1u, std::min<unsigned>(threads, col_blocks ? col_blocks : 1));
    const uint32_t per = (col_blocks + threads - 1) / threads;
    std::vector<std::thread> pool;
    for (unsigned t = 0; t < threads; ++t) {
        const uint32_t j0 = std::min<uint64_t>(n, (uint64_t)t * per * kCols);
        const uint32_t j1 = std::min<uint64_t>(n, (uint64_t)(t + 1) * per * kCols);
        if (j0 >= j1) continue;
        if (threads == 1)
            runner_blocked::cols(a, b, c, d, alpha, beta, m, k, j0, j1);
        else
            pool.emplace_back(runner_blocked::cols, a, b, c, d, alpha, beta, m, k, j0, j1);
    }
    for (auto& th : pool) th.join();
}

// "model name" of the first processor in /proc/cpuinfo ("unknown" if absent)
inline std::string runner_host_cpu_model() {
    std::ifstream f("/proc/cpuinfo");
    std::string line;
    while (std::getline(f, line)) {
        if (line.compare(0, 10, "model name") == 0) {
            const size_t colon = line.find(':');
            if (colon != std::string::npos) {
                size_t p = line.find_first_not_of(" \t", colon + 1);
                return p == std::string::npos ? std::string("unknown") : line.substr(p);
            }
        }
    }
    return "unknown";
}

// The validation run's CPU reference, with the reference runner's figure:
//   * "cpuGemm func: <ms> ms" is the reference's single-threaded loop
//     (generator_runner.cpp:225-230), one run, not divided by the run count.
//     When the whole matrix would take longer than `budget_ms`, the loop runs
//     on the first s columns only (each column is an independent cpuGemm of
//     n = 1, so the slice is exactly that many columns of the full result), and
//     the line gives the scaled whole-matrix figure with the slice it came from.
//   * The full reference `ref` comes from the blocked loop over `threads`
//     threads, printed on its own line, and is checked bitwise against the
//     single-thread loop's columns.
// Returns false if the two disagree (which would make the validation moot).
inline bool runner_cpu_reference(const float* a, const float* b, const float* c, float* ref, float alpha, float beta,
                                 uint32_t m, uint32_t n, uint32_t k, unsigned threads, double budget_ms,
                                 std::ostream& out) {
    using clk = std::chrono::steady_clock;
    const unsigned hw = std::thread::hardware_concurrency();
    out << "host CPU: " << runner_host_cpu_model() << ", hardware_concurrency " << hw << "\n";
    std::vector<float> slice;
    uint32_t s = 0;
    double slice_ms = 0.0;
    if (n) {
        // one column first, to size the slice to the budget
        slice.assign((size_t)m * n, 0.0f);
        auto t0 = clk::now();
        runner_cpu_gemm_cols(a, b, c, slice.data(), alpha, beta, m, k, 0, 1);
        const double one = std::chrono::duration<double, std::milli>(clk::now() - t0).count();
        s = 1;
        slice_ms = one;
        const double want = one > 0 ? budget_ms / one : (double)n;
        const uint32_t target = (uint32_t)std::max(1.0, std::min<double>(n, want));
        if (target > 1) {
            t0 = clk::now();
            runner_cpu_gemm_cols(a, b, c, slice.data(), alpha, beta, m, k, 0, target);
            slice_ms = std::chrono::duration<double, std::milli>(clk::now() - t0).count();
            s = target;
        }
    }
    if (s == n) {
        out << "cpuGemm func: " << slice_ms << " ms (1 thread, reference loop order, whole matrix)\n";
    } else {
        out << "cpuGemm func: " << slice_ms * n / s << " ms (1 thread, reference loop order; scaled by " << n << "/"
            << s << " from columns [0, " << s << ") of " << n << ", measured in " << slice_ms << " ms)\n";
    }
    const auto t0 = clk::now();
    runner_cpu_gemm_blocked(a, b, c, ref, alpha, beta, m, n, k, threads);
    const double blocked_ms = std::chrono::duration<double, std::milli>(clk::now() - t0).count();
    const size_t checked = (size_t)m * s * sizeof(float);  // zero when m or n is: no pointer is read then
    const bool same = checked == 0 || std::memcmp(slice.data(), ref, checked) == 0;
    out << "cpuGemm blocked, " << threads << " threads: " << blocked_ms << " ms (whole matrix; bitwise "
        << (same ? "equal" : "DIFFERENT") << " to the 1-thread loop on columns [0, " << s << "))\n";
    return same;
}

// float64 reference for the error report: for each column j, acc[i] += a[i + l*m] * b[l + j*k]
// in double (column-major friendly order), then d = beta * c + alpha * acc.  The
// rounding of this sum is ~1e-16 relative, so it measures the error of both the
// GPU result and the float cpuGemm above.
// Eight columns share each pass over A.
__attribute__((optimize("O3"))) inline void runner_gemm_f64_cols(const float* a, const float* b, const float* c,
                                                                 double* d, double alpha, double beta, uint32_t m,
                                                                 uint32_t k, uint32_t j0, uint32_t j1) {
    constexpr uint32_t kJ = 8;
    std::vector<double> acc((size_t)kJ * m);
    for (uint32_t j = j0; j < j1; j += kJ) {
        const uint32_t nj = std::min(kJ, j1 - j);
        std::fill(acc.begin(), acc.end(), 0.0);
        for (uint32_t l = 0; l < k; ++l) {
            const float* al = a + (size_t)l * m;
            for (uint32_t jj = 0; jj < nj; ++jj) {
                const double bl = b[l + (size_t)(j + jj) * k];
                double* ac = acc.data() + (size_t)jj * m;
                for (uint32_t i = 0; i < m; ++i) ac[i] += (double)al[i] * bl;
            }
        }
        for (uint32_t jj = 0; jj < nj; ++jj)
            for (uint32_t i = 0; i < m; ++i) {
                const size_t idx = i + (size_t)(j + jj) * m;
                d[idx] = beta * (double)c[idx] + alpha * acc[(size_t)jj * m + i];
            }
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
