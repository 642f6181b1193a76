// The runner's CPU validation GEMMs (amdgpu-arch-gemm_amd/runner/cpu_reference.hpp)
// under sanitizers: built by tests/test_sanitizers.py twice, once with
// AddressSanitizer + UndefinedBehaviorSanitizer and once with ThreadSanitizer
// (the column-split loop, the blocked loop and the float64 reference each
// share the output among worker threads).  Every shape runs all of them:
//   * runner_cpu_gemm at 1 and 3 threads and runner_cpu_gemm_blocked at 1, 5
//     and 64 threads must agree bitwise (one summation order per output);
//   * runner_cpu_reference, with a budget large enough for the whole matrix
//     and with a zero budget (one column timed), must fill the same result
//     and report agreement;
//   * runner_gemm_f64 at 1 and 7 threads must agree exactly, and the float
//     result must lie within 1e-5 * sqrt(k) of it, normwise.
// Shapes cover the blocked loop's full and partial row and column blocks,
// more threads than column blocks, and empty dimensions.  Exit 0 when every
// check holds; a failed check prints its shape and exits 1, a sanitizer
// report aborts.
#include "cpu_reference.hpp"

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <sstream>
#include <vector>

namespace {

// U[-1, 1) from a 64-bit LCG (Knuth's MMIX constants), top 24 bits
void fill(std::vector<float>& v, uint64_t seed) {
    uint64_t s = seed * 0x9E3779B97F4A7C15ull + 1;
    for (float& x : v) {
        s = s * 6364136223846793005ull + 1442695040888963407ull;
        x = (float)((double)(s >> 40) / (double)(1u << 23) - 1.0);
    }
}

bool same_bits(const std::vector<float>& x, const std::vector<float>& y) {
    return x.size() == y.size() && (x.empty() || std::memcmp(x.data(), y.data(), x.size() * sizeof(float)) == 0);
}

int failures = 0;

void expect(bool ok, const char* what, uint32_t m, uint32_t n, uint32_t k) {
    if (!ok) {
        std::printf("FAIL %s at m=%u n=%u k=%u\n", what, m, n, k);
        ++failures;
    }
}

void check_shape(uint32_t m, uint32_t n, uint32_t k, float alpha, float beta) {
    const size_t mn = (size_t)m * n;
    std::vector<float> a((size_t)m * k), b((size_t)k * n), c(mn);
    fill(a, 1000003u * m + 7u * k + 1u);
    fill(b, 1000033u * n + 11u * k + 2u);
    fill(c, 1000037u * m + 13u * n + 3u);
    const float* pa = a.data();
    const float* pb = b.data();
    const float* pc = c.data();

    std::vector<float> want(mn, -7.0f);
    runner_cpu_gemm(pa, pb, pc, want.data(), alpha, beta, m, n, k, 1);
    for (unsigned threads : {3u}) {
        std::vector<float> d(mn, -7.0f);
        runner_cpu_gemm(pa, pb, pc, d.data(), alpha, beta, m, n, k, threads);
        expect(same_bits(d, want), "runner_cpu_gemm thread count", m, n, k);
    }
    for (unsigned threads : {1u, 5u, 64u}) {
        std::vector<float> d(mn, -7.0f);
        runner_cpu_gemm_blocked(pa, pb, pc, d.data(), alpha, beta, m, n, k, threads);
        expect(same_bits(d, want), "runner_cpu_gemm_blocked", m, n, k);
    }
    for (double budget : {1e9, 0.0}) {
        std::vector<float> d(mn, -7.0f);
        std::ostringstream log;
        const bool agreed = runner_cpu_reference(pa, pb, pc, d.data(), alpha, beta, m, n, k, 4, budget, log);
        expect(agreed, "runner_cpu_reference reports agreement", m, n, k);
        expect(same_bits(d, want), "runner_cpu_reference result", m, n, k);
        expect(log.str().find("cpuGemm blocked, 4 threads: ") != std::string::npos, "runner_cpu_reference log", m,
               n, k);
    }
    std::vector<double> ref(mn, -7.0), ref7(mn, -7.0);
    runner_gemm_f64(pa, pb, pc, ref.data(), alpha, beta, m, n, k, 1);
    runner_gemm_f64(pa, pb, pc, ref7.data(), alpha, beta, m, n, k, 7);
    expect(ref.empty() || std::memcmp(ref.data(), ref7.data(), mn * sizeof(double)) == 0,
           "runner_gemm_f64 thread count", m, n, k);
    const double err = runner_normwise_error(want.data(), ref.data(), mn);
    expect(err <= 1e-5 * std::sqrt((double)(k ? k : 1)), "normwise error of the float loop", m, n, k);
}

}  // namespace

int main() {
    const uint32_t shapes[][3] = {
        {1, 1, 1},   {37, 29, 301}, {70, 9, 64},   {64, 8, 33},  {32, 4, 5},    {33, 5, 17},
        {96, 12, 1}, {5, 130, 40},  {128, 67, 19}, {31, 3, 200}, {256, 64, 512}, {17, 1, 1000},
        {0, 9, 13},  {9, 0, 13},    {9, 13, 0},    {0, 0, 0},
    };
    for (const auto& s : shapes) check_shape(s[0], s[1], s[2], 0.5f, -2.0f);
    check_shape(45, 22, 77, 1.0f, 0.0f);
    check_shape(45, 22, 77, -1.5f, 1.0f);

    // the error measure: exact agreement, a known relative error, NaN
    const std::vector<double> ref = {2.0, -4.0, 1.0};
    const std::vector<float> x0 = {2.0f, -4.0f, 1.0f}, x1 = {2.0f, -3.0f, 1.0f}, x2 = {NAN, -4.0f, 1.0f};
    expect(runner_normwise_error(x0.data(), ref.data(), 3) == 0.0, "normwise error of an exact result", 3, 1, 0);
    expect(runner_normwise_error(x1.data(), ref.data(), 3) == 0.25, "normwise error of 1 in 4", 3, 1, 0);
    expect(std::isinf(runner_normwise_error(x2.data(), ref.data(), 3)), "normwise error with NaN", 3, 1, 0);
    expect(!runner_host_cpu_model().empty(), "host CPU model", 0, 0, 0);

    std::printf("%s (%d failed checks)\n", failures ? "FAIL" : "ok", failures);
    return failures ? 1 : 0;
}
