/*
 * TEST INFRASTRUCTURE -- the CPU oracle for the gfx950 SGEMM.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker / the timed CPU baseline; the
 * product (amdgpu-arch-gemm_amd/) never links or calls it.
 *
 * Contents
 *   oracle_cpu_gemm        restatement of the reference runner's cpuGemm
 *                          (/root/reference/runner/generator_runner.cpp:16-33):
 *                          i -> j -> l loops, float accumulator, products and
 *                          sums rounded separately (built with
 *                          -ffp-contract=off), then d = beta*c + alpha*acc.
 *                          Pinned bit-exactly against the reference's own
 *                          cpuGemm compiled from its source (oracle/_ref), and
 *                          against hand-computed and closed-form cases.
 *   oracle_cpu_gemm_mt     the same arithmetic with columns split over threads
 *                          (bitwise identical: every output keeps its order).
 *   oracle_cpu_gemm_blocked
 *                          the same arithmetic again, cache- and register-
 *                          blocked so that whole-matrix checks at 4096^3 take
 *                          seconds: each output still owns one float
 *                          accumulator that adds the rounded products for
 *                          l = 0..k-1 in order, and the vector lanes run over
 *                          rows i (separate outputs), so the result is bitwise
 *                          that of oracle_cpu_gemm.  Pinned bitwise against it
 *                          and against the reference's cpuGemm (oracle/_ref).
 *   oracle_gemm_f64        double-accumulated reference (error bounds).
 *   oracle_splitmix64_at   SplitMix64 (Steele, Lea, Flood 2014; Vigna's
 *                          public-domain splitmix64.c), output i from state key.
 *   oracle_fill            restatement of the seeded input generator of
 *                          include/sgemm_shim.h (sgemm_fill): U[-1,1) from the
 *                          top 24 bits, N(0,1) by Box-Muller on word pairs.
 *                          It replaces the reference's unseeded mt19937
 *                          randomize() (runner/Utils/BufferUtils.hpp:6-16), so
 *                          there is no reference output to pin it to; it is
 *                          pinned by SplitMix64's published outputs, exactness
 *                          of the uniform map, a committed fixture and a
 *                          numpy restatement.
 */
#include <math.h>
#include <pthread.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>

void oracle_cpu_gemm(const float* a, const float* b, const float* c, float* d, float alpha, float beta,
                     uint32_t m, uint32_t n, uint32_t k) {
    for (uint32_t i = 0; i < m; ++i) {
        for (uint32_t j = 0; j < n; ++j) {
            float acc = 0.0f;
            for (uint32_t l = 0; l < k; ++l) acc += a[i + (size_t)l * m] * b[l + (size_t)j * k];
            const size_t idx = i + (size_t)j * m;
            d[idx] = beta * c[idx] + alpha * acc;
        }
    }
}

struct cols_job {
    const float *a, *b, *c;
    float* d;
    float alpha, beta;
    uint32_t m, k, j0, j1;
};

static void* cols_worker(void* p) {
    const struct cols_job* jb = (const struct cols_job*)p;
    /* the column slice [j0, j1) is itself a cpuGemm with n = j1 - j0 */
    oracle_cpu_gemm(jb->a, jb->b + (size_t)jb->j0 * jb->k, jb->c + (size_t)jb->j0 * jb->m,
                    jb->d + (size_t)jb->j0 * jb->m, jb->alpha, jb->beta, jb->m, jb->j1 - jb->j0, jb->k);
    return NULL;
}

int oracle_cpu_gemm_mt(const float* a, const float* b, const float* c, float* d, float alpha, float beta,
                       uint32_t m, uint32_t n, uint32_t k, int threads) {
    if (threads < 1) threads = 1;
    if ((uint32_t)threads > n) threads = n ? (int)n : 1;
    pthread_t tid[256];
    int created[256];
    struct cols_job jobs[256];
    if (threads > 256) threads = 256;
    const uint32_t chunk = (n + (uint32_t)threads - 1) / (uint32_t)threads;
    for (int t = 0; t < threads; ++t) {
        created[t] = 0;
        uint32_t j0 = (uint32_t)t * chunk, j1 = j0 + chunk;
        if (j1 > n) j1 = n;
        if (j0 >= j1) continue;
        jobs[t].a = a; jobs[t].b = b; jobs[t].c = c; jobs[t].d = d;
        jobs[t].alpha = alpha; jobs[t].beta = beta;
        jobs[t].m = m; jobs[t].k = k; jobs[t].j0 = j0; jobs[t].j1 = j1;
        if (pthread_create(&tid[t], NULL, cols_worker, &jobs[t]) == 0)
            created[t] = 1;
        else
            cols_worker(&jobs[t]); /* run inline if no thread is available */
    }
    for (int t = 0; t < threads; ++t)
        if (created[t]) pthread_join(tid[t], NULL);
    return 0;
}

/* ------------------------------------------------------ blocked cpuGemm */
/* An FB_R x FB_C block of outputs accumulates in acc[][] over l in order;
 * only the loop nest differs from oracle_cpu_gemm, never the operations a
 * single output sees (acc = acc + a*b rounded at each step, then
 * d = beta*c + alpha*acc).  Built with -ffp-contract=off: no fused
 * multiply-add may merge a product into its sum. */
enum { FB_R = 32, FB_C = 4 };

__attribute__((target_clones("avx2", "default"), optimize("O3")))
static void gemm_block_full(const float* a, const float* b, const float* c, float* d, float alpha, float beta,
                            uint32_t m, uint32_t k, uint32_t i0, uint32_t j0) {
    float acc[FB_C][FB_R];
    for (int jj = 0; jj < FB_C; ++jj)
        for (int ii = 0; ii < FB_R; ++ii) acc[jj][ii] = 0.0f;
    const float* bj0 = b + (size_t)j0 * k;
    for (uint32_t l = 0; l < k; ++l) {
        const float* al = a + (size_t)l * m + i0;
        for (int jj = 0; jj < FB_C; ++jj) {
            const float bl = bj0[l + (size_t)jj * k];
            for (int ii = 0; ii < FB_R; ++ii) acc[jj][ii] += al[ii] * bl;
        }
    }
    for (int jj = 0; jj < FB_C; ++jj)
        for (int ii = 0; ii < FB_R; ++ii) {
            const size_t idx = (size_t)(i0 + ii) + (size_t)(j0 + jj) * m;
            d[idx] = beta * c[idx] + alpha * acc[jj][ii];
        }
}

/* a partial block at the bottom or right edge: rows <= FB_R, cols <= FB_C */
static void gemm_block_edge(const float* a, const float* b, const float* c, float* d, float alpha, float beta,
                            uint32_t m, uint32_t k, uint32_t i0, uint32_t j0, uint32_t rows, uint32_t cols) {
    float acc[FB_C][FB_R];
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

static void* blocked_worker(void* p) {
    const struct cols_job* jb = (const struct cols_job*)p;
    /* row blocks outside, so one block's A rows (FB_R x k floats) are reused
     * from cache by every column block of this thread's range */
    for (uint32_t i0 = 0; i0 < jb->m; i0 += FB_R) {
        const uint32_t rows = jb->m - i0 < FB_R ? jb->m - i0 : FB_R;
        for (uint32_t j0 = jb->j0; j0 < jb->j1; j0 += FB_C) {
            const uint32_t cols = jb->j1 - j0 < FB_C ? jb->j1 - j0 : FB_C;
            if (rows == FB_R && cols == FB_C)
                gemm_block_full(jb->a, jb->b, jb->c, jb->d, jb->alpha, jb->beta, jb->m, jb->k, i0, j0);
            else
                gemm_block_edge(jb->a, jb->b, jb->c, jb->d, jb->alpha, jb->beta, jb->m, jb->k, i0, j0, rows, cols);
        }
    }
    return NULL;
}

int oracle_cpu_gemm_blocked(const float* a, const float* b, const float* c, float* d, float alpha, float beta,
                            uint32_t m, uint32_t n, uint32_t k, int threads) {
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    /* whole column blocks per thread */
    const uint32_t col_blocks = (n + FB_C - 1) / FB_C;
    if ((uint32_t)threads > col_blocks) threads = col_blocks ? (int)col_blocks : 1;
    pthread_t tid[256];
    int created[256];
    struct cols_job jobs[256];
    const uint32_t per = (col_blocks + (uint32_t)threads - 1) / (uint32_t)threads;
    for (int t = 0; t < threads; ++t) {
        created[t] = 0;
        uint32_t j0 = (uint32_t)t * per * FB_C, j1 = j0 + per * FB_C;
        if (j1 > n) j1 = n;
        if (j0 >= j1) continue;
        jobs[t].a = a; jobs[t].b = b; jobs[t].c = c; jobs[t].d = d;
        jobs[t].alpha = alpha; jobs[t].beta = beta;
        jobs[t].m = m; jobs[t].k = k; jobs[t].j0 = j0; jobs[t].j1 = j1;
        if (pthread_create(&tid[t], NULL, blocked_worker, &jobs[t]) == 0)
            created[t] = 1;
        else
            blocked_worker(&jobs[t]);
    }
    for (int t = 0; t < threads; ++t)
        if (created[t]) pthread_join(tid[t], NULL);
    return 0;
}

void oracle_gemm_f64(const float* a, const float* b, const float* c, double* d, double alpha, double beta,
                     uint32_t m, uint32_t n, uint32_t k) {
    for (uint32_t j = 0; j < n; ++j) {
        for (uint32_t i = 0; i < m; ++i) {
            double acc = 0.0;
            for (uint32_t l = 0; l < k; ++l) acc += (double)a[i + (size_t)l * m] * (double)b[l + (size_t)j * k];
            const size_t idx = i + (size_t)j * m;
            d[idx] = beta * (double)c[idx] + alpha * acc;
        }
    }
}

/* ---------------------------------------------------------------- inputs */
static const uint64_t GAMMA = 0x9E3779B97F4A7C15ull;

static uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t oracle_splitmix64_at(uint64_t key, uint64_t i) { return mix64(key + (i + 1) * GAMMA); }

uint64_t oracle_stream_key(uint64_t seed, uint32_t matrix_id) {
    return mix64(seed ^ (0xD1B54A32D192ED03ull * (uint64_t)(matrix_id + 1)));
}

int oracle_fill(float* out, size_t count, uint64_t seed, uint32_t matrix_id, int dist) {
    const uint64_t key = oracle_stream_key(seed, matrix_id);
    for (size_t i = 0; i < count; ++i) {
        if (dist == 0) {
            const uint64_t w = oracle_splitmix64_at(key, i);
            out[i] = (float)(w >> 40) / 16777216.0f * 2.0f - 1.0f;
        } else if (dist == 1) {
            const uint64_t p = i >> 1;
            const double u1 = ((double)((oracle_splitmix64_at(key, 2 * p) >> 11) + 1)) / 9007199254740992.0;
            const double u2 = ((double)(oracle_splitmix64_at(key, 2 * p + 1) >> 11)) / 9007199254740992.0;
            const double r = sqrt(-2.0 * log(u1));
            const double th = 2.0 * 3.141592653589793 * u2;
            out[i] = (float)((i & 1) ? r * sin(th) : r * cos(th));
        } else if (dist == 2) {
            out[i] = 0.0f;
        } else {
            return -1;
        }
    }
    return 0;
}
