/*
 * C-ABI of the gfx950 SGEMM host library (libsgemm_shim.so).
 *
 * The reference has no library boundary: its Python side shells out to the
 * GeneratorRunner executable (tuner/sgemm_tuner.py:112) and the executable
 * does everything in main().  This header is that executable's work split
 * into plain C entry points -- plain pointers and sizes, no C++ or torch
 * types -- so that Python (ctypes), the GeneratorRunner executable and any
 * other host language bind the same code.  Each entry point names the
 * reference code it replaces.
 *
 * Conventions
 *   - Every function returns 0 on success.  A positive value is the
 *     hipError_t of the failing HIP call; a negative value is one of the
 *     SGEMM_E_* codes below.  sgemm_last_error() returns a message for the
 *     last failure on the calling thread.  Nothing throws across this ABI.
 *   - The caller owns host arrays.  Device buffers come from sgemm_malloc and
 *     are owned by the caller until sgemm_free.  A handle owns its code
 *     object module, its stream and its events.
 *   - One handle is used by one thread at a time.  All work of a handle runs
 *     in order on the handle's stream (default priority).
 *   - Matrices are column-major FP32.  D = alpha * op(A) * op(B) + beta * C
 *     with op(A) m x k and op(B) k x n; A is stored m x k (lda >= m), or
 *     k x m (lda >= k) for a kernel built with trans_a; B is stored k x n
 *     (ldb >= k), or n x k (ldb >= n) with trans_b; C and D are m x n
 *     (ldc, ldd >= m).  C is not read when beta == 0.  dC may equal dD (with
 *     ldc == ldd): an in-place update D = alpha * op(A) * op(B) + beta * D.
 *     Any other overlap of D with C (when beta != 0), A or B is refused with
 *     SGEMM_E_INVALID: tiles write D while other tiles still read them.
 */
#ifndef SGEMM_SHIM_H
#define SGEMM_SHIM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SGEMM_SHIM_ABI_VERSION 9

/* Most K ranges generated_gemm_splitk splits one output tile into. */
#define SGEMM_MAX_SPLIT_K 16

enum {
    SGEMM_OK = 0,
    SGEMM_E_INVALID = -1,     /* bad argument (null pointer, bad distribution, ...) */
    SGEMM_E_IO = -2,          /* a file could not be read */
    SGEMM_E_CONFIG = -3,      /* .toml missing a key or describing an unsupported kernel */
    SGEMM_E_SHAPE = -4,       /* problem shape / leading dimensions the kernel cannot run */
    SGEMM_E_NO_DEVICE = -5    /* no HIP device visible */
};

enum {
    SGEMM_DIST_UNIFORM = 0,   /* U[-1, 1): exact multiples of 2^-23 */
    SGEMM_DIST_NORMAL = 1,    /* N(0, 1) by Box-Muller on pairs of uniforms */
    SGEMM_DIST_ZERO = 2       /* all zeros */
};

typedef struct sgemm_handle sgemm_handle;

/* Kernel configuration read from the .toml (generator.py:1001-1017 schema). */
typedef struct sgemm_kernel_info {
    int mfma[4];          /* atom (M, N, blocks, K) */
    int wave_group[2];
    int wave_tiling[2];
    int depth_k;
    int vmem_stage;
    int wavefront_size;
    int lds_usage_bytes;
    int tile_m;           /* MT0 = mfma[0] * wave_group[0] * wave_tiling[0] */
    int tile_n;           /* MT1 = mfma[1] * wave_group[1] * wave_tiling[1] */
    int workitems;        /* wave_group[0] * wave_group[1] * wavefront_size */
    int trans_a;          /* 1: A is stored k x m (lda >= k), op(A) = A^T */
    int trans_b;          /* 1: B is stored n x k (ldb >= n), op(B) = B^T */
    int split_k;          /* K ranges per output tile for sgemm_launch: 0 = chosen per problem
                             (sgemm_set_split_k), else a fixed count (toml key split_k, default 1) */
    int split_k_max;      /* SGEMM_MAX_SPLIT_K if the code object has generated_gemm_splitk, else 1 */
    int stream_k;         /* stream-K setting for unsplit launches (sgemm_set_stream_k; toml key
                             stream_k, default 0) */
    int stream_k_groups;  /* work-groups of generated_gemm_streamk resident at once (per-CU occupancy
                             x compute units), 0 when the code object has no stream-K kernel */
    int stream_k_rounds;  /* most rounds of whole tiles the auto setting still uses stream-K for
                             (toml key stream_k_rounds; 0: no limit) */
} sgemm_kernel_info;

/* Message of the last failure on this thread ("" if none). */
const char* sgemm_last_error(void);

/* ABI version of the loaded library (SGEMM_SHIM_ABI_VERSION). */
int sgemm_abi_version(void);

/* Device 0 properties: name, compute units, peak engine clock (kHz), LDS per
 * work-group (bytes).  Any output pointer may be null.
 * Replaces nothing in the reference (it never queries the device). */
int sgemm_device_info(char* name, size_t name_len, int* compute_units, int* clock_khz, int* lds_per_block);

/* Loads <co_path> (symbol "generated_gemm", and "generated_gemm_splitk" when
 * present) and its <toml_path> config.  It also looks up, once per device,
 * the device address of sgemm_launch_noalloc's static scratch on the current
 * device, so no launch ever does (the first no-alloc call may be captured).
 * Replaces getAsmKernelConfig + prepareASMKernel (generator_runner.cpp:100-124, :69-73). */
int sgemm_open(const char* co_path, const char* toml_path, sgemm_handle** out);

/* Unloads the module and releases the stream and events (generator_runner.cpp:318).
 * A handle attached to others as an edge kernel (sgemm_set_edge_kernels) is
 * detached from them first: their later launches run the whole problem on
 * their own kernel. */
void sgemm_close(sgemm_handle* h);

/* Copies the handle's kernel configuration (generator_runner.cpp:127-153 geometry). */
int sgemm_get_info(const sgemm_handle* h, sgemm_kernel_info* info);

/* Returns SGEMM_OK if the kernel can run this problem, SGEMM_E_SHAPE with a
 * message otherwise.  Any m, n, k is accepted (edge tiles and a K remainder are
 * masked in the kernel); the leading dimensions must cover the stored
 * matrices (lda >= m, or k with trans_a; ldb >= k, or n with trans_b;
 * ldc, ldd >= m), and one tile's span of each matrix must stay below 2^31
 * bytes (lda * depth_k, or lda * tile_m with trans_a; ldb * tile_n, or
 * ldb * depth_k with trans_b; ldc * tile_n and ldd * tile_n, times 4). */
int sgemm_check_shape(const sgemm_handle* h, uint32_t m, uint32_t n, uint32_t k,
                      uint32_t lda, uint32_t ldb, uint32_t ldc, uint32_t ldd);

/* Sets the number of K ranges (1..split_k_max) each output tile is split into
 * by later launches; 1 launches generated_gemm.  0 chooses per problem: with
 * T = ceil(m/MT0) * ceil(n/MT1) tiles and C compute units, no split when
 * T >= C; else the s in 1..min(split_k_max, ceil(k/depth_k) / 4) with the
 * least ceil(T * s / C) * (ceil(ceil(k/depth_k) / s) + 4) -- rounds of
 * work-groups times the K tiles of a range plus 4 for each range's fixed cost
 * -- (the smallest s among ties), so a problem with few tiles and a deep K
 * still fills the GPU.
 * With s > 1 ranges, sgemm_launch runs generated_gemm_splitk over a grid of
 * (ceil(m/MT0), ceil(n/MT1), s') blocks, s' = min(s, ceil(k/depth_k)): every
 * block multiplies one range of whole K tiles and the last block of a tile
 * to finish sums the partials in range order, so results do not depend on
 * timing.  The handle allocates the
 * partials (sgemm_workspace_size bytes) on the first launch that needs more
 * than it holds.  No counterpart in the reference, whose kernel has no K split
 * (its knob set is generator.py:827-854). */
int sgemm_set_split_k(sgemm_handle* h, int splits);

/* Device bytes the handle's workspace needs for an m x n x k launch with its
 * current split and stream-K settings (0 when the launch needs none; h's own
 * part: the interior when edge kernels take strips).  No
 * counterpart in the reference (its kernel needs no workspace). */
int sgemm_workspace_size(const sgemm_handle* h, uint32_t m, uint32_t n, uint32_t k, size_t* bytes);

/* K ranges an m x n x k launch with the handle's current setting uses on
 * h's own part (the interior when edge kernels take strips; 1:
 * generated_gemm, no split).  No counterpart in the reference. */
int sgemm_launch_splits(const sgemm_handle* h, uint32_t m, uint32_t n, uint32_t k, int* splits);

/* Sets how unsplit launches treat a tile grid that leaves a partial last
 * round of work-groups: 0 never uses stream-K; 1 (auto) launches
 * generated_gemm_streamk when the grid of T tiles over G = stream_k_groups
 * resident work-groups has T > G and ceil(T / G) rounds cost at least 3% over
 * T / G, within the instance's stream_k_rounds; 2 whenever T > G.  The stream-K launch runs G work-groups: the last
 * partial round plus one whole round of tiles (T % G + G tiles, G when T % G
 * == 0) are cut into G equal runs of K iterations, each at least one tile
 * long, so a tile is cut at most once and its two partials are added by the
 * later of the two work-groups (the same bits whichever finishes last); the
 * other tiles run whole.  The handle's workspace then holds 2 G partial tiles
 * and G tickets.  SGEMM_E_CONFIG without generated_gemm_streamk.  No
 * counterpart in the reference (its grid is one work-group per tile,
 * generator_runner.cpp:127-131). */
int sgemm_set_stream_k(sgemm_handle* h, int mode);

/* Attaches two other loaded kernels with the same trans_a / trans_b that
 * later launches of h use for thin edge strips: `rows` (tile_m below h's)
 * for the strip of rows past the last whole tile row, every column, when
 * m % MT0 is at most a quarter of h's tile height; `cols` (tile_n below h's)
 * for the strip of columns past the last whole tile column, interior rows,
 * when n % MT1 is at most a quarter of h's tile width -- and only when that
 * takes a round of work-groups off h's grid (ceil(tiles / resident
 * work-groups) falls; of the two strips, the fewest that reach the same
 * rounds).  h's own kernel then runs only the tile-aligned interior, and the
 * strips follow it on h's
 * stream, instead of paying a whole tile of MFMA work for each
 * sliver (4097^3 in 256 x 128 tiles: 561 tiles, 49 of them one row or one
 * column wide).  The strips use their kernels' own split-K / stream-K
 * settings and workspace.  Either may be NULL (that strip then stays with
 * h); the same handle may serve both.
 * Closing an attached handle detaches it (h's strips then stay with h).  A
 * handle serving as another's edge kernel cannot take edge kernels itself.
 * The attached handles must not run other work concurrently with launches
 * through h.  No counterpart in the
 * reference, whose tuner skips shapes its tiles do not divide
 * (tuner/sgemm_tuner.py:97-100). */
int sgemm_set_edge_kernels(sgemm_handle* h, sgemm_handle* rows, sgemm_handle* cols);

/* sgemm_set_edge_kernels(h, edge, edge). */
int sgemm_set_edge_kernel(sgemm_handle* h, sgemm_handle* edge);

/* The interior (*m_int x *n_int) an m x n x k launch of h gives h's own
 * kernel: m and n unless an edge kernel takes thin strips.  No counterpart in
 * the reference. */
int sgemm_edge_interior(const sgemm_handle* h, uint32_t m, uint32_t n, uint32_t k, uint32_t* m_int, uint32_t* n_int);

/* Tiles an m x n x k launch with the handle's current settings gives the
 * stream-K phase of h's own kernel (on the interior when edge kernels take
 * strips; 0: the launch does not use generated_gemm_streamk).  No
 * counterpart in the reference. */
int sgemm_stream_k_tiles(const sgemm_handle* h, uint32_t m, uint32_t n, uint32_t k, int* sk_tiles);

/* Device memory (generator_runner.cpp:236-242, :291, :319-322). */
int sgemm_malloc(void** dptr, size_t bytes);
int sgemm_free(void* dptr);
int sgemm_memcpy_h2d(void* dst, const void* src, size_t bytes);
int sgemm_memcpy_d2h(void* dst, const void* src, size_t bytes);
int sgemm_memset(void* dptr, int value, size_t bytes);

/* Enqueues one launch on the handle's stream; does not wait.
 * Replaces makeKernelArguments + launchASMKernel (generator_runner.cpp:126-190):
 * the same 80-byte kernarg buffer, passed through hipModuleLaunchKernel's
 * HIP_LAUNCH_PARAM_BUFFER_POINTER with a grid of (ceil(m/MT0), ceil(n/MT1)) blocks.
 * With a split count above 1 (sgemm_set_split_k) it launches the split kernel
 * instead (or, under sgemm_set_stream_k, the stream-K kernel), with the handle's
 * workspace; launches of one handle share that
 * workspace, so they must run in order on the handle's stream.  Device
 * pointers need 4-byte alignment only (SGEMM_E_INVALID otherwise). */
int sgemm_launch(sgemm_handle* h, const float* dA, const float* dB, const float* dC, float* dD,
                 uint32_t m, uint32_t n, uint32_t k, uint32_t lda, uint32_t ldb, uint32_t ldc, uint32_t ldd,
                 float alpha, float beta);

/* Static split-K scratch of sgemm_launch_noalloc: bytes of tile partials and
 * output tiles (one ticket each) one launch may use. */
#define SGEMM_NOALLOC_PARTIAL_BYTES (32u << 20)
#define SGEMM_NOALLOC_MAX_TILES 16384u

/* sgemm_launch without any device allocation.  No counterpart in the
 * reference (its kernel needs no workspace); it is for callers that cannot
 * call hipMalloc: code under HIP graph capture, serving loops, harnesses that
 * forbid allocation.  Same arguments, checks and results as sgemm_launch
 * (bit-identical D for the same handle settings); a split launch takes its
 * partials and tickets from a fixed device array compiled into this library
 * (SGEMM_NOALLOC_PARTIAL_BYTES + 4 * SGEMM_NOALLOC_MAX_TILES bytes per device,
 * held until the process ends) instead of the handle's workspace, and clears
 * the tickets it uses with a kernel on the handle's stream.  A launch
 * needing more partial bytes or tiles than that returns SGEMM_E_SHAPE.  Every call on
 * a device shares that device's array: calls that overlap on one device (two
 * streams, two handles, two threads) race and must be ordered by the caller. */
int sgemm_launch_noalloc(sgemm_handle* h, const float* dA, const float* dB, const float* dC, float* dD,
                         uint32_t m, uint32_t n, uint32_t k, uint32_t lda, uint32_t ldb, uint32_t ldc, uint32_t ldd,
                         float alpha, float beta);

/* `warmup` untimed launches, then `runs` launches bracketed by HIP events on
 * the handle's stream; *total_ms is the event time of all `runs` launches.
 * Replaces the timed loop of generator_runner.cpp:270-283. */
int sgemm_time(sgemm_handle* h, const float* dA, const float* dB, const float* dC, float* dD,
               uint32_t m, uint32_t n, uint32_t k, uint32_t lda, uint32_t ldb, uint32_t ldc, uint32_t ldd,
               float alpha, float beta, int warmup, int runs, float* total_ms);

/* Like sgemm_time but brackets every launch with its own event pair and
 * writes `runs` per-launch times (ms) to per_launch_ms. */
int sgemm_time_each(sgemm_handle* h, const float* dA, const float* dB, const float* dC, float* dD,
                    uint32_t m, uint32_t n, uint32_t k, uint32_t lda, uint32_t ldb, uint32_t ldc, uint32_t ldd,
                    float alpha, float beta, int runs, float* per_launch_ms);

/* Waits for all work of the handle's stream. */
int sgemm_synchronize(sgemm_handle* h);

/* Makes later launches, timings and synchronisations of h use `stream` (a
 * hipStream_t of the handle's device -- one of another device is refused
 * with SGEMM_E_INVALID -- owned by the caller, who keeps it alive
 * while h uses it) instead of the stream h created at sgemm_open; NULL goes
 * back to that one.  Work already enqueued through h is waited for first, so
 * the handle's launches stay ordered; the current stream must not be
 * capturing then.  For callers that order the GEMM on their own stream (a
 * framework's current stream, or one under HIP graph capture, where
 * sgemm_launch_noalloc records no allocation).  No counterpart in the
 * reference, which launches on the null stream (generator_runner.cpp:189). */
int sgemm_set_stream(sgemm_handle* h, void* stream);

/* Whole runner flow on host buffers with tight leading dimensions (lda = m
 * or k, ldb = k or n as the kernel's transposition says, ldc = ldd = m):
 * allocate, upload A, B (and C when beta != 0), warm up, time `runs`
 * launches, download D, free.  *ms_per_run = event time / runs.
 * Replaces main()'s device part (generator_runner.cpp:232-291). */
int sgemm_run(sgemm_handle* h, const float* A, const float* B, const float* C, float* D,
              uint32_t m, uint32_t n, uint32_t k, float alpha, float beta,
              int warmup, int runs, double* ms_per_run);

/* Fills host[0..count) with the seeded generator: element i of matrix
 * `matrix_id` under `seed` is a pure function of (seed, matrix_id, i), so any
 * slice can be regenerated independently.  Replaces the unseeded randomize()
 * of BufferUtils.hpp:6-16 (same U[-1, 1) range). */
int sgemm_fill(float* host, size_t count, uint64_t seed, uint32_t matrix_id, int dist);


#ifdef __cplusplus
}
#endif

#endif /* SGEMM_SHIM_H */
