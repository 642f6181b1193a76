// Host library behind include/sgemm_shim.h: loads a generated gfx950 SGEMM
// code object, owns its stream and events, packs the reference's 80-byte
// kernarg buffer and launches through the HIP module API.  Built as
// libsgemm_shim.so; the GeneratorRunner executable and the Python ctypes
// wrapper both call it.

#include "sgemm_shim.h"
#include "sgemm_internal.hpp"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cerrno>
#include <climits>
#include <cmath>
#include <cstdarg>
#include <cstddef>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <map>
#include <mutex>
#include <sstream>
#include <string>
#include <thread>
#include <vector>

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail((int)e, "%s failed: %s (%d)", what, hipGetErrorString(e), (int)e);
}

#define HIP_TRY(call)                                     \
    do {                                                  \
        hipError_t e_ = (call);                           \
        if (e_ != hipSuccess) return hip_fail(e_, #call); \
    } while (0)

// ---------------------------------------------------------------- TOML ----
// The kernel .toml is flat: `key = value` lines whose values are integers,
// booleans, strings or arrays of integers (generator.py:1001-1017).
struct TomlValue {
    enum Kind { INT, BOOL, STRING, INT_ARRAY } kind = INT;
    long long i = 0;
    bool b = false;
    std::string s;
    std::vector<long long> arr;
};

std::string trim(const std::string& x) {
    size_t a = x.find_first_not_of(" \t\r\n");
    if (a == std::string::npos) return "";
    size_t b = x.find_last_not_of(" \t\r\n");
    return x.substr(a, b - a + 1);
}

bool parse_int(const std::string& t, long long* out) {
    if (t.empty()) return false;
    char* end = nullptr;
    errno = 0;
    long long v = strtoll(t.c_str(), &end, 10);
    if (errno || *end != '\0') return false;
    *out = v;
    return true;
}

int parse_toml(const std::string& path, std::map<std::string, TomlValue>* out) {
    std::ifstream f(path);
    if (!f) return fail(SGEMM_E_IO, "cannot open %s", path.c_str());
    std::string line;
    int lineno = 0;
    while (std::getline(f, line)) {
        ++lineno;
        // strip comments outside strings
        bool in_str = false;
        for (size_t i = 0; i < line.size(); ++i) {
            if (line[i] == '"') in_str = !in_str;
            if (line[i] == '#' && !in_str) {
                line.resize(i);
                break;
            }
        }
        line = trim(line);
        if (line.empty()) continue;
        if (line[0] == '[') return fail(SGEMM_E_CONFIG, "%s:%d: tables are not part of the kernel schema", path.c_str(), lineno);
        size_t eq = line.find('=');
        if (eq == std::string::npos) return fail(SGEMM_E_CONFIG, "%s:%d: expected key = value", path.c_str(), lineno);
        std::string key = trim(line.substr(0, eq));
        std::string val = trim(line.substr(eq + 1));
        // bare keys only (A-Z a-z 0-9 _ -), as every key of the schema is
        bool bare = !key.empty();
        for (char ch : key)
            bare = bare && ((ch >= 'A' && ch <= 'Z') || (ch >= 'a' && ch <= 'z') || (ch >= '0' && ch <= '9') ||
                            ch == '_' || ch == '-');
        if (!bare) return fail(SGEMM_E_CONFIG, "%s:%d: bad key", path.c_str(), lineno);
        TomlValue v;
        if (val == "true" || val == "false") {
            v.kind = TomlValue::BOOL;
            v.b = (val == "true");
        } else if (!val.empty() && val[0] == '"') {
            if (val.size() < 2 || val.back() != '"') return fail(SGEMM_E_CONFIG, "%s:%d: bad string", path.c_str(), lineno);
            v.kind = TomlValue::STRING;
            v.s = val.substr(1, val.size() - 2);
        } else if (!val.empty() && val[0] == '[') {
            if (val.back() != ']') return fail(SGEMM_E_CONFIG, "%s:%d: bad array", path.c_str(), lineno);
            v.kind = TomlValue::INT_ARRAY;
            std::stringstream ss(val.substr(1, val.size() - 2));
            std::string item;
            while (std::getline(ss, item, ',')) {
                item = trim(item);
                if (item.empty()) continue;
                long long x;
                if (!parse_int(item, &x)) return fail(SGEMM_E_CONFIG, "%s:%d: bad array item '%s'", path.c_str(), lineno, item.c_str());
                v.arr.push_back(x);
            }
        } else {
            v.kind = TomlValue::INT;
            if (!parse_int(val, &v.i)) {
                // other scalars (floats) are tolerated and ignored by the kernel schema
                v.kind = TomlValue::STRING;
                v.s = val;
            }
        }
        (*out)[key] = v;
    }
    return SGEMM_OK;
}

int toml_int(const std::map<std::string, TomlValue>& t, const char* key, int* out, bool required = true, int dflt = 0) {
    auto it = t.find(key);
    if (it == t.end()) {
        if (required) return fail(SGEMM_E_CONFIG, "kernel config misses key '%s'", key);
        *out = dflt;
        return SGEMM_OK;
    }
    if (it->second.kind != TomlValue::INT) return fail(SGEMM_E_CONFIG, "key '%s' must be an integer", key);
    if (it->second.i < INT_MIN || it->second.i > INT_MAX)
        return fail(SGEMM_E_CONFIG, "key '%s' = %lld does not fit a 32-bit integer", key, it->second.i);
    *out = (int)it->second.i;
    return SGEMM_OK;
}

int toml_bool(const std::map<std::string, TomlValue>& t, const char* key, bool* out) {
    auto it = t.find(key);
    if (it == t.end()) return fail(SGEMM_E_CONFIG, "kernel config misses key '%s'", key);
    if (it->second.kind != TomlValue::BOOL) return fail(SGEMM_E_CONFIG, "key '%s' must be a boolean", key);
    *out = it->second.b;
    return SGEMM_OK;
}

int toml_arr(const std::map<std::string, TomlValue>& t, const char* key, int* out, size_t n) {
    auto it = t.find(key);
    if (it == t.end()) return fail(SGEMM_E_CONFIG, "kernel config misses key '%s'", key);
    if (it->second.kind != TomlValue::INT_ARRAY || it->second.arr.size() < n)
        return fail(SGEMM_E_CONFIG, "key '%s' must be an array of %zu integers", key, n);
    for (size_t i = 0; i < n; ++i) {
        const long long v = it->second.arr[i];
        if (v < INT_MIN || v > INT_MAX)
            return fail(SGEMM_E_CONFIG, "key '%s': item %lld does not fit a 32-bit integer", key, v);
        out[i] = (int)v;
    }
    return SGEMM_OK;
}

#define CFG_TRY(call)                 \
    do {                              \
        int r_ = (call);              \
        if (r_ != SGEMM_OK) return r_; \
    } while (0)

int load_config(const char* path, sgemm_kernel_info* info) {
    std::map<std::string, TomlValue> t;
    CFG_TRY(parse_toml(path, &t));
    int a_type, b_type, cd_type, scalar_type;
    bool trans_a, trans_b;
    // the keys the reference runner reads (generator_runner.cpp:100-124)
    CFG_TRY(toml_int(t, "a_type", &a_type));
    CFG_TRY(toml_int(t, "b_type", &b_type));
    CFG_TRY(toml_int(t, "cd_type", &cd_type));
    CFG_TRY(toml_int(t, "scalar_type", &scalar_type));
    CFG_TRY(toml_arr(t, "mfma", info->mfma, 4));
    CFG_TRY(toml_arr(t, "wave_group", info->wave_group, 2));
    CFG_TRY(toml_arr(t, "wave_tiling", info->wave_tiling, 2));
    CFG_TRY(toml_int(t, "depth_k", &info->depth_k));
    CFG_TRY(toml_bool(t, "trans_a", &trans_a));
    CFG_TRY(toml_bool(t, "trans_b", &trans_b));
    CFG_TRY(toml_int(t, "wavefront_size", &info->wavefront_size));
    CFG_TRY(toml_int(t, "lds_usage_bytes", &info->lds_usage_bytes));
    CFG_TRY(toml_int(t, "vmem_stage", &info->vmem_stage, false, 1));
    // default split count of generated_gemm_splitk (absent: no split; 0: per problem)
    CFG_TRY(toml_int(t, "split_k", &info->split_k, false, 1));
    // default stream-K setting (absent: off)
    CFG_TRY(toml_int(t, "stream_k", &info->stream_k, false, 0));
    if (info->stream_k < 0 || info->stream_k > 2)
        return fail(SGEMM_E_CONFIG, "stream_k = %d outside 0..2", info->stream_k);
    CFG_TRY(toml_int(t, "stream_k_rounds", &info->stream_k_rounds, false, 0));
    if (info->stream_k_rounds < 0) return fail(SGEMM_E_CONFIG, "stream_k_rounds = %d < 0", info->stream_k_rounds);
    if (info->split_k < 0 || info->split_k > SGEMM_MAX_SPLIT_K)
        return fail(SGEMM_E_CONFIG, "split_k = %d outside 0..%d", info->split_k, SGEMM_MAX_SPLIT_K);
    if (a_type || b_type || cd_type || scalar_type) return fail(SGEMM_E_CONFIG, "only FP32 (type 0) kernels are supported");
    info->trans_a = trans_a ? 1 : 0;
    info->trans_b = trans_b ? 1 : 0;
    if (info->wavefront_size != 64) return fail(SGEMM_E_CONFIG, "wavefront_size must be 64 on gfx950");
    const int* mf = info->mfma;
    const bool atom32 = mf[0] == 32 && mf[1] == 32 && mf[2] == 1 && mf[3] == 2;
    const bool atom16 = mf[0] == 16 && mf[1] == 16 && mf[2] == 1 && mf[3] == 4;
    if (!atom32 && !atom16) return fail(SGEMM_E_CONFIG, "unsupported mfma atom [%d, %d, %d, %d]", mf[0], mf[1], mf[2], mf[3]);
    // bounds far beyond any real kernel (a work-group holds at most 16 waves,
    // a tile edge at most a few hundred rows), so that the geometry below
    // cannot overflow
    for (int i = 0; i < 2; ++i) {
        if (info->wave_group[i] <= 0 || info->wave_tiling[i] <= 0)
            return fail(SGEMM_E_CONFIG, "wave_group and wave_tiling must be positive");
        if (info->wave_group[i] > 16 || info->wave_tiling[i] > 64)
            return fail(SGEMM_E_CONFIG, "wave_group [%d, %d] / wave_tiling [%d, %d] outside 1..16 / 1..64",
                        info->wave_group[0], info->wave_group[1], info->wave_tiling[0], info->wave_tiling[1]);
    }
    if (info->depth_k <= 0 || info->depth_k > 4096) return fail(SGEMM_E_CONFIG, "depth_k must be in 1..4096");
    if (info->vmem_stage < 1 || info->vmem_stage > 16) return fail(SGEMM_E_CONFIG, "vmem_stage must be in 1..16");
    if (info->lds_usage_bytes < 0) return fail(SGEMM_E_CONFIG, "lds_usage_bytes must not be negative");
    info->tile_m = mf[0] * info->wave_group[0] * info->wave_tiling[0];
    info->tile_n = mf[1] * info->wave_group[1] * info->wave_tiling[1];
    info->workitems = info->wave_group[0] * info->wave_group[1] * info->wavefront_size;
    if (info->workitems > 1024) return fail(SGEMM_E_CONFIG, "work-group of %d work-items exceeds 1024", info->workitems);
    return SGEMM_OK;
}

// ------------------------------------------------------------- kernargs ---
// Byte image of generated_gemm's explicit arguments (generator.py:2604-2620,
// generator_runner.cpp:132-148): 76 bytes, padded to 80.
struct KernArgs {
    const float* a;
    const float* b;
    const float* c;
    float* d;
    uint32_t m, n, k, lda, ldb, ldc, ldd;
    float alpha, beta;
    int32_t num_wg_x, num_wg_y;
    uint32_t pad;
};
static_assert(sizeof(KernArgs) == 80, "kernarg image must be 80 bytes");
static_assert(offsetof(KernArgs, m) == 32 && offsetof(KernArgs, ldd) == 56, "kernarg offsets");
static_assert(offsetof(KernArgs, alpha) == 60 && offsetof(KernArgs, beta) == 64, "kernarg offsets");
static_assert(offsetof(KernArgs, num_wg_x) == 68 && offsetof(KernArgs, num_wg_y) == 72, "kernarg offsets");

// generated_gemm_splitk: the same 15 arguments, then its workspace, the
// per-tile tickets and the split count: 100 bytes, padded to 104.
struct KernArgsSplit {
    KernArgs base;
    float* ws;
    uint32_t* tickets;
    uint32_t splits;
    uint32_t pad;
};
static_assert(sizeof(KernArgsSplit) == 104, "split kernarg image must be 104 bytes");
static_assert(offsetof(KernArgsSplit, ws) == 80 && offsetof(KernArgsSplit, tickets) == 88 &&
              offsetof(KernArgsSplit, splits) == 96, "split kernarg offsets");

// K ranges a launch really uses: the configured count (or, for 0, the
// per-problem choice documented at sgemm_set_split_k), at most one per K tile.
uint32_t effective_splits(const sgemm_kernel_info& i, int compute_units, uint32_t m, uint32_t n, uint32_t k) {
    const uint64_t ktiles = ((uint64_t)k + (uint32_t)i.depth_k - 1) / (uint32_t)i.depth_k;
    uint64_t s = (uint32_t)i.split_k;
    if (s == 0) {
        // Work-groups run in rounds of one per compute unit; a work-group
        // with a range of ceil(K tiles / s) K tiles costs that many K tiles
        // plus kSplitRangeOverhead (pipeline fill, partial store, fix-up), so
        // the time ~ rounds(T * s) * (ceil(K tiles / s) + overhead).  Pick the
        // s with the least (the smallest s among ties), keeping at least 4 K
        // tiles per range.
        constexpr uint64_t kSplitRangeOverhead = 4;
        const uint64_t tiles = (((uint64_t)m + (uint32_t)i.tile_m - 1) / (uint32_t)i.tile_m) *
                               (((uint64_t)n + (uint32_t)i.tile_n - 1) / (uint32_t)i.tile_n);
        const uint64_t cus = compute_units > 0 ? (uint64_t)compute_units : 1;
        s = 1;
        if (tiles > 0 && tiles < cus) {
            uint64_t smax = (uint64_t)i.split_k_max;
            if (smax > ktiles / 4) smax = ktiles / 4;
            uint64_t best = (uint64_t)ktiles + kSplitRangeOverhead;  // s = 1: one round
            for (uint64_t c = 2; c <= smax; ++c) {
                const uint64_t cost = (tiles * c + cus - 1) / cus * ((ktiles + c - 1) / c + kSplitRangeOverhead);
                if (cost < best) {
                    s = c;
                    best = cost;
                }
            }
        }
    }
    if (s > ktiles) s = ktiles;
    return s < 1 ? 1 : (uint32_t)s;
}

// Tiles of the stream-K phase of an unsplit launch (0: no stream-K).  With
// T tiles and G resident work-groups of generated_gemm_streamk, stream-K runs
// when T > G and the data-parallel grid would leave a partial last round that
// costs at least 3% (ceil(T / G) rounds against T / G) within the instance's
// stream_k_rounds (0: any number of rounds), or always when the setting is 2
// and T > G.  The stream-K phase then takes the last partial
// round plus one whole round, T % G + G tiles (G when T % G == 0), so every
// work-group covers at least one tile's worth of K iterations; the kernel's
// 32-bit iteration arithmetic needs those tiles' K tiles times G below 2^32.
uint32_t stream_k_tiles(const sgemm_kernel_info& i, size_t tiles, uint32_t k) {
    if (i.stream_k == 0 || i.stream_k_groups <= 0 || k == 0) return 0;
    const uint64_t g = (uint64_t)i.stream_k_groups, t = tiles;
    if (t <= g) return 0;
    const uint64_t rem = t % g;
    if (i.stream_k == 1) {
        const uint64_t rounds = (t + g - 1) / g;
        if (rem == 0 || rounds * g * 100 < t * 103) return 0;
        if (i.stream_k_rounds > 0 && rounds > (uint64_t)i.stream_k_rounds) return 0;
    }
    const uint64_t sk = rem ? rem + g : g;
    // the kernel's iteration arithmetic is 32-bit
    const uint64_t kt = ((uint64_t)k + (uint32_t)i.depth_k - 1) / (uint32_t)i.depth_k;
    if (sk * kt * g >= (1ull << 32)) return 0;
    return (uint32_t)sk;
}

// ------------------------------------------------------- seeded values ---
const uint64_t kGamma = 0x9E3779B97F4A7C15ull;

inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

inline uint64_t stream_key(uint64_t seed, uint32_t matrix_id) {
    return mix64(seed ^ (0xD1B54A32D192ED03ull * (uint64_t)(matrix_id + 1)));
}

// i-th output (from 0) of SplitMix64 started at `key`
inline uint64_t word_at(uint64_t key, uint64_t i) { return mix64(key + (i + 1) * kGamma); }

inline float uniform_pm1(uint64_t w) {
    const float u = (float)(w >> 40) * 5.9604644775390625e-08f;  // 24 bits * 2^-24, exact
    return u * 2.0f - 1.0f;                                      // exact
}

inline float normal_at(uint64_t key, uint64_t i) {
    const uint64_t p = i >> 1;
    const double u1 = (double)((word_at(key, 2 * p) >> 11) + 1) * 1.1102230246251565e-16;  // (0, 1]
    const double u2 = (double)(word_at(key, 2 * p + 1) >> 11) * 1.1102230246251565e-16;    // [0, 1)
    const double r = std::sqrt(-2.0 * std::log(u1));
    const double th = 6.283185307179586 * u2;
    return (float)((i & 1) ? r * std::sin(th) : r * std::cos(th));
}

}  // namespace

struct sgemm_handle {
    hipModule_t module = nullptr;
    hipFunction_t function = nullptr;
    hipStream_t stream = nullptr;
    hipEvent_t ev_start = nullptr;
    hipEvent_t ev_stop = nullptr;
    sgemm_kernel_info info{};
    hipFunction_t function_splitk = nullptr;  // null when the code object has none
    void* ws = nullptr;                       // split partials, grown on demand
    size_t ws_bytes = 0;
    uint32_t* tickets = nullptr;              // one per output tile, zero between launches
    size_t ticket_count = 0;
    int compute_units = 0;                    // of the device the module is loaded on
    int device = 0;                           // the device current at sgemm_open
    hipFunction_t function_streamk = nullptr; // null when the code object has none
    sgemm_handle* edge_rows = nullptr;        // kernels for thin edge strips (sgemm_set_edge_kernels): the
    sgemm_handle* edge_cols = nullptr;        // strip of rows past the last tile row, of columns past the last
    int resident = 0;                         // work-groups of generated_gemm the device holds at once (0: unknown)
    hipStream_t own_stream = nullptr;         // created at sgemm_open; `stream` is it unless sgemm_set_stream
    std::vector<sgemm_handle*> edge_of;       // handles this one serves as an edge kernel (under g_edge_mutex)
};

namespace {

// Guards edge_rows / edge_cols / edge_of links between handles, which
// sgemm_set_edge_kernels and sgemm_close of different handles update.
std::mutex g_edge_mutex;

void unlink_edge(sgemm_handle* edge, sgemm_handle* main) {
    if (!edge) return;
    auto& v = edge->edge_of;
    for (size_t i = 0; i < v.size(); ++i)
        if (v[i] == main) {
            v.erase(v.begin() + (long)i);
            return;  // one entry per attachment: rows and cols each add one
        }
}

}  // namespace

namespace {

// Bytes [lo, hi) a column-major rows x cols matrix with leading dimension ld
// occupies from p (empty for a null pointer or an empty matrix).
struct Span {
    uintptr_t lo = 0, hi = 0;
    bool overlaps(const Span& o) const { return lo < hi && o.lo < o.hi && lo < o.hi && o.lo < hi; }
};

Span span_of(const float* p, uint32_t rows, uint32_t cols, uint32_t ld) {
    Span s;
    if (!p || !rows || !cols) return s;
    s.lo = (uintptr_t)p;
    s.hi = s.lo + (((uintptr_t)(cols - 1) * ld + rows) * sizeof(float));
    return s;
}

}  // namespace

namespace sgemm_internal {

Plan plan(const sgemm_handle* h, uint32_t m, uint32_t n, uint32_t k) {
    const sgemm_kernel_info& i = h->info;
    Plan p;
    p.tiles = (size_t)((((uint64_t)m + (uint32_t)i.tile_m - 1) / (uint32_t)i.tile_m) *
                       (((uint64_t)n + (uint32_t)i.tile_n - 1) / (uint32_t)i.tile_n));
    const size_t tile_bytes = (size_t)i.tile_m * (size_t)i.tile_n * 4;
    p.splits = effective_splits(i, h->compute_units, m, n, k);
    if (p.splits > 1) {
        // saturates for shapes no device could hold (any allocation then fails)
        size_t bytes = 0;
        if (__builtin_mul_overflow(p.tiles, (size_t)p.splits, &bytes) ||
            __builtin_mul_overflow(bytes, tile_bytes, &bytes))
            bytes = SIZE_MAX;
        p.partial_bytes = bytes;
        p.ticket_count = p.tiles;
        return p;
    }
    p.sk_tiles = stream_k_tiles(i, p.tiles, k);
    if (p.sk_tiles) {
        p.sk_groups = (uint32_t)i.stream_k_groups;
        p.partial_bytes = (size_t)p.sk_groups * 2 * tile_bytes;
        p.ticket_count = p.sk_groups;
    }
    return p;
}

int launch(sgemm_handle* h, const float* dA, const float* dB, const float* dC, float* dD, uint32_t m, uint32_t n,
           uint32_t k, uint32_t lda, uint32_t ldb, uint32_t ldc, uint32_t ldd, float alpha, float beta,
           const Workspace* ws, hipStream_t stream) {
    const sgemm_kernel_info& i = h->info;
    KernArgs ka;
    memset(&ka, 0, sizeof(ka));
    ka.a = dA; ka.b = dB; ka.c = dC; ka.d = dD;
    ka.m = m; ka.n = n; ka.k = k; ka.lda = lda; ka.ldb = ldb; ka.ldc = ldc; ka.ldd = ldd;
    ka.alpha = alpha; ka.beta = beta;
    ka.num_wg_x = (int32_t)((m + (uint32_t)i.tile_m - 1) / (uint32_t)i.tile_m);
    ka.num_wg_y = (int32_t)((n + (uint32_t)i.tile_n - 1) / (uint32_t)i.tile_n);
    const Plan p = plan(h, m, n, k);
    if (p.splits == 1 && !p.sk_tiles) {
        size_t size = sizeof(ka);
        void* extra[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, &ka, HIP_LAUNCH_PARAM_BUFFER_SIZE, &size, HIP_LAUNCH_PARAM_END};
        HIP_TRY(hipModuleLaunchKernel(h->function, (unsigned)ka.num_wg_x, (unsigned)ka.num_wg_y, 1,
                                      (unsigned)i.workitems, 1, 1, 0, stream, nullptr, extra));
        return SGEMM_OK;
    }
    if (!ws || !ws->partials || !ws->tickets || ws->partial_bytes < p.partial_bytes || ws->ticket_count < p.ticket_count)
        return fail(SGEMM_E_INVALID, "launch needs %zu bytes of partials and %zu tickets", p.partial_bytes,
                    p.ticket_count);
    KernArgsSplit ks;
    memset(&ks, 0, sizeof(ks));
    ks.base = ka;
    ks.ws = ws->partials;
    ks.tickets = ws->tickets;
    size_t size = sizeof(ks);
    void* extra[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, &ks, HIP_LAUNCH_PARAM_BUFFER_SIZE, &size, HIP_LAUNCH_PARAM_END};
    if (p.splits > 1) {
        ks.splits = p.splits;
        HIP_TRY(hipModuleLaunchKernel(h->function_splitk, (unsigned)ka.num_wg_x, (unsigned)ka.num_wg_y, p.splits,
                                      (unsigned)i.workitems, 1, 1, 0, stream, nullptr, extra));
        return SGEMM_OK;
    }
    ks.splits = p.sk_tiles;      // generated_gemm_streamk: sk_tiles at 96, groups at 100
    ks.pad = p.sk_groups;
    HIP_TRY(hipModuleLaunchKernel(h->function_streamk, p.sk_groups, 1, 1, (unsigned)i.workitems, 1, 1, 0, stream,
                                  nullptr, extra));
    return SGEMM_OK;
}

int check_launch(const sgemm_handle* h, const float* dA, const float* dB, const float* dC, float* dD, uint32_t m,
                 uint32_t n, uint32_t k, uint32_t lda, uint32_t ldb, uint32_t ldc, uint32_t ldd, float beta) {
    int r = sgemm_check_shape(h, m, n, k, lda, ldb, ldc, ldd);
    if (r != SGEMM_OK) return r;
    if (m == 0 || n == 0) return SGEMM_OK;
    if (!dD || (k && (!dA || !dB)) || (beta != 0.0f && !dC))
        return fail(SGEMM_E_INVALID, "sgemm_launch: null device pointer");
    // buffer loads and stores need dword alignment only
    if (((uintptr_t)dA | (uintptr_t)dB | (uintptr_t)dC | (uintptr_t)dD) & 3u)
        return fail(SGEMM_E_INVALID, "sgemm_launch: device pointers must be 4-byte aligned");
    // Tiles store D while other tiles still read A, B and C: D may share no
    // byte with A or B, and may share bytes with C only as the very same
    // matrix (dC == dD, ldc == ldd: every tile reads its C block before it
    // writes the same D block, and no other tile touches that block).
    const uint32_t a_rows = h->info.trans_a ? k : m, a_cols = h->info.trans_a ? m : k;
    const uint32_t b_rows = h->info.trans_b ? n : k, b_cols = h->info.trans_b ? k : n;
    const Span d_span = span_of(dD, m, n, ldd);
    if (k && (d_span.overlaps(span_of(dA, a_rows, a_cols, lda)) || d_span.overlaps(span_of(dB, b_rows, b_cols, ldb))))
        return fail(SGEMM_E_INVALID, "sgemm_launch: D overlaps A or B");
    if (beta != 0.0f && d_span.overlaps(span_of(dC, m, n, ldc)) && !(dC == dD && ldc == ldd))
        return fail(SGEMM_E_INVALID, "sgemm_launch: C and D overlap without being the same matrix (dC == dD and "
                    "ldc == ldd)");
    return SGEMM_OK;
}

int decompose(const sgemm_handle* h, uint32_t m, uint32_t n, uint32_t k, uint32_t lda, uint32_t ldb, uint32_t ldc,
              uint32_t ldd, Part out[3]) {
    const sgemm_kernel_info& i = h->info;
    out[0] = Part{const_cast<sgemm_handle*>(h), m, n, 0, 0, 0, 0};
    if (k == 0) return 1;
    const uint32_t tm = (uint32_t)i.tile_m, tn = (uint32_t)i.tile_n;
    uint32_t me = m % tm, ne = n % tn;
    // thin strips only: at most a quarter of a tile, next to a non-empty
    // interior, and only with a kernel attached for that strip
    if (!(h->edge_rows && me && me * 4 <= tm && m > me)) me = 0;
    if (!(h->edge_cols && ne && ne * 4 <= tn && n > ne)) ne = 0;
    if ((!me && !ne) || h->resident <= 0) return 1;
    // and only where they save h a round of work-groups: a strip costs a
    // launch of its own (a memory-bound pass over A or B), the tiles it
    // replaces cost nothing while they fit in a round the interior needs anyway
    const uint64_t res = (uint64_t)h->resident;
    auto rounds = [&](uint32_t rm, uint32_t rn) {
        return ((((uint64_t)rm + tm - 1) / tm) * (((uint64_t)rn + tn - 1) / tn) + res - 1) / res;
    };
    const uint64_t both = rounds(m - me, n - ne);
    if (rounds(m, n) <= both) return 1;
    if (me && ne) {  // the fewest strips that reach the same rounds
        if (rounds(m - me, n) <= both)
            ne = 0;
        else if (rounds(m, n - ne) <= both)
            me = 0;
    }
    const uint32_t mi = m - me, ni = n - ne;
    int count = 0;
    out[count++] = Part{const_cast<sgemm_handle*>(h), mi, ni, 0, 0, 0, 0};
    if (me)  // rows [mi, m) of every column
        out[count++] = Part{h->edge_rows, me, n, i.trans_a ? (size_t)mi * lda : (size_t)mi, 0, (size_t)mi,
                            (size_t)mi};
    if (ne)  // columns [ni, n) of rows [0, mi)
        out[count++] = Part{h->edge_cols, mi, ne, 0, i.trans_b ? (size_t)ni : (size_t)ni * ldb, (size_t)ni * ldc,
                            (size_t)ni * ldd};
    return count;
}


hipStream_t stream(const sgemm_handle* h) { return h->stream; }

int device(const sgemm_handle* h) { return h->device; }

int set_error(int code, const char* message) { return fail(code, "%s", message); }

}  // namespace sgemm_internal

extern "C" {

const char* sgemm_last_error(void) { return g_last_error.c_str(); }

int sgemm_abi_version(void) { return SGEMM_SHIM_ABI_VERSION; }

int sgemm_device_info(char* name, size_t name_len, int* compute_units, int* clock_khz, int* lds_per_block) {
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count == 0) return fail(SGEMM_E_NO_DEVICE, "no HIP device visible (%s)", hipGetErrorString(e));
    hipDeviceProp_t p;
    HIP_TRY(hipGetDeviceProperties(&p, 0));
    if (name && name_len) {
        // some drivers report an empty marketing name: fall back to the ISA name alone
        if (p.name[0]) snprintf(name, name_len, "%s (%s)", p.name, p.gcnArchName);
        else snprintf(name, name_len, "%s, %d CUs", p.gcnArchName, p.multiProcessorCount);
    }
    if (compute_units) *compute_units = p.multiProcessorCount;
    if (clock_khz) *clock_khz = p.clockRate;
    if (lds_per_block) *lds_per_block = (int)p.sharedMemPerBlock;
    return SGEMM_OK;
}

int sgemm_open(const char* co_path, const char* toml_path, sgemm_handle** out) {
    if (!co_path || !toml_path || !out) return fail(SGEMM_E_INVALID, "sgemm_open: null argument");
    *out = nullptr;
    sgemm_kernel_info info{};
    int r = load_config(toml_path, &info);
    if (r != SGEMM_OK) return r;
    {
        std::ifstream f(co_path, std::ios::binary);
        if (!f) return fail(SGEMM_E_IO, "cannot open code object %s", co_path);
    }
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count == 0) return fail(SGEMM_E_NO_DEVICE, "no HIP device visible (%s)", hipGetErrorString(e));
    sgemm_handle* h = new sgemm_handle();
    h->info = info;
    hipError_t err = hipModuleLoad(&h->module, co_path);
    if (err != hipSuccess) {
        delete h;
        return hip_fail(err, "hipModuleLoad");
    }
    err = hipModuleGetFunction(&h->function, h->module, "generated_gemm");
    if (err == hipSuccess) {
        // optional second kernel; its absence only limits split_k to 1
        if (hipModuleGetFunction(&h->function_splitk, h->module, "generated_gemm_splitk") != hipSuccess) {
            h->function_splitk = nullptr;
            (void)hipGetLastError();
        }
        h->info.split_k_max = h->function_splitk ? SGEMM_MAX_SPLIT_K : 1;
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&h->compute_units, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
            h->compute_units = 0;
            (void)hipGetLastError();
        }
        h->device = dev;
        // optional stream-K kernel: G = resident work-groups per CU x CUs
        int per_cu_main = 0;
        if (hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu_main, h->function, h->info.workitems, 0) ==
                hipSuccess && per_cu_main > 0 && h->compute_units > 0) {
            h->resident = per_cu_main * h->compute_units;
        } else {
            (void)hipGetLastError();
        }
        h->info.stream_k_groups = 0;
        if (hipModuleGetFunction(&h->function_streamk, h->module, "generated_gemm_streamk") == hipSuccess) {
            int per_cu = 0;
            if (hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, h->function_streamk, h->info.workitems, 0) ==
                    hipSuccess && per_cu > 0 && h->compute_units > 0) {
                h->info.stream_k_groups = per_cu * h->compute_units;
            } else {
                (void)hipGetLastError();
            }
        } else {
            h->function_streamk = nullptr;
            (void)hipGetLastError();
        }
        if (!h->info.stream_k_groups) h->info.stream_k = 0;
        // the static scratch of sgemm_launch_noalloc on this device: looked
        // up here, so that no launch (maybe under graph capture) does it
        const int sr = sgemm_internal::noalloc_prepare(dev);
        if (sr != SGEMM_OK) {
            sgemm_close(h);
            return sr;
        }
        if (h->info.split_k > h->info.split_k_max) {
            sgemm_close(h);
            return fail(SGEMM_E_CONFIG, "split_k = %d but %s has no generated_gemm_splitk", info.split_k, co_path);
        }
    }
    if (err == hipSuccess) err = hipStreamCreate(&h->own_stream);
    h->stream = h->own_stream;
    if (err == hipSuccess) err = hipEventCreate(&h->ev_start);
    if (err == hipSuccess) err = hipEventCreate(&h->ev_stop);
    if (err != hipSuccess) {
        sgemm_close(h);
        return hip_fail(err, "sgemm_open");
    }
    *out = h;
    return SGEMM_OK;
}

void sgemm_close(sgemm_handle* h) {
    if (!h) return;
    {
        // detach h from every handle it serves as an edge kernel (those fall
        // back to running their whole problem themselves), and from its own
        // edge kernels' lists
        std::lock_guard<std::mutex> lock(g_edge_mutex);
        for (sgemm_handle* main : h->edge_of) {
            if (main->edge_rows == h) main->edge_rows = nullptr;
            if (main->edge_cols == h) main->edge_cols = nullptr;
        }
        h->edge_of.clear();
        unlink_edge(h->edge_rows, h);
        unlink_edge(h->edge_cols, h);
        h->edge_rows = h->edge_cols = nullptr;
    }
    if (h->stream) (void)hipStreamSynchronize(h->stream);
    if (h->own_stream && h->own_stream != h->stream) (void)hipStreamSynchronize(h->own_stream);
    if (h->ev_start) (void)hipEventDestroy(h->ev_start);
    if (h->ev_stop) (void)hipEventDestroy(h->ev_stop);
    if (h->own_stream) (void)hipStreamDestroy(h->own_stream);
    if (h->ws) (void)hipFree(h->ws);
    if (h->tickets) (void)hipFree(h->tickets);
    if (h->module) (void)hipModuleUnload(h->module);
    delete h;
}

int sgemm_get_info(const sgemm_handle* h, sgemm_kernel_info* info) {
    if (!h || !info) return fail(SGEMM_E_INVALID, "sgemm_get_info: null argument");
    *info = h->info;
    return SGEMM_OK;
}

int sgemm_check_shape(const sgemm_handle* h, uint32_t m, uint32_t n, uint32_t k,
                      uint32_t lda, uint32_t ldb, uint32_t ldc, uint32_t ldd) {
    if (!h) return fail(SGEMM_E_INVALID, "sgemm_check_shape: null handle");
    const sgemm_kernel_info& i = h->info;
    // Any m, n, k: the kernel masks edge tiles and a K remainder.  Leading
    // dimensions must cover the stored matrices: A is m x k (k x m when
    // transposed), B is k x n (n x k when transposed), C and D are m x n.
    const uint32_t a_rows = i.trans_a ? k : m, b_rows = i.trans_b ? n : k;
    if (lda < a_rows || ldb < b_rows || ldc < m || ldd < m || lda == 0 || ldb == 0 || ldc == 0 || ldd == 0)
        return fail(SGEMM_E_SHAPE, "leading dimensions too small: lda=%u (needs %u) ldb=%u (needs %u) ldc=%u ldd=%u (m=%u)",
                    lda, a_rows, ldb, b_rows, ldc, ldd, m);
    const uint64_t wgx = ((uint64_t)m + (uint32_t)i.tile_m - 1) / (uint32_t)i.tile_m;
    const uint64_t wgy = ((uint64_t)n + (uint32_t)i.tile_n - 1) / (uint32_t)i.tile_n;
    if (wgx > 0x7fffffffull || wgy > 65535ull || wgx * wgy > 0x7fffffffull)
        return fail(SGEMM_E_SHAPE, "grid %llux%llu too large", (unsigned long long)wgx, (unsigned long long)wgy);
    // row, column and k indices inside the kernel are 32-bit signed: the tile
    // grid padded to whole tiles, and k plus one K tile, stay below 2^31
    if (wgx * (uint32_t)i.tile_m > 0x7fffffffull || wgy * (uint32_t)i.tile_n > 0x7fffffffull ||
        (uint64_t)k + (uint32_t)i.depth_k > 0x7fffffffull)
        return fail(SGEMM_E_SHAPE, "m=%u n=%u k=%u: padded to whole tiles they must stay below 2^31", m, n, k);
    // the kernel addresses one K tile of each operand through a buffer
    // descriptor with 32-bit byte offsets: lda * depth_k (tile_m for A^T) and
    // ldb * tile_n (depth_k for B^T) floats must stay below 2^31 bytes
    const uint64_t a_span = (uint64_t)lda * (uint32_t)(i.trans_a ? i.tile_m : i.depth_k) * 4u;
    const uint64_t b_span = (uint64_t)ldb * (uint32_t)(i.trans_b ? i.depth_k : i.tile_n) * 4u;
    if (a_span >= (1ull << 31) || b_span >= (1ull << 31))
        return fail(SGEMM_E_SHAPE, "leading dimensions too large for 32-bit tile offsets (a K tile spans %llu / %llu "
                    "bytes of A / B, limit 2^31): lda=%u ldb=%u", (unsigned long long)a_span,
                    (unsigned long long)b_span, lda, ldb);
    // and one tile of C and of D the same way: ldc * tile_n and ldd * tile_n
    // floats below 2^31 bytes
    const uint64_t cd_span = (uint64_t)(ldc > ldd ? ldc : ldd) * (uint32_t)i.tile_n * 4u;
    if (cd_span >= (1ull << 31))
        return fail(SGEMM_E_SHAPE, "leading dimensions too large for 32-bit tile offsets (a tile of C / D spans %llu "
                    "bytes, limit 2^31): ldc=%u ldd=%u", (unsigned long long)cd_span, ldc, ldd);
    return SGEMM_OK;
}

int sgemm_set_split_k(sgemm_handle* h, int splits) {
    if (!h) return fail(SGEMM_E_INVALID, "sgemm_set_split_k: null handle");
    if (splits < 0 || splits > SGEMM_MAX_SPLIT_K)
        return fail(SGEMM_E_INVALID, "split count %d outside 0..%d", splits, SGEMM_MAX_SPLIT_K);
    if (splits > h->info.split_k_max)
        return fail(SGEMM_E_CONFIG, "split count %d needs generated_gemm_splitk, absent from this code object", splits);
    h->info.split_k = splits;
    return SGEMM_OK;
}

namespace {

// m x n of h's own part of an m x n x k launch: the interior when edge
// kernels take strips, else the whole problem.
void own_part(const sgemm_handle* h, uint32_t m, uint32_t n, uint32_t k, uint32_t* pm, uint32_t* pn) {
    sgemm_internal::Part parts[3];
    sgemm_internal::decompose(h, m, n, k, m, k, m, m, parts);
    *pm = parts[0].m;
    *pn = parts[0].n;
}

}  // namespace

int sgemm_workspace_size(const sgemm_handle* h, uint32_t m, uint32_t n, uint32_t k, size_t* bytes) {
    if (!h || !bytes) return fail(SGEMM_E_INVALID, "sgemm_workspace_size: null argument");
    *bytes = 0;
    if (m && n) {
        own_part(h, m, n, k, &m, &n);
        const sgemm_internal::Plan p = sgemm_internal::plan(h, m, n, k);
        size_t total = 0;
        if (p.partial_bytes && (__builtin_mul_overflow(p.ticket_count, (size_t)4, &total) ||
                                __builtin_add_overflow(total, p.partial_bytes, &total)))
            total = SIZE_MAX;
        *bytes = p.partial_bytes ? total : 0;
    }
    return SGEMM_OK;
}

int sgemm_set_stream_k(sgemm_handle* h, int mode) {
    if (!h) return fail(SGEMM_E_INVALID, "sgemm_set_stream_k: null handle");
    if (mode < 0 || mode > 2) return fail(SGEMM_E_INVALID, "stream-K mode %d outside 0..2", mode);
    if (mode && !h->info.stream_k_groups)
        return fail(SGEMM_E_CONFIG, "stream-K needs generated_gemm_streamk, absent from this code object");
    h->info.stream_k = mode;
    return SGEMM_OK;
}

int sgemm_stream_k_tiles(const sgemm_handle* h, uint32_t m, uint32_t n, uint32_t k, int* sk_tiles) {
    if (!h || !sk_tiles) return fail(SGEMM_E_INVALID, "sgemm_stream_k_tiles: null argument");
    *sk_tiles = 0;
    if (m && n) {
        own_part(h, m, n, k, &m, &n);
        *sk_tiles = (int)sgemm_internal::plan(h, m, n, k).sk_tiles;
    }
    return SGEMM_OK;
}

int sgemm_launch_splits(const sgemm_handle* h, uint32_t m, uint32_t n, uint32_t k, int* splits) {
    if (!h || !splits) return fail(SGEMM_E_INVALID, "sgemm_launch_splits: null argument");
    if (m && n) own_part(h, m, n, k, &m, &n);
    *splits = (int)effective_splits(h->info, h->compute_units, m, n, k);
    return SGEMM_OK;
}

int sgemm_malloc(void** dptr, size_t bytes) {
    if (!dptr) return fail(SGEMM_E_INVALID, "sgemm_malloc: null argument");
    *dptr = nullptr;
    HIP_TRY(hipMalloc(dptr, bytes ? bytes : 1));
    return SGEMM_OK;
}

int sgemm_free(void* dptr) {
    if (dptr) HIP_TRY(hipFree(dptr));
    return SGEMM_OK;
}

int sgemm_memcpy_h2d(void* dst, const void* src, size_t bytes) {
    if (bytes && (!dst || !src)) return fail(SGEMM_E_INVALID, "sgemm_memcpy_h2d: null argument");
    if (bytes) HIP_TRY(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
    return SGEMM_OK;
}

int sgemm_memcpy_d2h(void* dst, const void* src, size_t bytes) {
    if (bytes && (!dst || !src)) return fail(SGEMM_E_INVALID, "sgemm_memcpy_d2h: null argument");
    if (bytes) HIP_TRY(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
    return SGEMM_OK;
}

int sgemm_memset(void* dptr, int value, size_t bytes) {
    if (bytes && !dptr) return fail(SGEMM_E_INVALID, "sgemm_memset: null argument");
    if (bytes) HIP_TRY(hipMemset(dptr, value, bytes));
    return SGEMM_OK;
}

namespace {

// One part of a launch on `stream` with kernel handle `kh`: its split-K /
// stream-K workspace is kh's own, grown on demand (both streams drained
// first, fresh tickets zeroed on `stream`).
int launch_part(sgemm_handle* kh, hipStream_t stream, const float* dA, const float* dB, const float* dC, float* dD,
                uint32_t m, uint32_t n, uint32_t k, uint32_t lda, uint32_t ldb, uint32_t ldc, uint32_t ldd, float alpha,
                float beta) {
    const sgemm_internal::Plan p = sgemm_internal::plan(kh, m, n, k);
    if (!p.partial_bytes)
        return sgemm_internal::launch(kh, dA, dB, dC, dD, m, n, k, lda, ldb, ldc, ldd, alpha, beta, nullptr, stream);
    const size_t ws_need = p.partial_bytes, tickets = p.ticket_count;
    if (kh->ws_bytes < ws_need || kh->ticket_count < tickets) {
        HIP_TRY(hipStreamSynchronize(stream));
        HIP_TRY(hipStreamSynchronize(kh->stream));
        if (kh->ws_bytes < ws_need) {
            if (kh->ws) HIP_TRY(hipFree(kh->ws));
            kh->ws = nullptr;
            kh->ws_bytes = 0;
            HIP_TRY(hipMalloc(&kh->ws, ws_need));
            kh->ws_bytes = ws_need;
        }
        if (kh->ticket_count < tickets) {
            if (kh->tickets) HIP_TRY(hipFree(kh->tickets));
            kh->tickets = nullptr;
            kh->ticket_count = 0;
            HIP_TRY(hipMalloc((void**)&kh->tickets, tickets * 4));
            // ordered before the launch below on the same stream
            HIP_TRY(hipMemsetAsync(kh->tickets, 0, tickets * 4, stream));
            kh->ticket_count = tickets;
        }
    }
    const sgemm_internal::Workspace ws{(float*)kh->ws, kh->ws_bytes, kh->tickets, kh->ticket_count};
    return sgemm_internal::launch(kh, dA, dB, dC, dD, m, n, k, lda, ldb, ldc, ldd, alpha, beta, &ws, stream);
}

}  // namespace

int sgemm_launch(sgemm_handle* h, const float* dA, const float* dB, const float* dC, float* dD,
                 uint32_t m, uint32_t n, uint32_t k, uint32_t lda, uint32_t ldb, uint32_t ldc, uint32_t ldd,
                 float alpha, float beta) {
    if (!h) return fail(SGEMM_E_INVALID, "sgemm_launch: null handle");
    int r = sgemm_internal::check_launch(h, dA, dB, dC, dD, m, n, k, lda, ldb, ldc, ldd, beta);
    if (r != SGEMM_OK || m == 0 || n == 0) return r;
    sgemm_internal::Part parts[3];
    const int count = sgemm_internal::decompose(h, m, n, k, lda, ldb, ldc, ldd, parts);
    for (int q = 0; q < count; ++q) {
        const sgemm_internal::Part& pt = parts[q];
        if (pt.kh != h && (r = sgemm_check_shape(pt.kh, pt.m, pt.n, k, lda, ldb, ldc, ldd)) != SGEMM_OK) return r;
    }
    for (int q = 0; q < count; ++q) {
        const sgemm_internal::Part& pt = parts[q];
        r = launch_part(pt.kh, h->stream, dA ? dA + pt.a_off : dA, dB ? dB + pt.b_off : dB, dC ? dC + pt.c_off : dC,
                        dD + pt.d_off, pt.m, pt.n, k, lda, ldb, ldc, ldd, alpha, beta);
        if (r != SGEMM_OK) return r;
    }
    return SGEMM_OK;
}

namespace {

int check_edge(const sgemm_handle* h, const sgemm_handle* e, bool rows) {
    if (!e) return SGEMM_OK;
    if (e == h || e->edge_rows || e->edge_cols)
        return fail(SGEMM_E_INVALID, "an edge kernel must be another handle without edge kernels");
    if (e->info.trans_a != h->info.trans_a || e->info.trans_b != h->info.trans_b)
        return fail(SGEMM_E_CONFIG, "the edge kernel's layout (trans_a/trans_b) differs from the main kernel's");
    // a strip is at most a quarter of the main tile across, so an edge tile
    // as wide across it as the main tile's can only be a mistaken handle
    if (rows ? e->info.tile_m >= h->info.tile_m : e->info.tile_n >= h->info.tile_n)
        return fail(SGEMM_E_CONFIG, "the %s edge kernel's tile %dx%d is not narrower across the strip than the main "
                    "kernel's %dx%d", rows ? "row" : "column", e->info.tile_m, e->info.tile_n, h->info.tile_m,
                    h->info.tile_n);
    if (e->device != h->device) return fail(SGEMM_E_CONFIG, "the edge kernel is loaded on another device");
    return SGEMM_OK;
}

}  // namespace

int sgemm_set_edge_kernels(sgemm_handle* h, sgemm_handle* rows, sgemm_handle* cols) {
    if (!h) return fail(SGEMM_E_INVALID, "sgemm_set_edge_kernels: null handle");
    std::lock_guard<std::mutex> lock(g_edge_mutex);
    int r = check_edge(h, rows, true);
    if (r == SGEMM_OK) r = check_edge(h, cols, false);
    if (r != SGEMM_OK) return r;
    if (!h->edge_of.empty())
        return fail(SGEMM_E_INVALID, "sgemm_set_edge_kernels: this handle is itself attached as an edge kernel");
    unlink_edge(h->edge_rows, h);
    unlink_edge(h->edge_cols, h);
    h->edge_rows = rows;
    h->edge_cols = cols;
    if (rows) rows->edge_of.push_back(h);
    if (cols) cols->edge_of.push_back(h);
    return SGEMM_OK;
}

int sgemm_set_edge_kernel(sgemm_handle* h, sgemm_handle* edge) { return sgemm_set_edge_kernels(h, edge, edge); }

int sgemm_edge_interior(const sgemm_handle* h, uint32_t m, uint32_t n, uint32_t k, uint32_t* m_int, uint32_t* n_int) {
    if (!h || !m_int || !n_int) return fail(SGEMM_E_INVALID, "sgemm_edge_interior: null argument");
    sgemm_internal::Part parts[3];
    sgemm_internal::decompose(h, m, n, k, m, k, m, m, parts);
    *m_int = parts[0].m;
    *n_int = parts[0].n;
    return SGEMM_OK;
}

int sgemm_time(sgemm_handle* h, const float* dA, const float* dB, const float* dC, float* dD,
               uint32_t m, uint32_t n, uint32_t k, uint32_t lda, uint32_t ldb, uint32_t ldc, uint32_t ldd,
               float alpha, float beta, int warmup, int runs, float* total_ms) {
    if (!h || !total_ms || warmup < 0 || runs <= 0) return fail(SGEMM_E_INVALID, "sgemm_time: bad argument");
    int r;
    for (int w = 0; w < warmup; ++w)
        if ((r = sgemm_launch(h, dA, dB, dC, dD, m, n, k, lda, ldb, ldc, ldd, alpha, beta)) != SGEMM_OK) return r;
    HIP_TRY(hipStreamSynchronize(h->stream));
    HIP_TRY(hipEventRecord(h->ev_start, h->stream));
    for (int t = 0; t < runs; ++t)
        if ((r = sgemm_launch(h, dA, dB, dC, dD, m, n, k, lda, ldb, ldc, ldd, alpha, beta)) != SGEMM_OK) return r;
    HIP_TRY(hipEventRecord(h->ev_stop, h->stream));
    HIP_TRY(hipEventSynchronize(h->ev_stop));
    HIP_TRY(hipEventElapsedTime(total_ms, h->ev_start, h->ev_stop));
    return SGEMM_OK;
}

int sgemm_time_each(sgemm_handle* h, const float* dA, const float* dB, const float* dC, float* dD,
                    uint32_t m, uint32_t n, uint32_t k, uint32_t lda, uint32_t ldb, uint32_t ldc, uint32_t ldd,
                    float alpha, float beta, int runs, float* per_launch_ms) {
    if (!h || !per_launch_ms || runs <= 0) return fail(SGEMM_E_INVALID, "sgemm_time_each: bad argument");
    std::vector<hipEvent_t> ev(2 * (size_t)runs, nullptr);
    int result = SGEMM_OK;
    for (auto& e : ev) {
        hipError_t err = hipEventCreate(&e);
        if (err != hipSuccess) {
            result = hip_fail(err, "hipEventCreate");
            break;
        }
    }
    for (int t = 0; t < runs && result == SGEMM_OK; ++t) {
        hipError_t err = hipEventRecord(ev[2 * t], h->stream);
        if (err != hipSuccess) { result = hip_fail(err, "hipEventRecord"); break; }
        result = sgemm_launch(h, dA, dB, dC, dD, m, n, k, lda, ldb, ldc, ldd, alpha, beta);
        if (result != SGEMM_OK) break;
        err = hipEventRecord(ev[2 * t + 1], h->stream);
        if (err != hipSuccess) { result = hip_fail(err, "hipEventRecord"); break; }
    }
    if (result == SGEMM_OK) {
        hipError_t err = hipStreamSynchronize(h->stream);
        if (err != hipSuccess) result = hip_fail(err, "hipStreamSynchronize");
    }
    for (int t = 0; t < runs && result == SGEMM_OK; ++t) {
        hipError_t err = hipEventElapsedTime(&per_launch_ms[t], ev[2 * t], ev[2 * t + 1]);
        if (err != hipSuccess) result = hip_fail(err, "hipEventElapsedTime");
    }
    (void)hipStreamSynchronize(h->stream);
    for (auto& e : ev)
        if (e) (void)hipEventDestroy(e);
    return result;
}

int sgemm_set_stream(sgemm_handle* h, void* stream) {
    if (!h) return fail(SGEMM_E_INVALID, "sgemm_set_stream: null handle");
    hipStream_t next = stream ? static_cast<hipStream_t>(stream) : h->own_stream;
    if (stream) {
        // the handle's module, workspace and scratch live on its device
        hipDevice_t dev = -1;
        HIP_TRY(hipStreamGetDevice(next, &dev));
        if (dev != h->device)
            return fail(SGEMM_E_INVALID, "sgemm_set_stream: the stream belongs to device %d, the handle to device %d",
                        (int)dev, h->device);
    }
    if (next != h->stream) {
        // work already enqueued through h finishes before h moves on; not
        // under capture (a capturing stream cannot be synchronized)
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        HIP_TRY(hipStreamIsCapturing(h->stream, &cs));
        if (cs != hipStreamCaptureStatusNone)
            return fail(SGEMM_E_INVALID, "sgemm_set_stream: the handle's current stream is capturing");
        HIP_TRY(hipStreamSynchronize(h->stream));
        h->stream = next;
    }
    return SGEMM_OK;
}

int sgemm_synchronize(sgemm_handle* h) {
    if (!h) return fail(SGEMM_E_INVALID, "sgemm_synchronize: null handle");
    HIP_TRY(hipStreamSynchronize(h->stream));
    return SGEMM_OK;
}

int sgemm_run(sgemm_handle* h, const float* A, const float* B, const float* C, float* D,
              uint32_t m, uint32_t n, uint32_t k, float alpha, float beta,
              int warmup, int runs, double* ms_per_run) {
    if (!h || !D || !A || !B || (beta != 0.0f && !C) || runs <= 0 || warmup < 0)
        return fail(SGEMM_E_INVALID, "sgemm_run: bad argument");
    const uint32_t lda = h->info.trans_a ? k : m, ldb = h->info.trans_b ? n : k;
    int r = sgemm_check_shape(h, m, n, k, lda, ldb, m, m);
    if (r != SGEMM_OK) return r;
    const size_t bA = (size_t)m * k * 4, bB = (size_t)k * n * 4, bC = (size_t)m * n * 4;
    void *dA = nullptr, *dB = nullptr, *dC = nullptr, *dD = nullptr;
    float total = 0.0f;
    r = sgemm_malloc(&dA, bA);
    if (r == SGEMM_OK) r = sgemm_malloc(&dB, bB);
    if (r == SGEMM_OK && beta != 0.0f) r = sgemm_malloc(&dC, bC);
    if (r == SGEMM_OK) r = sgemm_malloc(&dD, bC);
    if (r == SGEMM_OK) r = sgemm_memcpy_h2d(dA, A, bA);
    if (r == SGEMM_OK) r = sgemm_memcpy_h2d(dB, B, bB);
    if (r == SGEMM_OK && dC) r = sgemm_memcpy_h2d(dC, C, bC);
    if (r == SGEMM_OK) r = sgemm_memset(dD, 0, bC);
    if (r == SGEMM_OK)
        r = sgemm_time(h, (const float*)dA, (const float*)dB, (const float*)dC, (float*)dD, m, n, k, lda, ldb, m, m,
                       alpha, beta, warmup, runs, &total);
    if (r == SGEMM_OK) r = sgemm_memcpy_d2h(D, dD, bC);
    if (r == SGEMM_OK && ms_per_run) *ms_per_run = (double)total / runs;
    std::string keep = g_last_error;
    sgemm_free(dA);
    sgemm_free(dB);
    sgemm_free(dC);
    sgemm_free(dD);
    g_last_error = keep;
    return r;
}

int sgemm_fill(float* host, size_t count, uint64_t seed, uint32_t matrix_id, int dist) {
    if (count && !host) return fail(SGEMM_E_INVALID, "sgemm_fill: null argument");
    if (dist != SGEMM_DIST_UNIFORM && dist != SGEMM_DIST_NORMAL && dist != SGEMM_DIST_ZERO)
        return fail(SGEMM_E_INVALID, "sgemm_fill: unknown distribution %d", dist);
    const uint64_t key = stream_key(seed, matrix_id);
    auto work = [=](size_t lo, size_t hi) {
        for (size_t i = lo; i < hi; ++i) {
            if (dist == SGEMM_DIST_UNIFORM) host[i] = uniform_pm1(word_at(key, i));
            else if (dist == SGEMM_DIST_NORMAL) host[i] = normal_at(key, i);
            else host[i] = 0.0f;
        }
    };
    unsigned nt = std::thread::hardware_concurrency();
    nt = std::max(1u, std::min(nt, 16u));
    if (count < (1u << 20) || nt == 1) {
        work(0, count);
        return SGEMM_OK;
    }
    std::vector<std::thread> pool;
    const size_t chunk = (count + nt - 1) / nt;
    for (unsigned t = 0; t < nt; ++t) {
        const size_t lo = t * chunk, hi = std::min(count, lo + chunk);
        if (lo < hi) pool.emplace_back(work, lo, hi);
    }
    for (auto& th : pool) th.join();
    return SGEMM_OK;
}

}  // extern "C"
