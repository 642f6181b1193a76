// lds_probe: replays wave-wide LDS access patterns, one dispatch per pattern,
// so that rocprofv3's SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE (or the event
// time) of each dispatch measures how gfx950's LDS serves that pattern.
//
//   lds_probe <pattern file> <iterations>
//
// The pattern file has one pattern per line:
//
//   <name> <r|w> <bytes per lane: 4|8|16> <64 byte addresses, one per lane>
//
// Every dispatch is 256 work-groups of one wave (one per CU on an MI355X);
// each wave issues <iterations> x 8 accesses of the pattern (ds_read_b32/b64/
// b128 or ds_write_b32/b64/b128 at the lane's address) with a wait after each
// group of 8, so a dispatch holds exactly 256 x 8 x <iterations> wave-wide
// LDS instructions of one kind.  Addresses are checked on the host: each must
// be a multiple of its width and the access must end inside the kernel's
// LDS array.  The program prints one line per pattern: its dispatch order,
// name and the event time per wave-wide instruction.

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <sstream>
#include <string>
#include <vector>

namespace {

constexpr int kLdsBytes = 64 * 1024;  // the probe's LDS array; patterns must stay inside it
constexpr int kWaves = 256;

typedef float f2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));

#define CHECK(call)                                                            \
    do {                                                                       \
        hipError_t e_ = (call);                                                \
        if (e_ != hipSuccess) {                                                \
            fprintf(stderr, "%s failed: %s\n", #call, hipGetErrorString(e_)); \
            return 1;                                                          \
        }                                                                      \
    } while (0)

// The array is the kernel's only LDS object, so its byte offset is 0 and a
// pattern's byte addresses are LDS addresses.  Touching every lane's word of
// it keeps the allocation; out[] keeps the loaded values alive.
template <int OP, int WIDTH>
__global__ void __launch_bounds__(64) lds_probe_kernel(const uint32_t* __restrict__ addrs, int iters,
                                                       float* __restrict__ out) {
    __shared__ f4 lds[kLdsBytes / 16];
    const int lane = (int)threadIdx.x;
    for (int i = lane; i < kLdsBytes / 16; i += 64) lds[i] = f4{(float)i, 1.0f, 2.0f, 3.0f};
    __syncthreads();
    const uint32_t a = addrs[lane];
    float acc = 0.0f;
    for (int it = 0; it < iters; ++it) {
        if constexpr (OP == 0 && WIDTH == 16) {
            f4 v0, v1, v2, v3, v4, v5, v6, v7;
            asm volatile(
                "ds_read_b128 %0, %8\n ds_read_b128 %1, %8\n ds_read_b128 %2, %8\n ds_read_b128 %3, %8\n"
                "ds_read_b128 %4, %8\n ds_read_b128 %5, %8\n ds_read_b128 %6, %8\n ds_read_b128 %7, %8\n"
                "s_waitcnt lgkmcnt(0)"
                : "=v"(v0), "=v"(v1), "=v"(v2), "=v"(v3), "=v"(v4), "=v"(v5), "=v"(v6), "=v"(v7)
                : "v"(a));
            acc += v0.x + v1.y + v2.z + v3.w + v4.x + v5.y + v6.z + v7.w;
        } else if constexpr (OP == 0 && WIDTH == 8) {
            f2 v0, v1, v2, v3, v4, v5, v6, v7;
            asm volatile(
                "ds_read_b64 %0, %8\n ds_read_b64 %1, %8\n ds_read_b64 %2, %8\n ds_read_b64 %3, %8\n"
                "ds_read_b64 %4, %8\n ds_read_b64 %5, %8\n ds_read_b64 %6, %8\n ds_read_b64 %7, %8\n"
                "s_waitcnt lgkmcnt(0)"
                : "=v"(v0), "=v"(v1), "=v"(v2), "=v"(v3), "=v"(v4), "=v"(v5), "=v"(v6), "=v"(v7)
                : "v"(a));
            acc += v0.x + v1.y + v2.x + v3.y + v4.x + v5.y + v6.x + v7.y;
        } else if constexpr (OP == 0 && WIDTH == 4) {
            float v0, v1, v2, v3, v4, v5, v6, v7;
            asm volatile(
                "ds_read_b32 %0, %8\n ds_read_b32 %1, %8\n ds_read_b32 %2, %8\n ds_read_b32 %3, %8\n"
                "ds_read_b32 %4, %8\n ds_read_b32 %5, %8\n ds_read_b32 %6, %8\n ds_read_b32 %7, %8\n"
                "s_waitcnt lgkmcnt(0)"
                : "=v"(v0), "=v"(v1), "=v"(v2), "=v"(v3), "=v"(v4), "=v"(v5), "=v"(v6), "=v"(v7)
                : "v"(a));
            acc += v0 + v1 + v2 + v3 + v4 + v5 + v6 + v7;
        } else if constexpr (OP == 1 && WIDTH == 16) {
            const f4 d{acc, 1.0f, 2.0f, 3.0f};
            asm volatile(
                "ds_write_b128 %0, %1\n ds_write_b128 %0, %1\n ds_write_b128 %0, %1\n ds_write_b128 %0, %1\n"
                "ds_write_b128 %0, %1\n ds_write_b128 %0, %1\n ds_write_b128 %0, %1\n ds_write_b128 %0, %1\n"
                "s_waitcnt lgkmcnt(0)" ::"v"(a), "v"(d) : "memory");
        } else if constexpr (OP == 1 && WIDTH == 8) {
            const f2 d{acc, 1.0f};
            asm volatile(
                "ds_write_b64 %0, %1\n ds_write_b64 %0, %1\n ds_write_b64 %0, %1\n ds_write_b64 %0, %1\n"
                "ds_write_b64 %0, %1\n ds_write_b64 %0, %1\n ds_write_b64 %0, %1\n ds_write_b64 %0, %1\n"
                "s_waitcnt lgkmcnt(0)" ::"v"(a), "v"(d) : "memory");
        } else {
            asm volatile(
                "ds_write_b32 %0, %1\n ds_write_b32 %0, %1\n ds_write_b32 %0, %1\n ds_write_b32 %0, %1\n"
                "ds_write_b32 %0, %1\n ds_write_b32 %0, %1\n ds_write_b32 %0, %1\n ds_write_b32 %0, %1\n"
                "s_waitcnt lgkmcnt(0)" ::"v"(a), "v"(acc) : "memory");
        }
    }
    __syncthreads();
    out[blockIdx.x * 64 + lane] = acc + lds[lane].x;
}

struct Pattern {
    std::string name;
    int op = 0;     // 0 read, 1 write
    int width = 0;  // bytes per lane
    std::vector<uint32_t> addr;
};

bool parse(const std::string& path, std::vector<Pattern>& out) {
    std::ifstream f(path);
    if (!f) {
        fprintf(stderr, "cannot open %s\n", path.c_str());
        return false;
    }
    std::string line;
    int lineno = 0;
    while (std::getline(f, line)) {
        ++lineno;
        if (line.empty() || line[0] == '#') continue;
        std::istringstream in(line);
        Pattern p;
        std::string op;
        in >> p.name >> op >> p.width;
        p.op = op == "w" ? 1 : 0;
        if ((op != "r" && op != "w") || (p.width != 4 && p.width != 8 && p.width != 16)) {
            fprintf(stderr, "%s:%d: expected <name> <r|w> <4|8|16> <64 addresses>\n", path.c_str(), lineno);
            return false;
        }
        long long v;
        while (in >> v) {
            if (v < 0 || v % p.width != 0 || v + p.width > kLdsBytes) {
                fprintf(stderr, "%s:%d: address %lld is not a multiple of %d inside %d bytes of LDS\n",
                        path.c_str(), lineno, v, p.width, kLdsBytes);
                return false;
            }
            p.addr.push_back((uint32_t)v);
        }
        if (p.addr.size() != 64) {
            fprintf(stderr, "%s:%d: %zu addresses, expected 64\n", path.c_str(), lineno, p.addr.size());
            return false;
        }
        out.push_back(p);
    }
    return true;
}

template <int OP, int WIDTH>
void launch(const uint32_t* addrs, int iters, float* out) {
    hipLaunchKernelGGL((lds_probe_kernel<OP, WIDTH>), dim3(kWaves), dim3(64), 0, 0, addrs, iters, out);
}

}  // namespace

int main(int argc, char** argv) {
    if (argc < 3) {
        fprintf(stderr, "usage: %s <pattern file> <iterations>\n", argv[0]);
        return 2;
    }
    std::vector<Pattern> pats;
    if (!parse(argv[1], pats)) return 2;
    const int iters = atoi(argv[2]);
    if (iters <= 0 || pats.empty()) {
        fprintf(stderr, "need at least one pattern and a positive iteration count\n");
        return 2;
    }
    uint32_t* d_addr = nullptr;
    float* d_out = nullptr;
    CHECK(hipMalloc(&d_addr, 64 * sizeof(uint32_t)));
    CHECK(hipMalloc(&d_out, kWaves * 64 * sizeof(float)));
    hipEvent_t e0, e1;
    CHECK(hipEventCreate(&e0));
    CHECK(hipEventCreate(&e1));
    const double instr = (double)kWaves * 8.0 * iters;
    for (size_t q = 0; q < pats.size(); ++q) {
        const Pattern& p = pats[q];
        CHECK(hipMemcpy(d_addr, p.addr.data(), 64 * sizeof(uint32_t), hipMemcpyHostToDevice));
        CHECK(hipEventRecord(e0, 0));
        if (p.op == 0 && p.width == 16) launch<0, 16>(d_addr, iters, d_out);
        else if (p.op == 0 && p.width == 8) launch<0, 8>(d_addr, iters, d_out);
        else if (p.op == 0) launch<0, 4>(d_addr, iters, d_out);
        else if (p.width == 16) launch<1, 16>(d_addr, iters, d_out);
        else if (p.width == 8) launch<1, 8>(d_addr, iters, d_out);
        else launch<1, 4>(d_addr, iters, d_out);
        CHECK(hipGetLastError());
        CHECK(hipEventRecord(e1, 0));
        CHECK(hipEventSynchronize(e1));
        float ms = 0.0f;
        CHECK(hipEventElapsedTime(&ms, e0, e1));
        printf("%zu %s %s b%d %.3f ns/instr/CU\n", q, p.name.c_str(), p.op ? "write" : "read", p.width * 8,
               ms * 1e6 / instr * kWaves);
        fflush(stdout);
    }
    CHECK(hipFree(d_addr));
    CHECK(hipFree(d_out));
    return 0;
}
