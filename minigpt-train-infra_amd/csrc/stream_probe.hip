// stream_probe.hip -- what the memory system gives streaming kernels shaped
// like pass 2 of the optimizer step, as a ceiling to read pass 2's bandwidth
// against.  A standalone executable (not part of libmgopt); bench.py
// --stream-probe runs it and forwards its JSON lines.
//
// Every kernel uses pass 2's launch shape: one 512-thread work-group per
// 1024-element chunk, lanes 0-255 each move one 16-byte group per stream,
// nontemporal loads and stores, chunks in XCD-contiguous order.  Kernels:
//   read      one fp32 stream read                 4 B/element
//   write     one fp32 stream written              4 B/element
//   copy      one read stream, one write stream    8 B/element
//   inplace3  three fp32 streams read and written 24 B/element
//   mix       pass 2's byte mix without its arithmetic: a 2-byte stream read,
//             three fp32 streams read and written, a 2-byte stream written
//             (28 B/element)
// Arrays hold N elements (N a multiple of 1024); the grid is N / 1024
// work-groups and every access index is below N.
//
// Usage: stream_probe [N [rounds [mode]]], mode one of
//   layouts   (default) every kernel; the arrays carved from one allocation,
//             the multi-stream kernels run twice: placed back to back at
//             power-of-two sizes ("aligned": the same offset in every array
//             falls on the same DRAM banks) and with a 1 MiB + 4 KiB gap after
//             each array ("staggered")
//   gaps      the mix kernel on arrays carved from one allocation with each
//             gap of a list between consecutive arrays
//   separate  the mix kernel on five arrays from five allocations, for six
//             such sets obtained in turn (three held together, then some freed
//             and obtained again): where each array lands in physical memory
//             is then the allocator's choice, as for separately allocated
//             tensors
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));

#define CK(x)                                                                                   \
    do {                                                                                        \
        hipError_t e_ = (x);                                                                    \
        if (e_ != hipSuccess) {                                                                 \
            std::printf("{\"error\": \"%s at line %d\"}\n", hipGetErrorString(e_), __LINE__);   \
            std::exit(1);                                                                       \
        }                                                                                       \
    } while (0)

__device__ __forceinline__ f4 ld(const f4* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ void st(f4* p, f4 v) { __builtin_nontemporal_store(v, p); }
__device__ __forceinline__ u2 ld2(const u2* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ void st2(u2* p, u2 v) { __builtin_nontemporal_store(v, p); }

__device__ __forceinline__ uint32_t item(uint32_t bid, uint32_t n) {
    const uint32_t per = n / 8, rem = n % 8, x = bid % 8;
    return x * per + min(x, rem) + bid / 8;
}

__device__ __forceinline__ int64_t lane_index() {
    return static_cast<int64_t>(item(blockIdx.x, gridDim.x)) * 256 + threadIdx.x;
}

__global__ void __launch_bounds__(512) k_read(const f4* a, float* sink) {
    if (threadIdx.x >= 256) return;
    const f4 x = ld(a + lane_index());
    if (x.x == 1234.5f) sink[0] = x.y;  // the arrays hold zeros: never taken
}

__global__ void __launch_bounds__(512) k_write(f4* a) {
    if (threadIdx.x >= 256) return;
    st(a + lane_index(), f4{1.f, 2.f, 3.f, 4.f});
}

__global__ void __launch_bounds__(512) k_copy(const f4* a, f4* b) {
    if (threadIdx.x >= 256) return;
    const int64_t i = lane_index();
    st(b + i, ld(a + i));
}

__global__ void __launch_bounds__(512) k_inplace3(f4* p, f4* m, f4* v) {
    if (threadIdx.x >= 256) return;
    const int64_t i = lane_index();
    const f4 x = ld(p + i), y = ld(m + i), z = ld(v + i);
    st(p + i, x + 1.f);
    st(m + i, y + 1.f);
    st(v + i, z + 1.f);
}

__global__ void __launch_bounds__(512) k_mix(const u2* g, f4* p, f4* m, f4* v, u2* l) {
    if (threadIdx.x >= 256) return;
    const int64_t i = lane_index();
    const u2 gg = ld2(g + i);
    f4 x = ld(p + i), y = ld(m + i), z = ld(v + i);
    const float gf = __uint_as_float(gg.x << 16);
    x += gf;
    y += gf;
    z += gf;
    st(p + i, x);
    st(m + i, y);
    st(v + i, z);
    st2(l + i, u2{__float_as_uint(x.x), __float_as_uint(x.z)});
}

// The five arrays of the mix kernel (p, m, v: 4 B/element; g, l: 2 B/element).
struct Layout {
    f4 *p, *m, *v;
    u2 *g, *l;
};

// Median of `reps` timed launches of kernel k (after one untimed launch when
// warm is set).
template <typename Launch>
float median_ms(Launch launch, hipEvent_t e0, hipEvent_t e1, int reps, bool warm) {
    if (warm) {
        launch();
        CK(hipGetLastError());
    }
    std::vector<float> t;
    for (int r = 0; r < reps; ++r) {
        CK(hipEventRecord(e0));
        launch();
        CK(hipGetLastError());
        CK(hipEventRecord(e1));
        CK(hipEventSynchronize(e1));
        float ms = 0.f;
        CK(hipEventElapsedTime(&ms, e0, e1));
        t.push_back(ms);
    }
    std::sort(t.begin(), t.end());
    return t[t.size() / 2];
}

void mix_line(const char* mode, const char* what, long long detail, int round, int64_t n, float ms) {
    std::printf("{\"probe\": \"mix\", \"mode\": \"%s\", \"%s\": %lld, \"round\": %d, \"elements\": %lld, "
                "\"bytes_per_element\": 28, \"median_ms\": %.4f, \"GBps\": %.1f}\n",
                mode, what, detail, round, static_cast<long long>(n), ms, 28.0 * n / (ms * 1e-3) / 1e9);
    std::fflush(stdout);
}

// Arrays carved from one allocation, each followed by `gap` bytes.
Layout carve(char* buf, int64_t total, int64_t n, int64_t gap) {
    Layout L;
    int64_t o = 0;
    L.p = reinterpret_cast<f4*>(buf + o); o += n * 4 + gap;
    L.m = reinterpret_cast<f4*>(buf + o); o += n * 4 + gap;
    L.v = reinterpret_cast<f4*>(buf + o); o += n * 4 + gap;
    L.g = reinterpret_cast<u2*>(buf + o); o += n * 2 + gap;
    L.l = reinterpret_cast<u2*>(buf + o); o += n * 2;
    if (o > total) {
        std::printf("{\"error\": \"layout exceeds the allocation\"}\n");
        std::exit(1);
    }
    return L;
}

int run_layouts(int64_t n, int rounds, hipEvent_t e0, hipEvent_t e1) {
    const uint32_t grid = static_cast<uint32_t>(n / 1024);
    const int64_t gap = (int64_t(1) << 20) + 4096;
    const int64_t total = 3 * (n * 4 + gap) + 2 * (n * 2 + gap);
    char* buf;
    float* sink;
    CK(hipMalloc(&buf, total));
    CK(hipMalloc(&sink, 64));
    CK(hipMemset(buf, 0, total));
    CK(hipDeviceSynchronize());
    const Layout A = carve(buf, total, n, 0), S = carve(buf, total, n, gap);
    struct Kernel {
        const char* name;
        double bytes_per_element;
    };
    const Kernel kernels[] = {{"read", 4},           {"write", 4},         {"copy_aligned", 8}, {"copy_staggered", 8},
                              {"inplace3_aligned", 24}, {"inplace3_staggered", 24}, {"mix_aligned", 28},
                              {"mix_staggered", 28}};
    for (int round = 0; round < rounds; ++round) {
        for (int k = 0; k < 8; ++k) {
            auto launch = [&]() {
                switch (k) {
                    case 0: hipLaunchKernelGGL(k_read, dim3(grid), dim3(512), 0, 0, A.p, sink); break;
                    case 1: hipLaunchKernelGGL(k_write, dim3(grid), dim3(512), 0, 0, A.m); break;
                    case 2: hipLaunchKernelGGL(k_copy, dim3(grid), dim3(512), 0, 0, A.p, A.m); break;
                    case 3: hipLaunchKernelGGL(k_copy, dim3(grid), dim3(512), 0, 0, S.p, S.m); break;
                    case 4: hipLaunchKernelGGL(k_inplace3, dim3(grid), dim3(512), 0, 0, A.p, A.m, A.v); break;
                    case 5: hipLaunchKernelGGL(k_inplace3, dim3(grid), dim3(512), 0, 0, S.p, S.m, S.v); break;
                    case 6: hipLaunchKernelGGL(k_mix, dim3(grid), dim3(512), 0, 0, A.g, A.p, A.m, A.v, A.l); break;
                    default: hipLaunchKernelGGL(k_mix, dim3(grid), dim3(512), 0, 0, S.g, S.p, S.m, S.v, S.l); break;
                }
            };
            const double med = median_ms(launch, e0, e1, 10, false);
            std::printf("{\"probe\": \"%s\", \"round\": %d, \"elements\": %lld, \"bytes_per_element\": %.0f, "
                        "\"median_ms\": %.4f, \"GBps\": %.1f}\n",
                        kernels[k].name, round, static_cast<long long>(n), kernels[k].bytes_per_element, med,
                        kernels[k].bytes_per_element * n / (med * 1e-3) / 1e9);
            std::fflush(stdout);
        }
    }
    CK(hipFree(buf));
    CK(hipFree(sink));
    return 0;
}

int run_gaps(int64_t n, int rounds, hipEvent_t e0, hipEvent_t e1) {
    const uint32_t grid = static_cast<uint32_t>(n / 1024);
    const int64_t K = 1024, M = 1024 * 1024;
    const int64_t gaps[] = {0,     4 * K, 16 * K,    64 * K,    128 * K, 256 * K, 512 * K, 768 * K, M,
                            M + 4 * K, 3 * M / 2, 2 * M, 2 * M + 4 * K, 3 * M, 4 * M, 8 * M + 4 * K, 32 * M + 4 * K};
    const int64_t gmax = 32 * M + 4 * K;
    const int64_t total = 3 * (n * 4 + gmax) + 2 * (n * 2 + gmax);
    char* buf;
    CK(hipMalloc(&buf, total));
    CK(hipMemset(buf, 0, total));
    CK(hipDeviceSynchronize());
    for (int round = 0; round < rounds; ++round) {
        for (int64_t gap : gaps) {
            const Layout L = carve(buf, total, n, gap);
            auto launch = [&]() { hipLaunchKernelGGL(k_mix, dim3(grid), dim3(512), 0, 0, L.g, L.p, L.m, L.v, L.l); };
            mix_line("gaps", "gap_bytes", static_cast<long long>(gap), round, n, median_ms(launch, e0, e1, 10, true));
        }
    }
    CK(hipFree(buf));
    return 0;
}

struct SeparateSet {
    Layout L;
    bool live = false;
};

void obtain(SeparateSet& s, int64_t n) {
    CK(hipMalloc(&s.L.p, n * 4));
    CK(hipMalloc(&s.L.m, n * 4));
    CK(hipMalloc(&s.L.v, n * 4));
    CK(hipMalloc(&s.L.g, n * 2));
    CK(hipMalloc(&s.L.l, n * 2));
    CK(hipMemset(s.L.p, 0, n * 4));
    CK(hipMemset(s.L.m, 0, n * 4));
    CK(hipMemset(s.L.v, 0, n * 4));
    CK(hipMemset(s.L.g, 0, n * 2));
    CK(hipMemset(s.L.l, 0, n * 2));
    CK(hipDeviceSynchronize());
    s.live = true;
}

void release(SeparateSet& s) {
    if (!s.live) return;
    CK(hipFree(s.L.p));
    CK(hipFree(s.L.m));
    CK(hipFree(s.L.v));
    CK(hipFree(s.L.g));
    CK(hipFree(s.L.l));
    s.live = false;
}

int run_separate(int64_t n, int rounds, hipEvent_t e0, hipEvent_t e1) {
    const uint32_t grid = static_cast<uint32_t>(n / 1024);
    // at most three sets (3 x 28 B x N) are held at once
    SeparateSet sets[6];
    auto measure = [&](int which, int round) {
        const Layout& L = sets[which].L;
        auto launch = [&]() { hipLaunchKernelGGL(k_mix, dim3(grid), dim3(512), 0, 0, L.g, L.p, L.m, L.v, L.l); };
        mix_line("separate", "set", which, round, n, median_ms(launch, e0, e1, 10, true));
    };
    obtain(sets[0], n);
    obtain(sets[1], n);
    obtain(sets[2], n);
    for (int round = 0; round < rounds; ++round)
        for (int k = 0; k < 3; ++k) measure(k, round);
    release(sets[0]);
    obtain(sets[3], n);
    release(sets[1]);
    release(sets[2]);
    obtain(sets[4], n);
    obtain(sets[5], n);
    for (int round = 0; round < rounds; ++round)
        for (int k = 3; k < 6; ++k) measure(k, round);
    for (auto& s : sets) release(s);
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    const int64_t n = (argc > 1) ? std::atoll(argv[1]) : (int64_t(1) << 30);
    const int rounds = (argc > 2) ? std::atoi(argv[2]) : 3;
    const std::string mode = (argc > 3) ? argv[3] : "layouts";
    if (n <= 0 || n % 1024 != 0 || n / 1024 > 0xFFFFFFFFll / 512 || rounds <= 0) {
        std::printf("{\"error\": \"N must be a positive multiple of 1024 of at most 8388607 chunks, rounds positive\"}\n");
        return 2;
    }
    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    if (mode == "layouts") return run_layouts(n, rounds, e0, e1);
    if (mode == "gaps") return run_gaps(n, rounds, e0, e1);
    if (mode == "separate") return run_separate(n, rounds, e0, e1);
    std::printf("{\"error\": \"mode must be layouts, gaps or separate\"}\n");
    return 2;
}
