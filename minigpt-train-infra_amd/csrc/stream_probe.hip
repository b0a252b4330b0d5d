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
// work-groups and every access index is below N.  All arrays are carved from
// one allocation.  The multi-stream kernels run twice: on arrays placed back
// to back at power-of-two sizes ("aligned": the same offset in every array
// falls on the same DRAM banks) and with a 1 MiB + 4 KiB gap after each array
// ("staggered"), the way separately allocated tensors of unrelated sizes sit.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
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

}  // namespace

int main(int argc, char** argv) {
    const int64_t n = (argc > 1) ? std::atoll(argv[1]) : (int64_t(1) << 30);
    const int rounds = (argc > 2) ? std::atoi(argv[2]) : 3;
    if (n <= 0 || n % 1024 != 0 || n / 1024 > 0xFFFFFFFFll / 512) {
        std::printf("{\"error\": \"N must be a positive multiple of 1024 of at most 8388607 chunks\"}\n");
        return 2;
    }
    const uint32_t grid = static_cast<uint32_t>(n / 1024);
    const int64_t gap = (int64_t(1) << 20) + 4096;
    const int64_t bytes4 = n * 4, bytes2 = n * 2;
    const int64_t total = 3 * (bytes4 + gap) + 2 * (bytes2 + gap);
    char* buf;
    float* sink;
    CK(hipMalloc(&buf, total));
    CK(hipMalloc(&sink, 64));
    CK(hipMemset(buf, 0, total));
    CK(hipDeviceSynchronize());
    // the five arrays (p, m, v: 4 B/element; g, l: 2 B/element) for a given gap
    struct Layout {
        f4 *p, *m, *v;
        u2 *g, *l;
    };
    auto carve = [&](int64_t pad) {
        Layout L;
        int64_t o = 0;
        L.p = reinterpret_cast<f4*>(buf + o); o += bytes4 + pad;
        L.m = reinterpret_cast<f4*>(buf + o); o += bytes4 + pad;
        L.v = reinterpret_cast<f4*>(buf + o); o += bytes4 + pad;
        L.g = reinterpret_cast<u2*>(buf + o); o += bytes2 + pad;
        L.l = reinterpret_cast<u2*>(buf + o); o += bytes2;
        if (o > total) {
            std::printf("{\"error\": \"layout exceeds the allocation\"}\n");
            std::exit(1);
        }
        return L;
    };
    const Layout A = carve(0), S = carve(gap);
    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    struct Kernel {
        const char* name;
        double bytes_per_element;
    };
    const Kernel kernels[] = {{"read", 4},           {"write", 4},         {"copy_aligned", 8}, {"copy_staggered", 8},
                              {"inplace3_aligned", 24}, {"inplace3_staggered", 24}, {"mix_aligned", 28},
                              {"mix_staggered", 28}};
    const int reps = 10;
    for (int round = 0; round < rounds; ++round) {
        for (int k = 0; k < 8; ++k) {
            std::vector<float> t;
            for (int r = 0; r < reps; ++r) {
                CK(hipEventRecord(e0));
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
                CK(hipGetLastError());
                CK(hipEventRecord(e1));
                CK(hipEventSynchronize(e1));
                float ms = 0.f;
                CK(hipEventElapsedTime(&ms, e0, e1));
                t.push_back(ms);
            }
            std::sort(t.begin(), t.end());
            const double med = t[reps / 2];
            std::printf("{\"probe\": \"%s\", \"round\": %d, \"elements\": %lld, \"bytes_per_element\": %.0f, "
                        "\"median_ms\": %.4f, \"GBps\": %.1f}\n",
                        kernels[k].name, round, static_cast<long long>(n), kernels[k].bytes_per_element, med,
                        kernels[k].bytes_per_element * n / (med * 1e-3) / 1e9);
            std::fflush(stdout);
        }
    }
    return 0;
}
