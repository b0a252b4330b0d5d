// mgopt.hip -- fused optimizer step for one MI355X (gfx950).
//
// One training-loop iteration of the reference (train.py:483-491) becomes:
//
//   pass 1   norm_kernel       read every grad once: unscale, non-finite flag,
//                              fp64 sum of squares -> one partial per chunk
//   finalize finalize_kernel   one work-group: total norm, clip coefficient,
//                              found_inf (fixed reduction order: bit-stable)
//   prologue prologue_kernel   one thread per tensor: step += 1 unless
//                              found_inf, then the tensor's fp32 constants
//                              for pass 2 (bias corrections, step size, decay)
//   pass 2   adamw_kernel      read grad/param/m/v once, write param/m/v
//                              (+ bf16/fp16 model copy): unscale, clip, AdamW
//   update   scaler_kernel     GradScaler scale/growth-tracker state machine
//
// Small plans (at most 2M elements) fold the finalize into pass 1 (the work-group
// taking the last ticket runs it) and the prologue into pass 2
// (adamw_fold_kernel): three kernels per step instead of five.
//
// Every scalar decision (skip, scale, coefficient, step count) stays on the
// device, so the host never waits on the GPU inside a step.
//
// The element arithmetic follows torch 2.10.0's CPU path (the reference's
// pinned numerics) operation by operation; the comments on adam_elem give the
// torch source lines.  Build with -ffp-contract=off: every fused multiply-add
// here is written out, and no other pair of operations may be fused.

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "mgopt.h"

namespace {

constexpr int kBlock = 512;          // work-group size of pass 1, finalize and the helper kernels
// Pass 2 runs one short work-group per chunk.  With the default 1024-element
// chunks a 512-thread work-group gives one 4-element group to lanes 0-255
// and lanes 256-511 retire at once: half of a CU's wave slots carry memory
// traffic and work-groups turn over quickly.  Measured on MI355X against
// 256-thread groups, 2048/4096/16384/65536-element chunks and LDS-reserved
// caps of 2-5 work-groups per CU, this was the fastest or tied on the
// 8.2B set and within 2 % of the best on 124M-2.5B sets.
constexpr int kAdamBlock = 512;      // work-group size of pass 2
constexpr size_t kAdamLds = 0;       // LDS bytes reserved per pass-2 work-group (0: no cap on work-groups per CU)
constexpr int kVec = 4;              // elements per thread per access: 4 = one 16-B fp32 access per lane;
                                     // 8 (two adjacent 16-B accesses) measured 1.8x slower (32-B lane stride)
constexpr int kStagingSlots = 4;     // pinned host buffers for grad-pointer uploads
// pass-2 access tuning (measured on MI355X with the Qwen3-8B-shaped set)
constexpr int kUnroll = 1;           // 4-element accesses in flight per thread before use
constexpr bool kNtLoad = true;       // nontemporal loads of grad/param/exp_avg/exp_avg_sq
constexpr bool kNtStore = true;      // nontemporal stores of param/exp_avg/exp_avg_sq
// Pass-1 accesses in flight per thread, and elements per access of 16-bit
// gradients (fp32 gradients take 4, one 16-B access).  Unrolls of 4 and 8
// and 16-B accesses of eight 16-bit values measured no faster on GPT-2-small
// (0.053 ms), and 16-B accesses 7-8 % slower on the Qwen3-8B set's bf16
// gradients (2.47-2.51 ms against 2.31).
constexpr int kNormUnroll = 2;
constexpr int kNormVec16 = 4;
// Pass 2 reads the gradients pass 1 has just read.  When a plan's gradients
// fit in the MI355X's 256 MB Infinity Cache (the memory-side cache in front
// of HBM), pass 1 reads them with ordinary loads, which allocate there, and
// pass 2's gradient reads hit it.  Measured on GPT-2-small (249 MB of fp16
// gradients): pass 2 0.513 ms against 0.560 ms after nontemporal pass-1
// loads, the whole step 0.573 against 0.614 ms.  Larger sets keep
// nontemporal pass-1 loads: allocating made pass 1 up to 15 % slower on the
// 2.6 GB and 16 GB gradient sets, with no gain in pass 2 beyond run-to-run
// spread.  Nontemporal pass-2 gradient loads still hit the cache.
constexpr int64_t kCachedGradBytes = int64_t(256) << 20;
// pass 1 has its own chunk table of kNormChunk elements per chunk and
// work-group, whatever the pass-2 chunk size: the finalize kernel then reads
// one partial per 128K elements.  Pass 1 + finalize measured in one process
// on the Qwen3-8B set: 16K-element chunks 2.94 ms, 32K 2.50, 64K 2.35,
// 128K 2.29, 256K 2.31, 512K 2.31; above 128K the smaller sets lose (GPT-2
// small 0.049 ms at 128K, 0.100 at 512K).  Smaller chunks on small sets
// (the largest power of two down to 16K giving 2048 work-groups: 32K on
// GPT-2-small, 16K on the 0.8M set) measured the same (0.047 ms, 0.015 ms).
// A grid-stride form with 1024-4096 work-groups per class was slower still.
constexpr int64_t kNormChunk = 131072;
// Small plans run a step as three kernels instead of five: pass 1 with the
// finalize in its last work-group, pass 2 with the prologue folded in, and
// the scaler update.  A plan qualifies with at most kFoldElems elements, no
// empty tensor and no tensor of more than kFoldTensorChunks pass-2 chunks:
// every chunk of a tensor takes a ticket from that tensor's counter, one
// counter per 128-byte line, and the atomics on one line serialize.  Beyond
// these limits the saved launches no longer pay for the tickets: measured per
// step on MI355X, the three-kernel form gains 2-7 us eager and 1-5 us as a
// replayed graph on sets of up to 2M elements in tensors of at most 256
// chunks, loses 2-6 us on 4M and 8M elements in 16 tensors, and 3.9 us
// replayed on one tensor of 1,024 chunks.  Their pass-1 chunks are shorter:
// replayed steps on 0.8M, 1M and 2M elements measured 16,384 the fastest or
// tied (4,096 2-5 us slower, 32,768 up to 0.8 us, 65,536 1.4-2.8 us).
// MGOPT_FOLD=0 in the environment at plan creation keeps the five-kernel
// form; MGOPT_FOLD=1 takes the three-kernel form beyond the limits too, up to
// kFoldForcedElems (for measuring them).
// (Folding only the finalize into a pass 1 of one round of work-groups,
// GPT-2-small's 950, measured 0.567 ms per step both ways: the ticket each
// work-group waits for costs what the saved launch gains.)
constexpr int64_t kFoldElems = int64_t(1) << 21;
constexpr int64_t kFoldTensorChunks = 256;
constexpr int64_t kFoldForcedElems = int64_t(1) << 26;
constexpr int64_t kNormChunkFold = 16384;
constexpr uint32_t kTicketStride = 32;  // uint32 counters per 128-byte line: one tensor's ticket per line
// A dispatch packet carries its grid size in work-items as a 32-bit value, so
// launches over more chunks than fit are issued in pieces, each piece given
// its first chunk (and first partial slot) as arguments.  8,388,607
// work-groups of 512 threads are the most one packet holds; at 1024-element
// chunks one piece covers 8.59e9 elements.
constexpr uint32_t kMaxGroupsPerLaunch = 0xFFFFFFFFu / 512;
static_assert(kBlock <= 512 && kAdamBlock <= 512, "kMaxGroupsPerLaunch assumes work-groups of at most 512 threads");
// The command processor hands work-groups to the 8 XCDs round-robin in
// blockIdx order.  With the remap each XCD instead walks one contiguous range
// of chunks, so its L2 and address-translation caches see 1/8 of the address
// window instead of every eighth chunk of all of it.  Measured on the
// Qwen3-8B-shaped set: pass 2 0.1-0.2 ms faster (within run-to-run spread),
// pass 1 0.0-0.3 ms slower, so only pass 2 uses it.
constexpr bool kXcdMapAdam = true;
constexpr bool kXcdMapNorm = false;
constexpr uint32_t kXcds = 8;

struct DevTensor {
    float* param;   // fp32 param or fp32 master
    void* lowp;     // bf16/fp16 model param or nullptr
    float* m;
    float* v;
    int64_t numel;
    int32_t group;
    uint32_t row_chunks;  // 0: param, m, v contiguous; else pass-2 chunks per row of row-laid-out storage
    int64_t ppitch;       // row stride of param (elements), when row_chunks > 0
    int64_t spitch;       // row stride of m and v (elements), when row_chunks > 0
};

// Where pass-2 chunk `index` (chunk_elems elements) of tensor T starts in
// its fp32 param, m and v.  Row-laid-out storage keeps a tensor's master, m
// and v rows side by side; a chunk never crosses a row (the row length is a
// multiple of chunk_elems), so one division per chunk places it.
struct ChunkPtrs {
    float* p;
    float* m;
    float* v;
};
__device__ __forceinline__ ChunkPtrs chunk_ptrs(const DevTensor& T, uint32_t index, int64_t chunk_elems) {
    if (T.row_chunks == 0) {
        const int64_t s = static_cast<int64_t>(index) * chunk_elems;
        return {T.param + s, T.m + s, T.v + s};
    }
    const uint32_t r = index / T.row_chunks;
    const int64_t c0 = static_cast<int64_t>(index - r * T.row_chunks) * chunk_elems;
    return {T.param + r * T.ppitch + c0, T.m + r * T.spitch + c0, T.v + r * T.spitch + c0};
}

struct Chunk {
    uint32_t tensor;
    uint32_t index;  // chunk number inside its tensor; start = index * chunk_elems
};

struct Partial {
    double sumsq;
    uint32_t nonfinite;
    uint32_t pad;
};

// Log-window statistics kept on the device so a training loop reads them once
// per window (train.py:434-441,487-489,501-507) instead of syncing per step.
struct Window {
    float norm_last;   // last clip_grad_norm_ result
    float norm_max;    // running maximum, torch.maximum semantics (NaN propagates)
    uint32_t skipped;  // optimizer steps skipped on found_inf
    uint32_t taken;    // optimizer steps taken
};

struct GroupConst {
    double lr, wd, beta1, beta2, eps;
    int32_t maximize;
    int32_t pad;
};

// ---------------------------------------------------------------------------
// element conversions
// ---------------------------------------------------------------------------

template <typename T>
struct GradIO;

template <>
struct GradIO<float> {
    static __device__ __forceinline__ float to_f32(float x) { return x; }
    static __device__ __forceinline__ float from_f32(float x) { return x; }
};

struct Bf16 {
    uint16_t bits;
};

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;  // NaN -> canonical quiet NaN
    return static_cast<uint16_t>((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

template <>
struct GradIO<Bf16> {
    static __device__ __forceinline__ float to_f32(Bf16 x) { return __uint_as_float(static_cast<uint32_t>(x.bits) << 16); }
    static __device__ __forceinline__ Bf16 from_f32(float x) { return Bf16{f32_to_bf16_rne(x)}; }
};

template <>
struct GradIO<_Float16> {
    static __device__ __forceinline__ float to_f32(_Float16 x) { return static_cast<float>(x); }
    static __device__ __forceinline__ _Float16 from_f32(float x) { return static_cast<_Float16>(x); }
};

// Four consecutive elements of a 2-byte type travel as one 8-byte access,
// four fp32 as one 16-byte access.
template <typename T>
struct Vec4 {
    T e[4];
};

template <typename T>
__device__ __forceinline__ Vec4<T> load4(const T* p) {
    Vec4<T> r;
    if constexpr (sizeof(T) == 4) {
        const float4 q = *reinterpret_cast<const float4*>(p);
        r.e[0] = reinterpret_cast<const T&>(q.x);
        r.e[1] = reinterpret_cast<const T&>(q.y);
        r.e[2] = reinterpret_cast<const T&>(q.z);
        r.e[3] = reinterpret_cast<const T&>(q.w);
    } else {
        const uint2 q = *reinterpret_cast<const uint2*>(p);
        uint16_t h[4] = {static_cast<uint16_t>(q.x & 0xFFFFu), static_cast<uint16_t>(q.x >> 16),
                         static_cast<uint16_t>(q.y & 0xFFFFu), static_cast<uint16_t>(q.y >> 16)};
#pragma unroll
        for (int k = 0; k < 4; ++k) std::memcpy(&r.e[k], &h[k], 2);
    }
    return r;
}

template <typename T>
__device__ __forceinline__ void store4(T* p, const Vec4<T>& r) {
    if constexpr (sizeof(T) == 4) {
        float4 q;
        q.x = reinterpret_cast<const float&>(r.e[0]);
        q.y = reinterpret_cast<const float&>(r.e[1]);
        q.z = reinterpret_cast<const float&>(r.e[2]);
        q.w = reinterpret_cast<const float&>(r.e[3]);
        *reinterpret_cast<float4*>(p) = q;
    } else {
        uint16_t h[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) std::memcpy(&h[k], &r.e[k], 2);
        uint2 q;
        q.x = static_cast<uint32_t>(h[0]) | (static_cast<uint32_t>(h[1]) << 16);
        q.y = static_cast<uint32_t>(h[2]) | (static_cast<uint32_t>(h[3]) << 16);
        *reinterpret_cast<uint2*>(p) = q;
    }
}

__device__ __forceinline__ bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

// Work item of work-group `bid` in a grid of `n`: a bijection of [0, n).
// Work-group bid runs on XCD bid % 8; XCD x gets items
// [x*per + min(x, rem), ...) of length per + (x < rem), in order.
template <bool kRemap>
__device__ __forceinline__ uint32_t xcd_item(uint32_t bid, uint32_t n) {
    if constexpr (!kRemap) return bid;
    const uint32_t per = n / kXcds, rem = n % kXcds;
    const uint32_t x = bid % kXcds;
    return x * per + min(x, rem) + bid / kXcds;
}

// Native vector types for 16-byte (4 x fp32) and 8-byte (4 x 16-bit) accesses;
// the nontemporal forms mark streamed data that no later access reuses.
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <bool NT>
__device__ __forceinline__ f32x4 ld16(const float* p) {
    if constexpr (NT) return __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
    else return *reinterpret_cast<const f32x4*>(p);
}
template <bool NT>
__device__ __forceinline__ void st16(float* p, f32x4 v) {
    if constexpr (NT) __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(p));
    else *reinterpret_cast<f32x4*>(p) = v;
}
template <bool NT>
__device__ __forceinline__ u32x2 ld8(const void* p) {
    if constexpr (NT) return __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
    else return *reinterpret_cast<const u32x2*>(p);
}
template <bool NT>
__device__ __forceinline__ void st8(void* p, u32x2 v) {
    if constexpr (NT) __builtin_nontemporal_store(v, reinterpret_cast<u32x2*>(p));
    else *reinterpret_cast<u32x2*>(p) = v;
}

// W consecutive gradient elements widened to fp32 (W = 4 or 8): 16-byte
// accesses for fp32 and for eight 16-bit values, an 8-byte access for four.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <typename GT>
__device__ __forceinline__ void unpack16(uint32_t w, float* out) {
    const uint16_t lo = static_cast<uint16_t>(w & 0xFFFFu), hi = static_cast<uint16_t>(w >> 16);
    GT a, b;
    std::memcpy(&a, &lo, 2);
    std::memcpy(&b, &hi, 2);
    out[0] = GradIO<GT>::to_f32(a);
    out[1] = GradIO<GT>::to_f32(b);
}

template <typename GT, bool NT, int W>
__device__ __forceinline__ void load_grad(const GT* G, float out[W]) {
    static_assert(W == 4 || W == 8, "4 or 8 elements per access");
    if constexpr (sizeof(GT) == 4) {
#pragma unroll
        for (int k = 0; k < W / 4; ++k) {
            const f32x4 x = ld16<NT>(reinterpret_cast<const float*>(G) + 4 * k);
            out[4 * k] = x.x; out[4 * k + 1] = x.y; out[4 * k + 2] = x.z; out[4 * k + 3] = x.w;
        }
    } else if constexpr (W == 4) {
        const u32x2 x = ld8<NT>(G);
        unpack16<GT>(x.x, out);
        unpack16<GT>(x.y, out + 2);
    } else {
        const f32x4 x = ld16<NT>(reinterpret_cast<const float*>(G));
        const u32x4 w = __builtin_bit_cast(u32x4, x);
        unpack16<GT>(w.x, out);
        unpack16<GT>(w.y, out + 2);
        unpack16<GT>(w.z, out + 4);
        unpack16<GT>(w.w, out + 6);
    }
}

// ---------------------------------------------------------------------------
// norm pieces shared by pass 1, the flat norm and finalize
// ---------------------------------------------------------------------------

// Outputs of the finalize step (any pointer may be NULL).
struct FinalizeArgs {
    double max_norm;
    float* norm_out;
    float* coef_out;
    float* found_inf_out;
    Window* win;
};

struct NormArgs {
    const DevTensor* tensors;
    const Chunk* chunks;
    const void* const* grads;
    Partial* partials;
    const float* scale;  // nullable
    int64_t chunk_elems;
    uint32_t chunk_begin;
    uint32_t count;         // chunks of this launch's class
    uint32_t partial_base;  // first partial slot of this launch
    // folded form only: the ticket counter, the plan's partial count and the finalize outputs
    uint32_t* ticket;
    uint32_t total;
    FinalizeArgs fin;
};

__device__ __forceinline__ double wave_sum(double x) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off);
    return x;
}

__device__ __forceinline__ uint32_t wave_or(uint32_t x) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) x |= __shfl_xor(x, off);
    return x;
}

// Reduces (sum, flag) over a work-group of NT threads in a fixed order and
// returns the result in thread 0.
template <int NT>
__device__ __forceinline__ void block_reduce(double& s, uint32_t& f) {
    __shared__ double ws[NT / 64];
    __shared__ uint32_t wf[NT / 64];
    s = wave_sum(s);
    f = wave_or(f);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) {
        ws[wave] = s;
        wf[wave] = f;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        double t = 0.0;
        uint32_t g = 0;
#pragma unroll
        for (int w = 0; w < NT / 64; ++w) {
            t += ws[w];
            g |= wf[w];
        }
        s = t;
        f = g;
    }
}

__device__ __forceinline__ void norm_accum(float x, float inv, bool unscale, double& acc, uint32_t& bad) {
    // grad_scaler.py:280-284: the finiteness test is on the scaled input value
    bad |= static_cast<uint32_t>(!isfinite(x));
    const float u = unscale ? x * inv : x;
    const double d = static_cast<double>(u);
    acc = fma(d, d, acc);  // u*u is exact in double
}

// One pass-1 chunk of `len` gradient elements from g, accumulated by a
// work-group of kBlock threads into (acc, bad) of each thread.
template <typename GT, bool NT>
__device__ __forceinline__ void norm_chunk(const GT* __restrict__ g, int64_t len, float inv, bool unscale, double& acc,
                                           uint32_t& bad) {
    constexpr int V = sizeof(GT) == 4 ? 4 : kNormVec16;
    int64_t done = 0;
    if (aligned(g, sizeof(GT) * V)) {
        const int64_t nvec = len / V;
        int64_t i = threadIdx.x;
        for (; i + (kNormUnroll - 1) * kBlock < nvec; i += kNormUnroll * kBlock) {
            float x[kNormUnroll][V];
#pragma unroll
            for (int u = 0; u < kNormUnroll; ++u) load_grad<GT, NT, V>(g + (i + u * kBlock) * V, x[u]);
#pragma unroll
            for (int u = 0; u < kNormUnroll; ++u)
#pragma unroll
                for (int k = 0; k < V; ++k) norm_accum(x[u][k], inv, unscale, acc, bad);
        }
        for (; i < nvec; i += kBlock) {
            float x[V];
            load_grad<GT, NT, V>(g + i * V, x);
#pragma unroll
            for (int k = 0; k < V; ++k) norm_accum(x[k], inv, unscale, acc, bad);
        }
        done = nvec * V;
    }
    for (int64_t i = done + threadIdx.x; i < len; i += kBlock) norm_accum(GradIO<GT>::to_f32(g[i]), inv, unscale, acc, bad);
}

__device__ __forceinline__ float inv_scale_of(const float* scale) {
    // grad_scaler.py:336-340: inv_scale = float(1 / double(scale))
    return scale != nullptr ? static_cast<float>(1.0 / static_cast<double>(*scale)) : 1.0f;
}

// ---------------------------------------------------------------------------
// finalize: total norm, clip coefficient, found_inf
// ---------------------------------------------------------------------------

// Sums the n partials in one work-group of kBlock threads, in an order that
// depends on n only: thread j adds partials j, j + 512, j + 1024, ... in
// turn (four loads in flight), then the fixed wave/LDS tree of block_reduce.
// Thread 0 writes the norm, the clip coefficient and found_inf.  (Folding
// this into pass 1's last work-group, through a device-scope counter and
// release fence in every work-group, measured 2.3x slower for the norm pass
// on the 8.2B set and 1.9x on GPT-2-small than this separate launch.)
__device__ __forceinline__ void finalize_core(const Partial* partials, int64_t n, const FinalizeArgs& a) {
    double s = 0.0;
    uint32_t f = 0;
    int64_t i = threadIdx.x;
    for (; i + 3 * kBlock < n; i += 4 * kBlock) {
        const Partial q0 = partials[i], q1 = partials[i + kBlock], q2 = partials[i + 2 * kBlock], q3 = partials[i + 3 * kBlock];
        s += q0.sumsq;
        s += q1.sumsq;
        s += q2.sumsq;
        s += q3.sumsq;
        f |= q0.nonfinite | q1.nonfinite | q2.nonfinite | q3.nonfinite;
    }
    for (; i < n; i += kBlock) {
        s += partials[i].sumsq;
        f |= partials[i].nonfinite;
    }
    block_reduce<kBlock>(s, f);
    if (threadIdx.x != 0) return;
    // Norm of the stacked per-tensor norms = sqrt of the total sum of squares
    // (clip_grad.py:96-108).  A sum beyond the fp32 range overflows to inf as
    // torch's fp32 accumulation does.
    float norm;
    if (isnan(s)) norm = __builtin_nanf("");
    else if (isinf(static_cast<float>(s))) norm = __builtin_inff();
    else norm = static_cast<float>(sqrt(s));
    if (a.norm_out) *a.norm_out = norm;
    if (a.norm_out && a.win) {
        a.win->norm_last = norm;
        const float m = a.win->norm_max;
        a.win->norm_max = (isnan(m) || isnan(norm)) ? __builtin_nanf("") : fmaxf(m, norm);
    }
    if (a.coef_out) {
        // clip_grad.py:165-169 -> reciprocal(norm + 1e-6) * max_norm, clamp(max=1);
        // NaN propagates through the clamp
        const float d = norm + 1e-6f;
        const float r = 1.0f / d;
        float c = r * static_cast<float>(a.max_norm);
        if (!isnan(c) && c > 1.0f) c = 1.0f;
        *a.coef_out = c;
    }
    if (a.found_inf_out) *a.found_inf_out = f ? 1.0f : 0.0f;
}

__global__ void __launch_bounds__(kBlock) finalize_kernel(const Partial* partials, int64_t n, const FinalizeArgs a) {
    finalize_core(partials, n, a);
}

// ---------------------------------------------------------------------------
// tickets: the last work-group of a folded pass does the follow-on work
// ---------------------------------------------------------------------------

// Pass 1 (folded): called by thread 0 of each work-group after its partial's
// atomic stores.  The add is an agent-scope release, so the partial is visible
// before any later ticket is taken; the holder of the last ticket
// (total - 1) issues an agent-scope acquire fence, which synchronizes with
// every earlier work-group's release (the adds form one release sequence),
// before the finalize reads the partials.  This is ordering by the HIP memory
// model.  On gfx950 the release is a write-back of this XCD's L2 dirty lines
// (buffer_wbl2: pass 1 writes nothing else, so there are none to write) and a
// wait; measured on MI355X it leaves the folded pass 1 within 0.3 us of the
// form without it.  Returns the ticket, 0 .. total - 1.
__device__ __forceinline__ uint32_t fetch_ticket_release(uint32_t* ticket, uint32_t total) {
    const uint32_t t = __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    if (t + 1 == total) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    return t;
}

// Pass 2 (folded): called by the lead thread of each work-group of a tensor
// after it read the tensor's step count; the holder of the last ticket writes
// the advanced count.  What must hold is that no work-group reads the count
// after the last ticket's holder wrote it.  This relies on gfx950's execution
// order rather than on a release/acquire pair: the fence keeps the compiler
// from moving the count's load below the add, and s_waitcnt(0) holds the wave
// until that load has returned its value into a register, so the read is
// complete before this work-group's ticket exists and no later write can reach
// it.  An agent-scope release here (the form pass 1 uses) writes back the
// XCD's L2 dirty lines, which in pass 2 are the other work-groups' parameter
// and moment stores: measured on MI355X it made the folded pass 2 1.6x slower
// on the 0.8M-parameter MiniGPT set (8.3 -> 13.5 us) and 3.9x on 2M elements
// in 16 tensors (14.9 -> 57.5 us).
__device__ __forceinline__ uint32_t fetch_ticket_after_read(uint32_t* ticket) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // no earlier access moves below this point
    __builtin_amdgcn_s_waitcnt(0);                         // every earlier access of this wave has completed
    return __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// By the holder of the last ticket: every other ticket is taken, so the
// counter starts the next launch at zero.
__device__ __forceinline__ void reset_ticket(uint32_t* ticket) {
    __hip_atomic_store(ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// pass 1: unscale + non-finite flag + sum of squares
// ---------------------------------------------------------------------------

// NT: nontemporal gradient loads (sets larger than the Infinity Cache).
// FOLD: small plans; the last work-group also runs the finalize.
template <typename GT, bool NT, bool FOLD>
__global__ void __launch_bounds__(kBlock) norm_kernel(const NormArgs a) {
    // work-group slot r (XCD-remapped) sums pass-1 chunk r of its class into
    // partial r: the partials' order does not depend on the remapping
    double acc = 0.0;
    uint32_t bad = 0;
    const uint32_t slot = xcd_item<kXcdMapNorm>(blockIdx.x, gridDim.x);
    const Chunk ck = a.chunks[a.chunk_begin + slot];
    const GT* __restrict__ g = static_cast<const GT*>(a.grads[ck.tensor]);
    if (g != nullptr) {
        const int64_t numel = a.tensors[ck.tensor].numel;
        const int64_t start = static_cast<int64_t>(ck.index) * a.chunk_elems;
        norm_chunk<GT, NT>(g + start, min(a.chunk_elems, numel - start), inv_scale_of(a.scale), a.scale != nullptr, acc,
                           bad);
    }
    block_reduce<kBlock>(acc, bad);
    if constexpr (!FOLD) {
        if (threadIdx.x == 0) {
            Partial p;
            p.sumsq = acc;
            p.nonfinite = bad;
            p.pad = 0;
            a.partials[a.partial_base + slot] = p;
        }
    } else {
        __shared__ bool last;
        if (threadIdx.x == 0) {
            Partial* p = a.partials + a.partial_base + slot;
            __hip_atomic_store(&p->sumsq, acc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&p->nonfinite, bad, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            last = fetch_ticket_release(a.ticket, a.total) + 1 == a.total;
            if (last) reset_ticket(a.ticket);
        }
        __syncthreads();
        if (last) {
            // thread 0 acquired; every wave of this work-group drops its
            // cached lines of the partials before reading them
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            finalize_core(a.partials, a.total, a.fin);
        }
    }
}

// Pass 1 over one flat gradient buffer: work-group r sums elements
// [r * kNormChunk, (r + 1) * kNormChunk) into partial r, the chunks and
// partials a one-tensor plan has.
template <typename GT, bool NT>
__global__ void __launch_bounds__(kBlock)
    norm_flat_kernel(const GT* __restrict__ g, int64_t n, const float* scale, Partial* partials) {
    double acc = 0.0;
    uint32_t bad = 0;
    const int64_t start = static_cast<int64_t>(blockIdx.x) * kNormChunk;
    norm_chunk<GT, NT>(g + start, min(kNormChunk, n - start), inv_scale_of(scale), scale != nullptr, acc, bad);
    block_reduce<kBlock>(acc, bad);
    if (threadIdx.x == 0) {
        Partial p;
        p.sumsq = acc;
        p.nonfinite = bad;
        p.pad = 0;
        partials[blockIdx.x] = p;
    }
}

// ---------------------------------------------------------------------------
// prologue: step counts and each tensor's constants for pass 2
// ---------------------------------------------------------------------------

// The fp32 constants of one tensor's update this step, formed once per tensor
// by the prologue and read by every pass-2 work-group of that tensor with
// scalar loads.
struct TensorConst {
    float inv, coef, decay, w1, w1m1, b2, w2, bc2s, eps, nss;
    uint32_t flags;  // kc* bits below
    uint32_t pad;
};
static_assert(sizeof(TensorConst) == 48, "two scalar loads per record");
constexpr uint32_t kcSkip = 1, kcUnscale = 2, kcClip = 4, kcDecay = 8, kcSmall = 16, kcMaximize = 32;

struct PrologueArgs {
    void* const* grads;
    const DevTensor* tensors;
    float* steps;
    TensorConst* consts;
    const double* bc;
    int64_t bc_cap;
    const float* scale;            // nullable
    const float* coef;             // nullable
    const float* found_inf;        // nullable
    Window* win;                   // nullable
    int* flags;                    // set to 1 when a tensor's bias corrections were computed here
    const GroupConst* groups_dev;  // nullable: group records read from device memory at run time
    int32_t n;
    int32_t pad;
    GroupConst groups[MGOPT_MAX_GROUPS];
};

__device__ __forceinline__ void count_window(Window* win, bool skip) {
    if (win == nullptr) return;
    if (skip) win->skipped += 1u;
    else win->taken += 1u;
}

// (1 - beta1**t, (1 - beta2**t) ** 0.5) for step count t (adam.py:529-536).
// Integer counts inside the host table read the host's values (Python's
// float ** of the same expressions, so bit-identical to the CPU path); entry
// 0 of a group's row holds the betas the row was built for.  Any other count
// -- one written into the state in place, a non-integer count, a graph replay
// beyond the table -- or betas other than the row's (a device record changed
// between replays) is evaluated here in double with the same expressions; the
// device pow can differ from the host's by an ulp of the double, which reaches
// the fp32 constants only when it crosses one of their rounding boundaries.
__device__ __forceinline__ void bias_corrections(const PrologueArgs& a, const GroupConst& G, int32_t group, float count,
                                                 double& bc1, double& bc2s) {
    const double t = static_cast<double>(count);
    const double* row = a.bc + static_cast<int64_t>(group) * a.bc_cap * 2;
    if (t >= 1.0 && t < static_cast<double>(a.bc_cap) && t == floor(t) && row[0] == G.beta1 && row[1] == G.beta2) {
        const double* bc = row + static_cast<int64_t>(t) * 2;
        bc1 = bc[0];
        bc2s = bc[1];
        return;
    }
    bc1 = 1.0 - pow(G.beta1, t);
    bc2s = sqrt(1.0 - pow(G.beta2, t));
    *a.flags = 1;
}

// The constants of tensor i for this step (kcSkip when the step is skipped or
// the tensor has no gradient; then `count` is its unchanged step count).
// adam.py:414 (step_t += 1) runs only when the step is taken: GradScaler
// skips optimizer.step() on found_inf (grad_scaler.py:348-358); the fused path
// subtracts found_inf back (adam.py:877-899).  Tensors without grad keep their
// count (adam.py:153).  The constants follow adam.py:416-547 and
// grad_scaler.py:336-340 in double, each rounded to fp32 once, as torch's CPU
// path forms them.
__device__ __forceinline__ TensorConst tensor_const(const PrologueArgs& a, int32_t i, bool skip, float& count) {
    TensorConst c{};
    if (skip || a.grads[i] == nullptr) {
        c.flags = kcSkip;
        count = a.steps[i];
        return c;
    }
    count = a.steps[i] + 1.0f;
    const int32_t group = a.tensors[i].group;
    const GroupConst G = a.groups_dev != nullptr ? a.groups_dev[group] : a.groups[group];
    double bc1, bc2s;
    bias_corrections(a, G, group, count, bc1, bc2s);
    c.inv = a.scale != nullptr ? static_cast<float>(1.0 / static_cast<double>(*a.scale)) : 1.0f;
    c.coef = a.coef != nullptr ? *a.coef : 1.0f;
    c.decay = static_cast<float>(1.0 - G.lr * G.wd);
    c.w1 = static_cast<float>(1.0 - G.beta1);
    c.w1m1 = c.w1 - 1.0f;
    c.b2 = static_cast<float>(G.beta2);
    c.w2 = static_cast<float>(1.0 - G.beta2);
    c.bc2s = static_cast<float>(bc2s);
    c.eps = static_cast<float>(G.eps);
    c.nss = static_cast<float>(-(G.lr / bc1));
    c.flags = (a.scale != nullptr ? kcUnscale : 0u) | (a.coef != nullptr ? kcClip : 0u) | (G.wd != 0.0 ? kcDecay : 0u) |
              (fabsf(c.w1) < 0.5f ? kcSmall : 0u) | (G.maximize != 0 ? kcMaximize : 0u);
    return c;
}

// One thread per tensor: the step counts and the constants pass 2 reads.
// (Large plans keep this kernel: advancing the counts from pass 2 through a
// device-scope ticket in every work-group measured 2.5x slower for pass 2 on
// GPT-2-small.  Small plans fold it into pass 2, adamw_fold_kernel.)
__global__ void __launch_bounds__(kBlock) prologue_kernel(const PrologueArgs a) {
    const bool skip = a.found_inf != nullptr && *a.found_inf != 0.0f;
    if (blockIdx.x == 0 && threadIdx.x == 0) count_window(a.win, skip);
    const int32_t i = blockIdx.x * kBlock + threadIdx.x;
    if (i >= a.n) return;
    float count;
    const TensorConst c = tensor_const(a, i, skip, count);
    if (!(c.flags & kcSkip)) a.steps[i] = count;
    a.consts[i] = c;
}

// ---------------------------------------------------------------------------
// pass 2: fused unscale + clip + AdamW
// ---------------------------------------------------------------------------

struct AdamArgs {
    const DevTensor* tensors;
    const Chunk* chunks;
    void* const* grads;
    const TensorConst* consts;
    int64_t chunk_elems;
    uint32_t chunk_begin;
    int32_t writeback;
};

struct ElemConst {
    float inv, coef, decay, w1, w1m1, b2, w2, bc2s, eps, nss;
    bool unscale, clip, do_decay, small, maximize;
};

// One element of the step, in torch's order:
//   grad_scaler.py:280-284  g = g * inv_scale              (unscale_)
//   clip_grad.py:174        g = g * clip_coef              (clip_grad_norm_)
//   adam.py:397             g = -g                         (maximize)
//   adam.py:416-419         p = p * float(1 - lr*wd)
//   adam.py:457             m = lerp(m, g, float(1-beta1)) as ATen's vector lerp
//   adam.py:476             v = fma(float(1-beta2)*g, g, v*float(beta2))
//   adam.py:542             d = sqrt(v) / float(sqrt(bc2)) + float(eps)
//   adam.py:547             p = p + (float(-lr/bc1) * m) / d
__device__ __forceinline__ float adam_elem(float g, float& p, float& m, float& v, const ElemConst& c) {
    if (c.unscale) g = g * c.inv;
    if (c.clip) g = g * c.coef;
    const float gc = g;
    if (c.maximize) g = -g;
    if (c.do_decay) p = p * c.decay;
    const float diff = g - m;
    m = c.small ? __builtin_fmaf(c.w1, diff, m) : __builtin_fmaf(c.w1m1, diff, g);
    v = v * c.b2;
    v = __builtin_fmaf(c.w2 * g, g, v);
    float d = __builtin_sqrtf(v);
    d = d / c.bc2s;
    d = d + c.eps;
    float u = c.nss * m;
    u = u / d;
    p = p + u;
    return gc;
}

template <int LOWP>
struct LowpStore;
template <>
struct LowpStore<MGOPT_NONE> {
    template <int W>
    static __device__ __forceinline__ void store(void*, const float*) {}
    static __device__ __forceinline__ void store1(void*, float) {}
};
template <>
struct LowpStore<MGOPT_BF16> {
    template <int W>
    static __device__ __forceinline__ void store(void* p, const float* x) {
        uint32_t w[W / 2];
#pragma unroll
        for (int k = 0; k < W / 2; ++k)
            w[k] = static_cast<uint32_t>(f32_to_bf16_rne(x[2 * k])) | (static_cast<uint32_t>(f32_to_bf16_rne(x[2 * k + 1])) << 16);
        if constexpr (W == 4) st8<kNtStore>(p, u32x2{w[0], w[1]});
        else st16<kNtStore>(static_cast<float*>(p), __builtin_bit_cast(f32x4, u32x4{w[0], w[1], w[2], w[3]}));
    }
    static __device__ __forceinline__ void store1(void* p, float x) { *static_cast<uint16_t*>(p) = f32_to_bf16_rne(x); }
};
template <>
struct LowpStore<MGOPT_F16> {
    template <int W>
    static __device__ __forceinline__ void store(void* p, const float* x) {
        uint32_t w[W / 2];
#pragma unroll
        for (int k = 0; k < W / 2; ++k) {
            const _Float16 a = static_cast<_Float16>(x[2 * k]), b = static_cast<_Float16>(x[2 * k + 1]);
            uint16_t ha, hb;
            std::memcpy(&ha, &a, 2);
            std::memcpy(&hb, &b, 2);
            w[k] = static_cast<uint32_t>(ha) | (static_cast<uint32_t>(hb) << 16);
        }
        if constexpr (W == 4) st8<kNtStore>(p, u32x2{w[0], w[1]});
        else st16<kNtStore>(static_cast<float*>(p), __builtin_bit_cast(f32x4, u32x4{w[0], w[1], w[2], w[3]}));
    }
    static __device__ __forceinline__ void store1(void* p, float x) { *static_cast<_Float16*>(p) = static_cast<_Float16>(x); }
};

// kVec consecutive elements of one tensor through pass 2: load() issues the
// memory reads, finish() does the arithmetic and the writes.
template <typename GT>
struct Group {
    static constexpr int W = kVec;
    float g[W];
    f32x4 p[W / 4], m[W / 4], v[W / 4];

    __device__ __forceinline__ void load(const GT* G, const float* P, const float* M, const float* V, int64_t e) {
        load_grad<GT, kNtLoad, W>(G + e, g);
#pragma unroll
        for (int k = 0; k < W / 4; ++k) {
            p[k] = ld16<kNtLoad>(P + e + 4 * k);
            m[k] = ld16<kNtLoad>(M + e + 4 * k);
            v[k] = ld16<kNtLoad>(V + e + 4 * k);
        }
    }

    template <int LOWP>
    __device__ __forceinline__ void finish(GT* G, float* P, float* M, float* V, void* L, int64_t e, const ElemConst& c,
                                           bool wb) {
        float pf[W], mf[W], vf[W], gc[W];
#pragma unroll
        for (int k = 0; k < W / 4; ++k) {
            pf[4 * k] = p[k].x; pf[4 * k + 1] = p[k].y; pf[4 * k + 2] = p[k].z; pf[4 * k + 3] = p[k].w;
            mf[4 * k] = m[k].x; mf[4 * k + 1] = m[k].y; mf[4 * k + 2] = m[k].z; mf[4 * k + 3] = m[k].w;
            vf[4 * k] = v[k].x; vf[4 * k + 1] = v[k].y; vf[4 * k + 2] = v[k].z; vf[4 * k + 3] = v[k].w;
        }
#pragma unroll
        for (int k = 0; k < W; ++k) gc[k] = adam_elem(g[k], pf[k], mf[k], vf[k], c);
#pragma unroll
        for (int k = 0; k < W / 4; ++k) {
            st16<kNtStore>(P + e + 4 * k, f32x4{pf[4 * k], pf[4 * k + 1], pf[4 * k + 2], pf[4 * k + 3]});
            st16<kNtStore>(M + e + 4 * k, f32x4{mf[4 * k], mf[4 * k + 1], mf[4 * k + 2], mf[4 * k + 3]});
            st16<kNtStore>(V + e + 4 * k, f32x4{vf[4 * k], vf[4 * k + 1], vf[4 * k + 2], vf[4 * k + 3]});
        }
        if constexpr (LOWP != MGOPT_NONE) LowpStore<LOWP>::template store<W>(static_cast<uint16_t*>(L) + e, pf);
        if (wb) {
#pragma unroll
            for (int k = 0; k < W / 4; ++k) {
                Vec4<GT> go;
#pragma unroll
                for (int j = 0; j < 4; ++j) go.e[j] = GradIO<GT>::from_f32(gc[4 * k + j]);
                store4(G + e + 4 * k, go);
            }
        }
    }
};

__device__ __forceinline__ ElemConst elem_const(const TensorConst& k) {
    ElemConst c;
    c.inv = k.inv;
    c.coef = k.coef;
    c.decay = k.decay;
    c.w1 = k.w1;
    c.w1m1 = k.w1m1;
    c.b2 = k.b2;
    c.w2 = k.w2;
    c.bc2s = k.bc2s;
    c.eps = k.eps;
    c.nss = k.nss;
    c.unscale = (k.flags & kcUnscale) != 0;
    c.clip = (k.flags & kcClip) != 0;
    c.do_decay = (k.flags & kcDecay) != 0;
    c.small = (k.flags & kcSmall) != 0;
    c.maximize = (k.flags & kcMaximize) != 0;
    return c;
}

// The update of one pass-2 chunk of a tensor that has a gradient.
template <typename GT, int LOWP>
__device__ __forceinline__ void adamw_chunk(const AdamArgs& a, const Chunk ck, GT* __restrict__ g, const TensorConst& k) {
    const DevTensor T = a.tensors[ck.tensor];
    ElemConst c;
    c.inv = k.inv;
    c.coef = k.coef;
    c.decay = k.decay;
    c.w1 = k.w1;
    c.w1m1 = k.w1m1;
    c.b2 = k.b2;
    c.w2 = k.w2;
    c.bc2s = k.bc2s;
    c.eps = k.eps;
    c.nss = k.nss;
    c.unscale = (k.flags & kcUnscale) != 0;
    c.clip = (k.flags & kcClip) != 0;
    c.do_decay = (k.flags & kcDecay) != 0;
    c.small = (k.flags & kcSmall) != 0;
    c.maximize = (k.flags & kcMaximize) != 0;

    const int64_t start = static_cast<int64_t>(ck.index) * a.chunk_elems;
    const int64_t len = min(a.chunk_elems, T.numel - start);
    const ChunkPtrs cp = chunk_ptrs(T, ck.index, a.chunk_elems);
    float* __restrict__ P = cp.p;
    float* __restrict__ M = cp.m;
    float* __restrict__ V = cp.v;
    g += start;
    void* L = nullptr;
    if constexpr (LOWP != MGOPT_NONE) L = static_cast<uint16_t*>(T.lowp) + start;
    const bool wb = a.writeback != 0;

    int64_t done = 0;
    const bool vec = aligned(P, 16) && aligned(M, 16) && aligned(V, 16) && aligned(g, sizeof(GT) * kVec) &&
                     (LOWP == MGOPT_NONE || aligned(L, 2 * kVec));
    if (vec) {
        // four elements per thread per access; kUnroll accesses issued before
        // the first one is consumed, to keep more bytes in flight per wave
        const int64_t nvec = len / kVec;
        int64_t i = threadIdx.x;
        for (; i + (kUnroll - 1) * kAdamBlock < nvec; i += kUnroll * kAdamBlock) {
            Group<GT> q[kUnroll];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) q[u].load(g, P, M, V, (i + u * kAdamBlock) * kVec);
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) q[u].template finish<LOWP>(g, P, M, V, L, (i + u * kAdamBlock) * kVec, c, wb);
        }
        for (; i < nvec; i += kAdamBlock) {
            Group<GT> q;
            q.load(g, P, M, V, i * kVec);
            q.template finish<LOWP>(g, P, M, V, L, i * kVec, c, wb);
        }
        done = nvec * kVec;
    }
    for (int64_t i = done + threadIdx.x; i < len; i += kAdamBlock) {
        float p = P[i], m = M[i], v = V[i];
        const float gc = adam_elem(GradIO<GT>::to_f32(g[i]), p, m, v, c);
        P[i] = p;
        M[i] = m;
        V[i] = v;
        if constexpr (LOWP != MGOPT_NONE) LowpStore<LOWP>::store1(static_cast<uint16_t*>(L) + i, p);
        if (wb) g[i] = GradIO<GT>::from_f32(gc);
    }
}

template <typename GT, int LOWP>
__global__ void __launch_bounds__(kAdamBlock) adamw_kernel(const AdamArgs a) {
    const uint32_t cidx = a.chunk_begin + xcd_item<kXcdMapAdam>(blockIdx.x, gridDim.x);
    const Chunk ck = a.chunks[cidx];
    const TensorConst k = a.consts[ck.tensor];
    if (k.flags & kcSkip) return;  // a skipped step, or no gradient this step
    adamw_chunk<GT, LOWP>(a, ck, static_cast<GT*>(a.grads[ck.tensor]), k);
}

// Pass 2 of a small plan with the prologue folded in.  Every thread issues
// the loads of its first element group while the first lane of the last wave
// (no data in a 1,024-element chunk) forms the tensor's constants from the
// tensor's current step count (read, not written) and, when the tensor has
// several chunks, takes one of the tensor's tickets; the work-group of the
// tensor's last ticket (or of its only chunk) advances the count once every
// work-group of the tensor has read it.
template <typename GT, int LOWP>
__global__ void __launch_bounds__(kAdamBlock)
    adamw_fold_kernel(const AdamArgs a, const PrologueArgs pa, uint32_t* tickets) {
    const Chunk ck = a.chunks[a.chunk_begin + blockIdx.x];
    const bool skip = pa.found_inf != nullptr && *pa.found_inf != 0.0f;
    const DevTensor T = a.tensors[ck.tensor];
    GT* __restrict__ g = static_cast<GT*>(a.grads[ck.tensor]);
    const int64_t start = static_cast<int64_t>(ck.index) * a.chunk_elems;
    const int64_t len = min(a.chunk_elems, T.numel - start);
    const ChunkPtrs cp = chunk_ptrs(T, ck.index, a.chunk_elems);
    float* __restrict__ P = cp.p;
    float* __restrict__ M = cp.m;
    float* __restrict__ V = cp.v;
    void* L = nullptr;
    if constexpr (LOWP != MGOPT_NONE) L = static_cast<uint16_t*>(T.lowp) + start;
    if (g != nullptr) g += start;
    const bool vec = g != nullptr && aligned(P, 16) && aligned(M, 16) && aligned(V, 16) &&
                     aligned(g, sizeof(GT) * kVec) && (LOWP == MGOPT_NONE || aligned(L, 2 * kVec));
    const int64_t nvec = vec ? len / kVec : 0;
    const bool first = threadIdx.x < nvec;
    Group<GT> q;
    if (first) q.load(g, P, M, V, threadIdx.x * kVec);

    __shared__ TensorConst kc;
    constexpr uint32_t kLead = kAdamBlock - 64;  // first lane of the last wave
    const uint32_t nch = static_cast<uint32_t>((T.numel + a.chunk_elems - 1) / a.chunk_elems);
    uint32_t t = 0;
    float count = 0.0f;
    if (threadIdx.x == kLead) {
        kc = tensor_const(pa, static_cast<int32_t>(ck.tensor), skip, count);
        if (nch > 1) t = fetch_ticket_after_read(tickets + ck.tensor * kTicketStride);
    }
    __syncthreads();
    const TensorConst k = kc;
    if (!(k.flags & kcSkip)) {
        const ElemConst c = elem_const(k);
        const bool wb = a.writeback != 0;
        if (first) q.template finish<LOWP>(g, P, M, V, L, threadIdx.x * kVec, c, wb);
        for (int64_t i = threadIdx.x + kAdamBlock; i < nvec; i += kAdamBlock) {
            Group<GT> r;
            r.load(g, P, M, V, i * kVec);
            r.template finish<LOWP>(g, P, M, V, L, i * kVec, c, wb);
        }
        for (int64_t i = nvec * kVec + threadIdx.x; i < len; i += kAdamBlock) {
            float p = P[i], m = M[i], v = V[i];
            const float gc = adam_elem(GradIO<GT>::to_f32(g[i]), p, m, v, c);
            P[i] = p;
            M[i] = m;
            V[i] = v;
            if constexpr (LOWP != MGOPT_NONE) LowpStore<LOWP>::store1(static_cast<uint16_t*>(L) + i, p);
            if (wb) g[i] = GradIO<GT>::from_f32(gc);
        }
    }
    if (threadIdx.x != kLead) return;
    if (a.chunk_begin + blockIdx.x == 0) count_window(pa.win, skip);  // once per step, whatever the class launches
    if (nch > 1) {
        if (t + 1 != nch) return;
        reset_ticket(tickets + ck.tensor * kTicketStride);
    }
    if (!(k.flags & kcSkip)) pa.steps[ck.tensor] = count;
}

// ---------------------------------------------------------------------------
// GradScaler.update
// ---------------------------------------------------------------------------

struct FoundList {
    const float* p[8];
};

// grad_scaler.py:517-536: found_inf_combined = sum of the per-optimizer flags
// (fp32, in order); torch._amp_update_scale_ then backs off on any nonzero
// value (NaN included) or counts a good step, growing after growth_interval of
// them unless the product overflows.  Factor products in double, rounded once.
__global__ void scaler_kernel(float* scale, int32_t* tracker, FoundList fl, int32_t n, double growth, double backoff,
                              int32_t interval) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    float fi = *fl.p[0];
    for (int k = 1; k < n; ++k) fi = fi + *fl.p[k];
    if (fi != 0.0f) {
        *scale = static_cast<float>(static_cast<double>(*scale) * backoff);
        *tracker = 0;
    } else {
        const int32_t ok = *tracker + 1;
        if (ok == interval) {
            const float ns = static_cast<float>(static_cast<double>(*scale) * growth);
            if (isfinite(ns)) *scale = ns;
            *tracker = 0;
        } else {
            *tracker = ok;
        }
    }
}

// ---------------------------------------------------------------------------
// grad scaling for the stand-alone clip path, master sync, synthetic data
// ---------------------------------------------------------------------------

template <typename GT>
__global__ void __launch_bounds__(kBlock)
    scale_grads_kernel(const DevTensor* tensors, const Chunk* chunks, void* const* grads, const float* coefp,
                       int64_t chunk_elems, uint32_t chunk_begin) {
    const Chunk ck = chunks[chunk_begin + blockIdx.x];
    GT* g = static_cast<GT*>(grads[ck.tensor]);
    if (g == nullptr) return;
    const float coef = *coefp;
    const int64_t start = static_cast<int64_t>(ck.index) * chunk_elems;
    const int64_t len = min(chunk_elems, tensors[ck.tensor].numel - start);
    g += start;
    int64_t done = 0;
    if (aligned(g, sizeof(GT) * 4)) {
        // four elements per thread per access, as torch's vectorised _foreach_mul_ reads them
        const int64_t nvec = len / 4;
        for (int64_t i = threadIdx.x; i < nvec; i += kBlock) {
            Vec4<GT> q = load4(g + 4 * i);
#pragma unroll
            for (int k = 0; k < 4; ++k) q.e[k] = GradIO<GT>::from_f32(GradIO<GT>::to_f32(q.e[k]) * coef);
            store4(g + 4 * i, q);
        }
        done = nvec * 4;
    }
    for (int64_t i = done + threadIdx.x; i < len; i += kBlock) g[i] = GradIO<GT>::from_f32(GradIO<GT>::to_f32(g[i]) * coef);
}

template <typename LT>
__global__ void __launch_bounds__(kBlock)
    sync_master_kernel(const DevTensor* tensors, const Chunk* chunks, int64_t chunk_elems, uint32_t chunk_begin) {
    const Chunk ck = chunks[chunk_begin + blockIdx.x];
    const DevTensor T = tensors[ck.tensor];
    const int64_t start = static_cast<int64_t>(ck.index) * chunk_elems;
    const int64_t len = min(chunk_elems, T.numel - start);
    const LT* l = static_cast<const LT*>(T.lowp) + start;
    float* p = chunk_ptrs(T, ck.index, chunk_elems).p;
    int64_t done = 0;
    if (aligned(l, sizeof(LT) * 4) && aligned(p, 16)) {
        const int64_t nvec = len / 4;
        for (int64_t i = threadIdx.x; i < nvec; i += kBlock) {
            const Vec4<LT> q = load4(l + 4 * i);
            store4(p + 4 * i, Vec4<float>{{GradIO<LT>::to_f32(q.e[0]), GradIO<LT>::to_f32(q.e[1]),
                                           GradIO<LT>::to_f32(q.e[2]), GradIO<LT>::to_f32(q.e[3])}});
        }
        done = nvec * 4;
    }
    for (int64_t i = done + threadIdx.x; i < len; i += kBlock) p[i] = GradIO<LT>::to_f32(l[i]);
}

__device__ __host__ __forceinline__ uint64_t mix64(uint64_t x) {
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}
constexpr uint64_t kGamma = 0x9E3779B97F4A7C15ull;

template <typename T>
__global__ void __launch_bounds__(kBlock)
    synth_kernel(T* dst, int64_t n, uint64_t key, double k, uint64_t tail_every, double tail_mult) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) {
        const uint64_t h = mix64(key + (static_cast<uint64_t>(i) + 1ull) * kGamma);
        const int32_t s = static_cast<int32_t>(h & 0xFFFFu) + static_cast<int32_t>((h >> 16) & 0xFFFFu) +
                          static_cast<int32_t>((h >> 32) & 0xFFFFu) + static_cast<int32_t>(h >> 48) - 131070;
        double x = static_cast<double>(s) * k;
        if (tail_every) {
            const uint64_t h2 = mix64(h ^ 0xD1B54A32D192ED03ull);
            if (h2 % tail_every == 0) x = x * tail_mult;
        }
        dst[i] = GradIO<T>::from_f32(static_cast<float>(x));
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(static_cast<int>(e), std::string(what) + ": " + hipGetErrorString(e));
}

#define HIP_TRY(expr)                                   \
    do {                                                \
        hipError_t _e = (expr);                         \
        if (_e != hipSuccess) return hip_fail(_e, #expr); \
    } while (0)

// Runs the body with the plan's device current, restoring the caller's.
struct DeviceGuard {
    int prev = -1;
    bool switched = false;
    explicit DeviceGuard(int dev) {
        // restores the caller's device only when it had to switch: the common
        // case (the plan's device is current) costs one hipGetDevice
        if (hipGetDevice(&prev) == hipSuccess && prev != dev) switched = hipSetDevice(dev) == hipSuccess;
    }
    ~DeviceGuard() {
        if (switched) (void)hipSetDevice(prev);
    }
};

}  // namespace

struct mgopt_plan {
    int device = 0;
    int32_t n_tensors = 0;
    int32_t n_groups = 0;
    int64_t chunk_elems = 0;
    int64_t n_chunks = 0;
    DevTensor* d_tensors = nullptr;
    Chunk* d_chunks = nullptr;       // pass 2 (and helpers): chunk_elems elements per chunk
    Chunk* d_norm_chunks = nullptr;  // pass 1: kNormChunk elements per chunk
    void** d_grads = nullptr;
    Partial* d_partials = nullptr;
    int* d_flags = nullptr;          // set by the prologue when it computed bias corrections on the device
    TensorConst* d_consts = nullptr;  // each tensor's constants for the coming pass 2 (written by the prologue)
    float* d_steps = nullptr;
    Window* d_window = nullptr;  // caller-owned, optional
    struct Class {
        int32_t grad_dtype;
        int32_t lowp_dtype;
        uint32_t begin;
        uint32_t count;
        uint32_t norm_begin;    // first entry of the class in the pass-1 chunk table
        uint32_t norm_count;    // pass-1 chunks (= work-groups = partials) of the class
        uint32_t partial_base;  // first partial slot of the class
    };
    int64_t n_partials = 0;
    int64_t grad_bytes = 0;  // all gradients of the plan, for pass 1's load policy
    int64_t norm_chunk = kNormChunk;  // elements per pass-1 chunk
    bool fold = false;                // small plan: three kernels per step
    uint32_t* d_tickets = nullptr;    // [0] pass 1, [kTicketStride * (1 + i)] tensor i in pass 2 (folded form only)
    std::vector<Class> classes;
    bool has_state = false;  // false: grads-only plan (norm and grad scaling only)
    std::vector<const void*> cached;
    bool grads_uploaded = false;
    void* staging[kStagingSlots] = {};
    hipEvent_t staging_ev[kStagingSlots] = {};
    bool staging_used[kStagingSlots] = {};
    int slot = 0;
};

namespace {

int launch_check(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, what);
    return 0;
}

template <typename GT>
int launch_norm(const mgopt_plan* P, const mgopt_plan::Class& c, const float* scale, const FinalizeArgs& fin,
                hipStream_t s) {
    // partial slot = partial_base + chunk position, so the pieces fill the
    // class's partials exactly as one launch would
    for (uint64_t done = 0; done < c.norm_count; done += kMaxGroupsPerLaunch) {
        const uint32_t n = static_cast<uint32_t>(std::min<uint64_t>(c.norm_count - done, kMaxGroupsPerLaunch));
        NormArgs a{P->d_tensors, P->d_norm_chunks, P->d_grads, P->d_partials, scale, P->norm_chunk,
                   static_cast<uint32_t>(c.norm_begin + done), n, static_cast<uint32_t>(c.partial_base + done),
                   P->d_tickets, static_cast<uint32_t>(P->n_partials), fin};
        if (P->fold)
            hipLaunchKernelGGL((norm_kernel<GT, false, true>), dim3(n), dim3(kBlock), 0, s, a);
        else if (P->grad_bytes <= kCachedGradBytes)
            hipLaunchKernelGGL((norm_kernel<GT, false, false>), dim3(n), dim3(kBlock), 0, s, a);
        else
            hipLaunchKernelGGL((norm_kernel<GT, true, false>), dim3(n), dim3(kBlock), 0, s, a);
        if (int rc = launch_check("norm_kernel")) return rc;
    }
    return 0;
}

template <typename GT>
void launch_norm_flat(const void* grads, int64_t n, const float* scale, Partial* part, dim3 grid, hipStream_t s) {
    const GT* g = static_cast<const GT*>(grads);
    if (n * static_cast<int64_t>(sizeof(GT)) <= kCachedGradBytes)
        hipLaunchKernelGGL((norm_flat_kernel<GT, false>), grid, dim3(kBlock), 0, s, g, n, scale, part);
    else
        hipLaunchKernelGGL((norm_flat_kernel<GT, true>), grid, dim3(kBlock), 0, s, g, n, scale, part);
}

// The extra arguments of a folded pass 2.
struct FoldLaunch {
    PrologueArgs pa;
    uint32_t* tickets;  // one per tensor
};

template <typename GT, int LOWP>
int launch_adamw(AdamArgs a, uint32_t count, const FoldLaunch* f, hipStream_t s) {
    if (f != nullptr) {  // small plans: one piece
        hipLaunchKernelGGL((adamw_fold_kernel<GT, LOWP>), dim3(count), dim3(kAdamBlock), 0, s, a, f->pa, f->tickets);
        return launch_check("adamw_fold_kernel");
    }
    const uint32_t begin = a.chunk_begin;
    for (uint64_t done = 0; done < count; done += kMaxGroupsPerLaunch) {
        const uint32_t n = static_cast<uint32_t>(std::min<uint64_t>(count - done, kMaxGroupsPerLaunch));
        a.chunk_begin = static_cast<uint32_t>(begin + done);
        hipLaunchKernelGGL((adamw_kernel<GT, LOWP>), dim3(n), dim3(kAdamBlock), kAdamLds, s, a);
        if (int rc = launch_check("adamw_kernel")) return rc;
    }
    return 0;
}

template <typename GT>
int launch_adamw_lowp(const AdamArgs& a, int32_t lowp, uint32_t count, const FoldLaunch* f, hipStream_t s) {
    switch (lowp) {
        case MGOPT_NONE: return launch_adamw<GT, MGOPT_NONE>(a, count, f, s);
        case MGOPT_BF16: return launch_adamw<GT, MGOPT_BF16>(a, count, f, s);
        case MGOPT_F16: return launch_adamw<GT, MGOPT_F16>(a, count, f, s);
        default: return fail(MGOPT_E_INVALID, "unknown lowp dtype");
    }
}

int dtype_size(int32_t dt) {
    switch (dt) {
        case MGOPT_F32: return 4;
        case MGOPT_F16:
        case MGOPT_BF16: return 2;
        default: return 0;
    }
}

// ---------------------------------------------------------------------------
// allocation-free norm: partials in a static device array
// ---------------------------------------------------------------------------

// Partials of mgopt_grad_norm_noalloc, one per 131,072-element chunk: 1 MiB,
// so one call covers at most 65,536 x 131,072 = 8,589,934,592 elements.  Each
// GPU the library runs on holds its own copy until the process ends, and every
// call on that GPU shares it (calls that overlap on one GPU race).  Every slot
// a call reads is written by the same call, so nothing needs clearing.
constexpr int64_t kScratchPartials = 65536;
static __device__ __align__(256) Partial scratch[kScratchPartials];

constexpr int kMaxDevices = 64;
// The device address of `scratch` on each GPU, looked up once per GPU with
// that GPU current.  Host code passes these addresses, never the symbol itself
// (which names a host-side stand-in).
std::atomic<Partial*> g_scratch_addr[kMaxDevices];

int scratch_on_current_device(Partial** out) {
    int dev = -1;
    HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) return fail(MGOPT_E_LIMIT, "device index above 63");
    Partial* p = g_scratch_addr[dev].load(std::memory_order_acquire);
    if (p == nullptr) {
        void* addr = nullptr;
        HIP_TRY(hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch)));
        p = static_cast<Partial*>(addr);
        g_scratch_addr[dev].store(p, std::memory_order_release);
    }
    *out = p;
    return 0;
}

}  // namespace

extern "C" {

MGOPT_API const char* mgopt_last_error(void) { return g_last_error.c_str(); }

MGOPT_API const char* mgopt_version(void) { return "mgopt 0.2 gfx950"; }

MGOPT_API int mgopt_plan_create(const mgopt_tensor_desc* descs, int32_t n_tensors, int32_t n_groups, float* steps_dev,
                                int64_t chunk_elems, mgopt_plan** out) {
    if (!out) return fail(MGOPT_E_INVALID, "out is NULL");
    *out = nullptr;
    if (n_tensors <= 0 || !descs) return fail(MGOPT_E_INVALID, "empty tensor list");
    if (n_groups <= 0 || n_groups > MGOPT_MAX_GROUPS) return fail(MGOPT_E_LIMIT, "n_groups must be in 1..16");
    if (chunk_elems <= 0 || chunk_elems % 512 != 0 || chunk_elems > (int64_t(1) << 30))
        return fail(MGOPT_E_INVALID, "chunk_elems must be a positive multiple of 512, at most 2^30");

    // Validate and bucket tensors by (grad dtype, lowp dtype): one kernel instance per bucket.
    std::vector<std::vector<int32_t>> buckets(9);
    auto bucket_of = [](int32_t gd, int32_t ld) { return gd * 3 + (ld == MGOPT_NONE ? 0 : (ld == MGOPT_BF16 ? 1 : 2)); };
    std::vector<DevTensor> host_t(n_tensors);
    bool grads_only = false, with_state = false;
    for (int32_t i = 0; i < n_tensors; ++i) {
        const mgopt_tensor_desc& d = descs[i];
        if (d.numel < 0) return fail(MGOPT_E_INVALID, "tensor " + std::to_string(i) + ": negative numel");
        const bool none = !d.param_dev && !d.exp_avg_dev && !d.exp_avg_sq_dev && !d.lowp_dev;
        const bool all = d.param_dev && d.exp_avg_dev && d.exp_avg_sq_dev;
        if (d.numel > 0 && !none && !all)
            return fail(MGOPT_E_INVALID, "tensor " + std::to_string(i) + ": set all of param/exp_avg/exp_avg_sq or none");
        if (d.numel > 0 && none) grads_only = true;
        if (d.numel > 0 && all) with_state = true;
        if (d.group < 0 || d.group >= n_groups) return fail(MGOPT_E_INVALID, "tensor " + std::to_string(i) + ": bad group");
        if (dtype_size(d.grad_dtype) == 0) return fail(MGOPT_E_INVALID, "tensor " + std::to_string(i) + ": bad grad dtype");
        if (d.lowp_dtype != MGOPT_NONE && d.lowp_dtype != MGOPT_BF16 && d.lowp_dtype != MGOPT_F16)
            return fail(MGOPT_E_INVALID, "tensor " + std::to_string(i) + ": bad lowp dtype");
        if ((d.lowp_dtype == MGOPT_NONE) != (d.lowp_dev == nullptr) && d.numel > 0 && all)
            return fail(MGOPT_E_INVALID, "tensor " + std::to_string(i) + ": lowp_dev and lowp_dtype disagree");
        if (d.numel >= (int64_t(1) << 31) * chunk_elems)
            return fail(MGOPT_E_LIMIT, "tensor " + std::to_string(i) + ": too many chunks");
        const int32_t lowp = all ? d.lowp_dtype : MGOPT_NONE;
        uint32_t row_chunks = 0;
        if (d.row_elems != 0) {
            if (d.row_elems < 0 || d.row_elems % chunk_elems != 0 || d.numel % d.row_elems != 0 ||
                d.param_pitch < d.row_elems || d.state_pitch < d.row_elems || !all)
                return fail(MGOPT_E_INVALID, "tensor " + std::to_string(i) +
                                                 ": row_elems must divide numel and be a multiple of chunk_elems, "
                                                 "with pitches of at least row_elems, on a tensor with optimizer state");
            if (d.row_elems / chunk_elems > 0xFFFFFFFFll)
                return fail(MGOPT_E_LIMIT, "tensor " + std::to_string(i) + ": rows of too many chunks");
            row_chunks = static_cast<uint32_t>(d.row_elems / chunk_elems);
        }
        host_t[i] = DevTensor{d.param_dev, all ? d.lowp_dev : nullptr, d.exp_avg_dev, d.exp_avg_sq_dev, d.numel, d.group,
                              row_chunks, d.param_pitch, d.state_pitch};
        buckets[bucket_of(d.grad_dtype, lowp)].push_back(i);
    }
    if (grads_only && with_state) return fail(MGOPT_E_INVALID, "a plan is either grads-only or has optimizer state for every tensor");
    if (with_state && !steps_dev) return fail(MGOPT_E_INVALID, "steps_dev is NULL");

    std::vector<Chunk> chunks, norm_chunks;
    mgopt_plan* P = new mgopt_plan();
    // the folded pass 2 advances a tensor's count from one of its chunks, so a
    // plan with an empty tensor keeps the prologue
    int64_t total_elems = 0, largest = 0;
    bool has_empty = false;
    for (int32_t i = 0; i < n_tensors; ++i) {
        total_elems += descs[i].numel;
        largest = std::max(largest, descs[i].numel);
        has_empty |= descs[i].numel == 0;
    }
    const char* fold_env = std::getenv("MGOPT_FOLD");
    const bool fold_off = fold_env && std::strcmp(fold_env, "0") == 0;
    const bool fold_forced = fold_env && std::strcmp(fold_env, "1") == 0;
    const bool fold_fits = total_elems <= kFoldElems && (largest + chunk_elems - 1) / chunk_elems <= kFoldTensorChunks;
    P->fold = total_elems > 0 && !has_empty && !fold_off && (fold_fits || (fold_forced && total_elems <= kFoldForcedElems));
    P->norm_chunk = P->fold ? kNormChunkFold : kNormChunk;
    P->n_tensors = n_tensors;
    P->n_groups = n_groups;
    P->chunk_elems = chunk_elems;
    P->d_steps = steps_dev;
    P->has_state = with_state;
    for (int b = 0; b < 9; ++b) {
        if (buckets[b].empty()) continue;
        mgopt_plan::Class c;
        c.grad_dtype = b / 3;
        const int l = b % 3;
        c.lowp_dtype = l == 0 ? MGOPT_NONE : (l == 1 ? MGOPT_BF16 : MGOPT_F16);
        c.begin = static_cast<uint32_t>(chunks.size());
        for (int32_t i : buckets[b]) {
            const int64_t nch = (descs[i].numel + chunk_elems - 1) / chunk_elems;
            for (int64_t k = 0; k < nch; ++k) chunks.push_back(Chunk{static_cast<uint32_t>(i), static_cast<uint32_t>(k)});
        }
        c.count = static_cast<uint32_t>(chunks.size() - c.begin);
        c.norm_begin = static_cast<uint32_t>(norm_chunks.size());
        for (int32_t i : buckets[b]) {
            P->grad_bytes += descs[i].numel * static_cast<int64_t>(dtype_size(descs[i].grad_dtype));
            const int64_t nch = (descs[i].numel + P->norm_chunk - 1) / P->norm_chunk;
            for (int64_t k = 0; k < nch; ++k) norm_chunks.push_back(Chunk{static_cast<uint32_t>(i), static_cast<uint32_t>(k)});
        }
        c.norm_count = static_cast<uint32_t>(norm_chunks.size() - c.norm_begin);
        c.partial_base = static_cast<uint32_t>(P->n_partials);
        P->n_partials += c.norm_count;
        if (c.count) P->classes.push_back(c);
        if (chunks.size() > 0xFFFFFFF0ull) {
            delete P;
            return fail(MGOPT_E_LIMIT, "too many chunks");
        }
    }
    P->n_chunks = static_cast<int64_t>(chunks.size());

    auto cleanup = [&](int rc) {
        mgopt_plan_destroy(P);
        return rc;
    };
    if (hipGetDevice(&P->device) != hipSuccess) return cleanup(fail(MGOPT_E_INVALID, "no current HIP device"));
    hipError_t e;
    if ((e = hipMalloc(&P->d_tensors, sizeof(DevTensor) * n_tensors)) != hipSuccess) return cleanup(hip_fail(e, "hipMalloc tensors"));
    if ((e = hipMalloc(&P->d_grads, sizeof(void*) * n_tensors)) != hipSuccess) return cleanup(hip_fail(e, "hipMalloc grads"));
    if ((e = hipMalloc(&P->d_flags, sizeof(int))) != hipSuccess) return cleanup(hip_fail(e, "hipMalloc flags"));
    if ((e = hipMalloc(&P->d_consts, sizeof(TensorConst) * n_tensors)) != hipSuccess)
        return cleanup(hip_fail(e, "hipMalloc consts"));
    if (P->n_chunks > 0) {
        if ((e = hipMalloc(&P->d_chunks, sizeof(Chunk) * P->n_chunks)) != hipSuccess) return cleanup(hip_fail(e, "hipMalloc chunks"));
        if ((e = hipMalloc(&P->d_norm_chunks, sizeof(Chunk) * norm_chunks.size())) != hipSuccess)
            return cleanup(hip_fail(e, "hipMalloc norm chunks"));
        if ((e = hipMemcpy(P->d_norm_chunks, norm_chunks.data(), sizeof(Chunk) * norm_chunks.size(), hipMemcpyHostToDevice)) !=
            hipSuccess)
            return cleanup(hip_fail(e, "upload norm chunks"));
        if ((e = hipMalloc(&P->d_partials, sizeof(Partial) * P->n_partials)) != hipSuccess) return cleanup(hip_fail(e, "hipMalloc partials"));
        if ((e = hipMemcpy(P->d_chunks, chunks.data(), sizeof(Chunk) * P->n_chunks, hipMemcpyHostToDevice)) != hipSuccess)
            return cleanup(hip_fail(e, "upload chunks"));
    }
    if ((e = hipMemcpy(P->d_tensors, host_t.data(), sizeof(DevTensor) * n_tensors, hipMemcpyHostToDevice)) != hipSuccess)
        return cleanup(hip_fail(e, "upload tensors"));
    if ((e = hipMemset(P->d_grads, 0, sizeof(void*) * n_tensors)) != hipSuccess) return cleanup(hip_fail(e, "clear grads"));
    if ((e = hipMemset(P->d_flags, 0, sizeof(int))) != hipSuccess) return cleanup(hip_fail(e, "clear flags"));
    if (P->fold) {
        const size_t tb = sizeof(uint32_t) * kTicketStride * (1 + static_cast<size_t>(n_tensors));
        if ((e = hipMalloc(&P->d_tickets, tb)) != hipSuccess) return cleanup(hip_fail(e, "hipMalloc tickets"));
        if ((e = hipMemset(P->d_tickets, 0, tb)) != hipSuccess) return cleanup(hip_fail(e, "clear tickets"));
    }
    for (int k = 0; k < kStagingSlots; ++k) {
        if ((e = hipHostMalloc(&P->staging[k], sizeof(void*) * n_tensors, hipHostMallocDefault)) != hipSuccess)
            return cleanup(hip_fail(e, "hipHostMalloc staging"));
        if ((e = hipEventCreateWithFlags(&P->staging_ev[k], hipEventDisableTiming)) != hipSuccess)
            return cleanup(hip_fail(e, "hipEventCreate"));
    }
    P->cached.assign(n_tensors, nullptr);
    if ((e = hipDeviceSynchronize()) != hipSuccess) return cleanup(hip_fail(e, "plan upload"));
    *out = P;
    return 0;
}

MGOPT_API int mgopt_plan_destroy(mgopt_plan* P) {
    if (!P) return 0;
    DeviceGuard guard(P->device);
    for (int k = 0; k < kStagingSlots; ++k) {
        if (P->staging_ev[k]) {
            (void)hipEventSynchronize(P->staging_ev[k]);
            (void)hipEventDestroy(P->staging_ev[k]);
        }
        if (P->staging[k]) (void)hipHostFree(P->staging[k]);
    }
    // Kernels of this plan may still be queued: drain before freeing their tables.
    (void)hipDeviceSynchronize();
    (void)hipFree(P->d_tensors);
    (void)hipFree(P->d_chunks);
    (void)hipFree(P->d_norm_chunks);
    (void)hipFree(P->d_grads);
    (void)hipFree(P->d_partials);
    (void)hipFree(P->d_flags);
    (void)hipFree(P->d_consts);
    (void)hipFree(P->d_tickets);
    delete P;
    return 0;
}

MGOPT_API int64_t mgopt_plan_num_chunks(const mgopt_plan* P) { return P ? P->n_chunks : -1; }

MGOPT_API int mgopt_plan_folded(const mgopt_plan* P) { return P ? (P->fold ? 1 : 0) : -1; }

MGOPT_API int mgopt_plan_set_grads(mgopt_plan* P, const void* const* grads_host, void* stream) {
    if (!P || !grads_host) return fail(MGOPT_E_INVALID, "NULL argument");
    if (P->grads_uploaded && std::memcmp(P->cached.data(), grads_host, sizeof(void*) * P->n_tensors) == 0) return 0;
    DeviceGuard guard(P->device);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int k = P->slot;
    // The staging slot may still feed an earlier copy; its event says when it is free.
    if (P->staging_used[k]) HIP_TRY(hipEventSynchronize(P->staging_ev[k]));
    std::memcpy(P->staging[k], grads_host, sizeof(void*) * P->n_tensors);
    HIP_TRY(hipMemcpyAsync(P->d_grads, P->staging[k], sizeof(void*) * P->n_tensors, hipMemcpyHostToDevice, s));
    HIP_TRY(hipEventRecord(P->staging_ev[k], s));
    P->staging_used[k] = true;
    P->slot = (k + 1) % kStagingSlots;
    std::memcpy(P->cached.data(), grads_host, sizeof(void*) * P->n_tensors);
    P->grads_uploaded = true;
    return 0;
}

MGOPT_API int mgopt_grad_norm(mgopt_plan* P, const float* scale_dev, double max_norm, float* norm_dev, float* coef_dev,
                              float* found_inf_dev, void* stream) {
    if (!P) return fail(MGOPT_E_INVALID, "NULL plan");
    if (!P->grads_uploaded) return fail(MGOPT_E_INVALID, "mgopt_plan_set_grads was not called");
    DeviceGuard guard(P->device);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const FinalizeArgs fin{max_norm, norm_dev, coef_dev, found_inf_dev, P->d_window};
    for (const auto& c : P->classes) {
        int rc = 0;
        switch (c.grad_dtype) {
            case MGOPT_F32: rc = launch_norm<float>(P, c, scale_dev, fin, s); break;
            case MGOPT_F16: rc = launch_norm<_Float16>(P, c, scale_dev, fin, s); break;
            case MGOPT_BF16: rc = launch_norm<Bf16>(P, c, scale_dev, fin, s); break;
            default: rc = fail(MGOPT_E_INVALID, "bad grad dtype");
        }
        if (rc) return rc;
    }
    if (P->fold) return 0;  // the last pass-1 work-group ran the finalize
    hipLaunchKernelGGL(finalize_kernel, dim3(1), dim3(kBlock), 0, s, P->d_partials, P->n_partials, fin);
    return launch_check("finalize_kernel");
}

MGOPT_API int mgopt_adamw_step(mgopt_plan* P, const mgopt_group_hparams* groups, const double* bc_dev, int64_t bc_cap,
                               const float* scale_dev, const float* coef_dev, const float* found_inf_dev, int32_t flags,
                               void* stream) {
    if (!P || !groups || !bc_dev) return fail(MGOPT_E_INVALID, "NULL argument");
    const bool groups_on_device = (flags & MGOPT_GROUPS_ON_DEVICE) != 0;
    if (!P->has_state) return fail(MGOPT_E_INVALID, "grads-only plan: no optimizer state to update");
    if (!P->grads_uploaded) return fail(MGOPT_E_INVALID, "mgopt_plan_set_grads was not called");
    if (bc_cap < 2) return fail(MGOPT_E_INVALID, "bias-correction table too small");
    DeviceGuard guard(P->device);
    hipStream_t s = static_cast<hipStream_t>(stream);

    PrologueArgs pa{};
    pa.grads = P->d_grads;
    pa.tensors = P->d_tensors;
    pa.steps = P->d_steps;
    pa.consts = P->d_consts;
    pa.bc = bc_dev;
    pa.bc_cap = bc_cap;
    pa.scale = scale_dev;
    pa.coef = coef_dev;
    pa.found_inf = found_inf_dev;
    pa.win = P->d_window;
    pa.flags = P->d_flags;
    pa.groups_dev = groups_on_device ? reinterpret_cast<const GroupConst*>(groups) : nullptr;
    pa.n = P->n_tensors;
    for (int gi = 0; gi < MGOPT_MAX_GROUPS && gi < P->n_groups && !groups_on_device; ++gi)
        pa.groups[gi] = GroupConst{groups[gi].lr, groups[gi].weight_decay, groups[gi].beta1, groups[gi].beta2,
                                   groups[gi].eps, groups[gi].maximize, 0};
    FoldLaunch fl{pa, P->d_tickets + kTicketStride};
    const FoldLaunch* f = P->fold ? &fl : nullptr;
    if (!P->fold) {
        hipLaunchKernelGGL(prologue_kernel, dim3((P->n_tensors + kBlock - 1) / kBlock), dim3(kBlock), 0, s, pa);
        if (int rc = launch_check("prologue_kernel")) return rc;
    }

    AdamArgs a{P->d_tensors, P->d_chunks, P->d_grads, P->d_consts, P->chunk_elems, 0,
               (flags & MGOPT_WRITEBACK_GRADS) ? 1 : 0};
    for (const auto& c : P->classes) {
        a.chunk_begin = c.begin;
        int rc = 0;
        switch (c.grad_dtype) {
            case MGOPT_F32: rc = launch_adamw_lowp<float>(a, c.lowp_dtype, c.count, f, s); break;
            case MGOPT_F16: rc = launch_adamw_lowp<_Float16>(a, c.lowp_dtype, c.count, f, s); break;
            case MGOPT_BF16: rc = launch_adamw_lowp<Bf16>(a, c.lowp_dtype, c.count, f, s); break;
            default: rc = fail(MGOPT_E_INVALID, "bad grad dtype");
        }
        if (rc) return rc;
    }
    return 0;
}

MGOPT_API int mgopt_scaler_update(float* scale_dev, int32_t* tracker_dev, const float* const* found_inf_devs, int32_t n_found,
                                  double growth, double backoff, int32_t interval, void* stream) {
    if (!scale_dev || !tracker_dev || !found_inf_devs) return fail(MGOPT_E_INVALID, "NULL argument");
    if (n_found < 1 || n_found > 8) return fail(MGOPT_E_LIMIT, "n_found must be in 1..8");
    FoundList fl{};
    for (int k = 0; k < n_found; ++k) {
        if (!found_inf_devs[k]) return fail(MGOPT_E_INVALID, "NULL found_inf");
        fl.p[k] = found_inf_devs[k];
    }
    hipLaunchKernelGGL(scaler_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream), scale_dev, tracker_dev, fl,
                       n_found, growth, backoff, interval);
    return launch_check("scaler_kernel");
}

MGOPT_API int mgopt_scale_grads(mgopt_plan* P, const float* coef_dev, void* stream) {
    if (!P || !coef_dev) return fail(MGOPT_E_INVALID, "NULL argument");
    if (!P->grads_uploaded) return fail(MGOPT_E_INVALID, "mgopt_plan_set_grads was not called");
    DeviceGuard guard(P->device);
    hipStream_t s = static_cast<hipStream_t>(stream);
    for (const auto& c : P->classes) {
        for (uint64_t done = 0; done < c.count; done += kMaxGroupsPerLaunch) {
            const uint32_t n = static_cast<uint32_t>(std::min<uint64_t>(c.count - done, kMaxGroupsPerLaunch));
            switch (c.grad_dtype) {
                case MGOPT_F32:
                    hipLaunchKernelGGL(scale_grads_kernel<float>, dim3(n), dim3(kBlock), 0, s, P->d_tensors, P->d_chunks,
                                       P->d_grads, coef_dev, P->chunk_elems, static_cast<uint32_t>(c.begin + done));
                    break;
                case MGOPT_F16:
                    hipLaunchKernelGGL(scale_grads_kernel<_Float16>, dim3(n), dim3(kBlock), 0, s, P->d_tensors,
                                       P->d_chunks, P->d_grads, coef_dev, P->chunk_elems, static_cast<uint32_t>(c.begin + done));
                    break;
                case MGOPT_BF16:
                    hipLaunchKernelGGL(scale_grads_kernel<Bf16>, dim3(n), dim3(kBlock), 0, s, P->d_tensors, P->d_chunks,
                                       P->d_grads, coef_dev, P->chunk_elems, static_cast<uint32_t>(c.begin + done));
                    break;
                default: return fail(MGOPT_E_INVALID, "bad grad dtype");
            }
            if (int rc = launch_check("scale_grads_kernel")) return rc;
        }
    }
    return 0;
}

MGOPT_API int mgopt_sync_master(mgopt_plan* P, void* stream) {
    if (!P) return fail(MGOPT_E_INVALID, "NULL plan");
    if (!P->has_state) return fail(MGOPT_E_INVALID, "grads-only plan: no master weights");
    DeviceGuard guard(P->device);
    hipStream_t s = static_cast<hipStream_t>(stream);
    for (const auto& c : P->classes) {
        if (c.lowp_dtype != MGOPT_BF16 && c.lowp_dtype != MGOPT_F16) continue;
        for (uint64_t done = 0; done < c.count; done += kMaxGroupsPerLaunch) {
            const uint32_t n = static_cast<uint32_t>(std::min<uint64_t>(c.count - done, kMaxGroupsPerLaunch));
            if (c.lowp_dtype == MGOPT_BF16)
                hipLaunchKernelGGL(sync_master_kernel<Bf16>, dim3(n), dim3(kBlock), 0, s, P->d_tensors, P->d_chunks,
                                   P->chunk_elems, static_cast<uint32_t>(c.begin + done));
            else
                hipLaunchKernelGGL(sync_master_kernel<_Float16>, dim3(n), dim3(kBlock), 0, s, P->d_tensors, P->d_chunks,
                                   P->chunk_elems, static_cast<uint32_t>(c.begin + done));
            if (int rc = launch_check("sync_master_kernel")) return rc;
        }
    }
    return 0;
}

MGOPT_API int mgopt_plan_set_window(mgopt_plan* P, void* window_dev) {
    if (!P) return fail(MGOPT_E_INVALID, "NULL plan");
    if (reinterpret_cast<uintptr_t>(window_dev) % 4 != 0) return fail(MGOPT_E_ALIGN, "window buffer must be 4-byte aligned");
    P->d_window = static_cast<Window*>(window_dev);
    return 0;
}

MGOPT_API int mgopt_plan_flags(mgopt_plan* P, int* out) {
    if (!P || !out) return fail(MGOPT_E_INVALID, "NULL argument");
    DeviceGuard guard(P->device);
    HIP_TRY(hipMemcpy(out, P->d_flags, sizeof(int), hipMemcpyDeviceToHost));
    return 0;
}

MGOPT_API int mgopt_grad_norm_noalloc(const void* grads_dev, int32_t grad_dtype, int64_t n, const float* scale_dev,
                                      double max_norm, float* norm_dev, float* coef_dev, float* found_inf_dev,
                                      void* stream) {
    if (n < 1 || grads_dev == nullptr) return fail(MGOPT_E_INVALID, "need n >= 1 and a gradient buffer");
    const int64_t chunks = (n + kNormChunk - 1) / kNormChunk;
    if (chunks > kScratchPartials)
        return fail(MGOPT_E_LIMIT, "n = " + std::to_string(n) + " is above the allocation-free norm's maximum of " +
                                       std::to_string(kScratchPartials * kNormChunk) + " elements");
    Partial* part = nullptr;
    if (int rc = scratch_on_current_device(&part)) return rc;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const dim3 grid(static_cast<unsigned>(chunks));
    switch (grad_dtype) {
        case MGOPT_F32: launch_norm_flat<float>(grads_dev, n, scale_dev, part, grid, s); break;
        case MGOPT_F16: launch_norm_flat<_Float16>(grads_dev, n, scale_dev, part, grid, s); break;
        case MGOPT_BF16: launch_norm_flat<Bf16>(grads_dev, n, scale_dev, part, grid, s); break;
        default: return fail(MGOPT_E_INVALID, "bad grad dtype");
    }
    if (int rc = launch_check("norm_flat_kernel")) return rc;
    const FinalizeArgs fin{max_norm, norm_dev, coef_dev, found_inf_dev, nullptr};
    hipLaunchKernelGGL(finalize_kernel, dim3(1), dim3(kBlock), 0, s, part, chunks, fin);
    return launch_check("finalize_kernel");
}

MGOPT_API int mgopt_synth_fill(void* dst, int32_t dtype, int64_t n, uint64_t seed, uint64_t stream_id, double k,
                               uint64_t tail_every, double tail_mult, void* stream) {
    if (n < 0 || (n > 0 && !dst)) return fail(MGOPT_E_INVALID, "bad destination");
    if (n == 0) return 0;
    const uint64_t key = mix64(seed * kGamma + mix64(stream_id + kGamma));
    const int64_t blocks64 = std::min<int64_t>((n + kBlock - 1) / kBlock, 256 * 64);
    const dim3 grid(static_cast<unsigned>(blocks64));
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (dtype) {
        case MGOPT_F32:
            hipLaunchKernelGGL(synth_kernel<float>, grid, dim3(kBlock), 0, s, static_cast<float*>(dst), n, key, k, tail_every, tail_mult);
            break;
        case MGOPT_F16:
            hipLaunchKernelGGL(synth_kernel<_Float16>, grid, dim3(kBlock), 0, s, static_cast<_Float16*>(dst), n, key, k,
                               tail_every, tail_mult);
            break;
        case MGOPT_BF16:
            hipLaunchKernelGGL(synth_kernel<Bf16>, grid, dim3(kBlock), 0, s, static_cast<Bf16*>(dst), n, key, k, tail_every, tail_mult);
            break;
        default: return fail(MGOPT_E_INVALID, "bad dtype");
    }
    return launch_check("synth_kernel");
}

}  // extern "C"
