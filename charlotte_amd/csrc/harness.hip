// Test and benchmark harness (libcharlotte_hip_harness.so) — not part of
// the product's ABI. Device memory, copies, streams, events and graphs for
// Python callers that do not load a framework, plus two kernels:
//   chx_unpack — the formats' unpack (formats.hpp, the code the product's
//     kernels inline) writing each group's 32 weights out, so a test can hold
//     it to the CPU dequant bit for bit (tests/gpu/support/unpack.h:30-109's
//     role);
//   chx_copy — a plain copy of known size, the yardstick rocprofv3's
//     FETCH_SIZE / WRITE_SIZE counters are scaled by;
//   chx_read — a streaming read of known size and nothing else, copied a
//     9 KB step a wave at a time into LDS by global_load_lds_dwordx4,
//     non-temporal, as the LDS-streamed decodes copy their weights: the rate
//     a decode of the same bytes could reach were its arithmetic free;
//   chx_touch — one-wave workgroups that each read a few KB and write a
//     word: a small decode's dispatch and memory round trip with its
//     arithmetic, reduction and epilogue taken away;
//   chx_mfma_rate — a matrix-core instruction shape issued back to back by
//     every wave, C independent accumulators a wave: the shape's sustained
//     rate, and with one accumulator its dependent-chain rate;
//   chx_read_sweep — the same read in other forms, for the ceiling of a
//     pure read on this part: 16-byte loads into registers (grid-strided or
//     a contiguous chunk a workgroup, U loads in flight a lane, plain or
//     non-temporal) and the LDS copy at 4, 9 or 16 KB a wave step with one
//     or two steps in flight.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <cstdio>
#include <type_traits>

#include "formats.hpp"

namespace {

template <uint32_t F>
__global__ void unpack_kernel(const uint8_t* piece, uint64_t blocks, uint64_t groups, float* out) {
    const uint64_t g = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (g >= groups) return;
    float w[32];
    chm::unpack<F>(piece, blocks, g, w);
    float4* dst = reinterpret_cast<float4*>(out + 32 * g);
#pragma unroll
    for (int v = 0; v < 8; ++v) dst[v] = make_float4(w[4 * v], w[4 * v + 1], w[4 * v + 2], w[4 * v + 3]);
}

__global__ void copy_kernel(const float4* __restrict__ src, float4* __restrict__ dst, uint64_t n) {
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<uint64_t>(gridDim.x) * blockDim.x)
        dst[i] = src[i];
}

__global__ void null_kernel() {}

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void* lds_void_t;
constexpr uint32_t kReadChunks = 9;  // 1 KB chunks a step: 9 KB, a streamed Q4_0 step's size
constexpr uint32_t kReadWaves = 4;

// Each wave copies steps of kReadChunks 1 KB chunks into its own LDS stage,
// one step in flight, and waits for it; steps are grid-strided. `sink`
// takes one word a thread from the stage at the end, so the copies have a
// reader.
__global__ __launch_bounds__(64 * kReadWaves) void read_kernel(const uint8_t* src, uint64_t chunks, uint32_t* sink) {
    __shared__ u32x4_t stage[kReadWaves][kReadChunks * 64];
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63u;
    const uint64_t steps = (chunks + kReadChunks - 1) / kReadChunks;
    for (uint64_t s = static_cast<uint64_t>(blockIdx.x) * kReadWaves + wave; s < steps;
         s += static_cast<uint64_t>(gridDim.x) * kReadWaves) {
#pragma unroll
        for (uint32_t i = 0; i < kReadChunks; ++i) {
            const uint64_t c = s * kReadChunks + i;
            if (c < chunks)
                __builtin_amdgcn_global_load_lds(src + 1024 * c + 16 * lane, (lds_void_t)(stage[wave] + 64 * i), 16, 0,
                                                 2);
        }
        __builtin_amdgcn_s_waitcnt((0x7 << 4) | (0xF << 8));  // vmcnt(0)
    }
    __syncthreads();
    sink[static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x] = stage[wave][lane].x;
}

// Wave w (a workgroup of one) reads `kib` 1 KB runs from src + w * kib KB,
// 16 bytes a lane a run, eight runs' loads issued before any is used, and
// writes one word a lane.
__global__ __launch_bounds__(64) void touch_kernel(const u32x4_t* src, uint32_t kib, uint32_t* sink) {
    const u32x4_t* p = src + static_cast<uint64_t>(blockIdx.x) * kib * 64 + threadIdx.x;
    uint32_t acc = 0;
    for (uint32_t i = 0; i < kib; i += 8) {
        u32x4_t v[8];
#pragma unroll
        for (uint32_t j = 0; j < 8; ++j)
            if (i + j < kib) v[j] = p[64 * (i + j)];
#pragma unroll
        for (uint32_t j = 0; j < 8; ++j)
            if (i + j < kib) acc ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
    }
    sink[static_cast<uint64_t>(blockIdx.x) * 64 + threadIdx.x] = acc;
}

// vmcnt(n) for s_waitcnt (expcnt and lgkmcnt left at their maxima).
constexpr int vmcnt(int n) { return (n & 0xF) | (0x7 << 4) | (0xF << 8) | ((n >> 4) << 14); }

// A lane's sink word is written only when its fold of every loaded word
// meets a value no data here makes, so the loads cannot be dropped and
// nothing is stored.
constexpr uint32_t kNever = 0x9E3779B9u;

// 16-byte loads into registers, U a lane in flight: grid-strided over the
// buffer (CHUNK false) or over one contiguous chunk a workgroup.
template <int U, bool NT, bool CHUNK>
__global__ __launch_bounds__(1024) void sweep_regs(const u32x4_t* src, uint64_t n16, uint32_t* sink) {
    uint64_t i, stride, end;
    if constexpr (CHUNK) {
        const uint64_t per = (n16 + gridDim.x - 1) / gridDim.x;
        i = blockIdx.x * per + threadIdx.x;
        end = min(n16, (blockIdx.x + 1) * per);
        stride = blockDim.x;
    } else {
        i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
        end = n16;
        stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    }
    uint32_t acc = 0;
    for (; i + (U - 1) * stride < end; i += U * stride) {
        u32x4_t v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = NT ? __builtin_nontemporal_load(src + i + u * stride) : src[i + u * stride];
#pragma unroll
        for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; i < end; i += stride) {
        const u32x4_t v = src[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == kNever) sink[static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x] = acc;
}

// The LDS copy: each of a workgroup's four waves copies steps of CH 1 KB
// chunks (grid-strided) into its own stage, DEPTH steps in flight; POLICY
// the copies' cache policy bits (0, or 2: non-temporal).
template <int CH, int DEPTH, int POLICY>
__global__ __launch_bounds__(256) void sweep_lds(const uint8_t* src, uint64_t chunks, uint32_t* sink) {
    __shared__ u32x4_t stage[4][DEPTH][CH * 64];
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63u;
    const uint64_t steps = (chunks + CH - 1) / CH;
    uint32_t k = 0;
    for (uint64_t s = static_cast<uint64_t>(blockIdx.x) * 4 + wave; s < steps;
         s += static_cast<uint64_t>(gridDim.x) * 4, ++k) {
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            const uint64_t c = s * CH + i;
            if (c < chunks)
                __builtin_amdgcn_global_load_lds(src + 1024 * c + 16 * lane,
                                                 (lds_void_t)(stage[wave][k % DEPTH] + 64 * i), 16, 0, POLICY);
        }
        __builtin_amdgcn_s_waitcnt(vmcnt(CH * (DEPTH - 1)));
    }
    __builtin_amdgcn_s_waitcnt(vmcnt(0));
    __syncthreads();
    const uint32_t v = stage[wave][0][lane].x;
    if (v == kNever) sink[static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x] = v;
}

typedef _Float16 mh8 __attribute__((ext_vector_type(8)));
typedef __bf16 mb8 __attribute__((ext_vector_type(8)));
typedef float mf4 __attribute__((ext_vector_type(4)));
typedef float mf16 __attribute__((ext_vector_type(16)));
typedef int mi4 __attribute__((ext_vector_type(4)));
typedef int mi16 __attribute__((ext_vector_type(16)));

typedef float mf32 __attribute__((ext_vector_type(32)));

// Shape S (0 f16 16x16x32, 1 f16 32x32x16, 2 bf16 16x16x32, 3 i8 16x16x64,
// 4 i8 32x32x32, 5 f32 32x32x1 two blocks, 6 f32 16x16x1 four blocks, 7 f32
// 32x32x2, 8 f32 16x16x4), C chains, `iters` rounds of C instructions a wave.
template <int S, int C>
__global__ __launch_bounds__(256) void mfma_rate_kernel(uint32_t iters, uint32_t* sink) {
    const float f = static_cast<float>(threadIdx.x & 7u) * 0.125f;
    if constexpr (S >= 5) {
        using Acc = std::conditional_t<S == 5, mf32, std::conditional_t<S == 8, mf4, mf16>>;
        // 32x32x1's 32 accumulators a chain: at most 4 chains (never launched with 8)
        constexpr int CC = S == 5 && C > 4 ? 4 : C;
        const float g = 1.0f + f;
        Acc acc[CC] = {};
        for (uint32_t i = 0; i < iters; ++i) {
#pragma unroll
            for (int c = 0; c < CC; ++c) {
                if constexpr (S == 5) acc[c] = __builtin_amdgcn_mfma_f32_32x32x1f32(f, g, acc[c], 0, 0, 0);
                else if constexpr (S == 6) acc[c] = __builtin_amdgcn_mfma_f32_16x16x1f32(f, g, acc[c], 0, 0, 0);
                else if constexpr (S == 7) acc[c] = __builtin_amdgcn_mfma_f32_32x32x2f32(f, g, acc[c], 0, 0, 0);
                else acc[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(f, g, acc[c], 0, 0, 0);
            }
        }
        uint32_t fold = 0;
#pragma unroll
        for (int c = 0; c < CC; ++c) fold ^= __builtin_bit_cast(uint32_t, acc[c][0]);
        if (fold == kNever) sink[static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x] = fold;
        return;
    }
    const mh8 h = {(_Float16)f, (_Float16)0.5f, (_Float16)f, (_Float16)1.0f,
                   (_Float16)f, (_Float16)0.25f, (_Float16)f, (_Float16)2.0f};
    const mb8 bb = {(__bf16)f, (__bf16)0.5f, (__bf16)f, (__bf16)1.0f, (__bf16)f, (__bf16)0.25f, (__bf16)f, (__bf16)2.0f};
    const mi4 iv = {static_cast<int>(threadIdx.x), 0x01020304, 0x7F00FF01, 3};
    uint32_t fold = 0;
    if constexpr (S == 0 || S == 2 || S == 3) {
        using Acc = std::conditional_t<S == 3, mi4, mf4>;
        Acc acc[C] = {};
        for (uint32_t i = 0; i < iters; ++i) {
#pragma unroll
            for (int c = 0; c < C; ++c) {
                if constexpr (S == 0) acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(h, h, acc[c], 0, 0, 0);
                else if constexpr (S == 2) acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bb, bb, acc[c], 0, 0, 0);
                else acc[c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(iv, iv, acc[c], 0, 0, 0);
            }
        }
#pragma unroll
        for (int c = 0; c < C; ++c) fold ^= __builtin_bit_cast(uint32_t, acc[c][0]);
    } else {
        using Acc = std::conditional_t<S == 4, mi16, mf16>;
        Acc acc[C] = {};
        for (uint32_t i = 0; i < iters; ++i) {
#pragma unroll
            for (int c = 0; c < C; ++c) {
                if constexpr (S == 1) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(h, h, acc[c], 0, 0, 0);
                else acc[c] = __builtin_amdgcn_mfma_i32_32x32x32_i8(iv, iv, acc[c], 0, 0, 0);
            }
        }
#pragma unroll
        for (int c = 0; c < C; ++c) fold ^= __builtin_bit_cast(uint32_t, acc[c][0]);
    }
    if (fold == kNever) sink[static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x] = fold;
}

// Whether a K = 1 f32 matrix instruction rounds as one fused multiply-add:
// S 5 the 32x32x1 (two blocks, 32 registers), 6 the 16x16x1 (four blocks, 16
// registers). Pair p gives a and b to every lane, and the wave's accumulator
// values c[p][64 v + lane] (v < the shape's registers; 2,048 floats a pair);
// every element of the result is then c + a b whatever its place in the
// blocks, so no layout is assumed: lane l compares its result v with fmaf(a,
// b, c) bit for bit (two NaNs agree). out: [0] elements differing, [1]
// elements compared, then for the first 64 differing: pair, element, the
// instruction's bits, fmaf's bits.
template <int S>
__global__ __launch_bounds__(64) void mfma_fma_check_kernel(const float* ab, const float* c, uint32_t pairs,
                                                            uint32_t* out) {
    constexpr int R = S == 5 ? 32 : 16;
    using Acc = std::conditional_t<R == 32, mf32, mf16>;
    const uint32_t lane = threadIdx.x;
    uint32_t compared = 0;
    for (uint32_t p = blockIdx.x; p < pairs; p += gridDim.x) {
        const float a = ab[2 * p], b = ab[2 * p + 1];
        const float* cp = c + static_cast<uint64_t>(p) * 2048;
        Acc acc;
#pragma unroll
        for (int v = 0; v < R; ++v) acc[v] = cp[64 * v + lane];
        Acc d;
        if constexpr (S == 5) d = __builtin_amdgcn_mfma_f32_32x32x1f32(a, b, acc, 0, 0, 0);
        else d = __builtin_amdgcn_mfma_f32_16x16x1f32(a, b, acc, 0, 0, 0);
#pragma unroll
        for (int v = 0; v < R; ++v) {
            // the element copied out first: this compiler lowers a bit cast of
            // a vector's element d[v] to element 0 whatever v is
            const float dv = d[v];
            const float r = __builtin_fmaf(a, b, acc[v]);
            const uint32_t rb = __builtin_bit_cast(uint32_t, r), db = __builtin_bit_cast(uint32_t, dv);
            const bool same = rb == db || (r != r && dv != dv);
            ++compared;
            if (!same) {
                const uint32_t at = atomicAdd(out, 1u);
                if (at < 64) {
                    out[2 + 4 * at] = p;
                    out[3 + 4 * at] = 64 * v + lane;
                    out[4 + 4 * at] = db;
                    out[5 + 4 * at] = rb;
                }
            }
        }
    }
    atomicAdd(out + 1, compared);
}

// The K = 2 and K = 4 f32 shapes (32x32x2: lane l supplies k = l / 32; 16x16x4:
// k = l / 16) against fmaf in k order: pair p gives a[k] and b[k] to the
// lanes of its k, so every element is c + a0 b0 + a1 b1 (+ ...) whatever its
// place; each lane compares its results with fmaf(a1, b1, fmaf(a0, b0, c))
// (and so on) bit for bit. ab: 2 K floats a pair (a0 b0 a1 b1 ...); c: 64 R
// floats a pair. out as mfma_fma_check's.
template <int K>
__global__ __launch_bounds__(64) void mfma_chain_check_kernel(const float* ab, const float* c, uint32_t pairs,
                                                              uint32_t* out) {
    constexpr int R = K == 2 ? 16 : 4;
    using Acc = std::conditional_t<R == 16, mf16, mf4>;
    const uint32_t lane = threadIdx.x;
    uint32_t compared = 0;
    for (uint32_t p = blockIdx.x; p < pairs; p += gridDim.x) {
        const float* q = ab + static_cast<uint64_t>(p) * 2 * K;
        const uint32_t my_k = K == 2 ? lane / 32 : lane / 16;
        const float a = q[2 * my_k], b = q[2 * my_k + 1];
        Acc acc;
#pragma unroll
        for (int v = 0; v < R; ++v) acc[v] = c[static_cast<uint64_t>(p) * 64 * R + 64 * v + lane];
        Acc d;
        if constexpr (K == 2) d = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc, 0, 0, 0);
        else d = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc, 0, 0, 0);
#pragma unroll
        for (int v = 0; v < R; ++v) {
            const float dv = d[v];
            float r = acc[v];
#pragma unroll
            for (int k = 0; k < K; ++k) r = __builtin_fmaf(q[2 * k], q[2 * k + 1], r);
            const uint32_t rb = __builtin_bit_cast(uint32_t, r), db = __builtin_bit_cast(uint32_t, dv);
            ++compared;
            if (!(rb == db || (r != r && dv != dv))) {
                const uint32_t at = atomicAdd(out, 1u);
                if (at < 64) {
                    out[2 + 4 * at] = p;
                    out[3 + 4 * at] = 64 * v + lane;
                    out[4 + 4 * at] = db;
                    out[5 + 4 * at] = rb;
                }
            }
        }
    }
    atomicAdd(out + 1, compared);
}

// Where a shape puts each accumulator it is given: a = b = 0 and C read from
// c[64 v + lane] (v < the shape's registers), D written to out at the same
// places, so out = c where the instruction adds C element by element in its
// own layout. S: 5 f32 32x32x1 two blocks, 6 f32 16x16x1 four blocks, 7 f32
// 32x32x2, 8 f32 16x16x4, 9 f32 4x4x1 sixteen blocks, 1 f16 32x32x16.
template <int S>
__global__ __launch_bounds__(64) void mfma_c_probe_kernel(const float* c, float* out) {
    const uint32_t lane = threadIdx.x;
    constexpr int R = S == 5 ? 32 : S == 8 || S == 9 ? 4 : 16;
    using Acc = std::conditional_t<R == 32, mf32, std::conditional_t<R == 4, mf4, mf16>>;
    Acc acc;
#pragma unroll
    for (int v = 0; v < R; ++v) acc[v] = c[64 * v + lane];
    Acc d;
    if constexpr (S == 5) d = __builtin_amdgcn_mfma_f32_32x32x1f32(0.0f, 0.0f, acc, 0, 0, 0);
    else if constexpr (S == 6) d = __builtin_amdgcn_mfma_f32_16x16x1f32(0.0f, 0.0f, acc, 0, 0, 0);
    else if constexpr (S == 7) d = __builtin_amdgcn_mfma_f32_32x32x2f32(0.0f, 0.0f, acc, 0, 0, 0);
    else if constexpr (S == 8) d = __builtin_amdgcn_mfma_f32_16x16x4f32(0.0f, 0.0f, acc, 0, 0, 0);
    else if constexpr (S == 9) d = __builtin_amdgcn_mfma_f32_4x4x1f32(0.0f, 0.0f, acc, 0, 0, 0);
    else {
        const mh8 z = {};
        d = __builtin_amdgcn_mfma_f32_32x32x16_f16(z, z, acc, 0, 0, 0);
    }
#pragma unroll
    for (int v = 0; v < R; ++v) out[64 * v + lane] = d[v];
}

// A K = 1 f32 instruction's lane layout (S 5 the 32x32x1, 6 the 16x16x1):
// with C = 0, a = lane + 1 and b = 1 each result names the lane whose a it
// took (its row); with a = 1 and b = lane + 1, the lane whose b it took (its
// column). out: 2 x 64 lanes x the shape's registers, [64 v + lane].
template <int S>
__global__ __launch_bounds__(64) void mfma_layout_kernel(float* out) {
    constexpr int R = S == 5 ? 32 : 16;
    using Acc = std::conditional_t<R == 32, mf32, mf16>;
    const uint32_t lane = threadIdx.x;
    const Acc zero = {};
    const float id = static_cast<float>(lane + 1);
    Acc rows, cols;
    if constexpr (S == 5) {
        rows = __builtin_amdgcn_mfma_f32_32x32x1f32(id, 1.0f, zero, 0, 0, 0);
        cols = __builtin_amdgcn_mfma_f32_32x32x1f32(1.0f, id, zero, 0, 0, 0);
    } else {
        rows = __builtin_amdgcn_mfma_f32_16x16x1f32(id, 1.0f, zero, 0, 0, 0);
        cols = __builtin_amdgcn_mfma_f32_16x16x1f32(1.0f, id, zero, 0, 0, 0);
    }
#pragma unroll
    for (int v = 0; v < R; ++v) {
        out[64 * v + lane] = rows[v];
        out[64 * R + 64 * v + lane] = cols[v];
    }
}

}  // namespace

extern "C" {

// An empty kernel of one workgroup: the floor under any launch.
int chx_null(void* s) {
    hipLaunchKernelGGL(null_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(s));
    return hipGetLastError();
}

int chx_device_count() {
    int n = 0;
    return hipGetDeviceCount(&n) == hipSuccess ? n : 0;
}

int chx_set_device(int d) { return hipSetDevice(d); }

int chx_device_name(int d, char* out, int len) {
    hipDeviceProp_t p;
    const hipError_t e = hipGetDeviceProperties(&p, d);
    if (e != hipSuccess) return e;
    snprintf(out, len, "%s|%s|cus=%d|clock_khz=%d|mem=%zu", p.name, p.gcnArchName, p.multiProcessorCount,
             p.clockRate, static_cast<size_t>(p.totalGlobalMem));
    return 0;
}

const char* chx_error_string(int e) { return hipGetErrorString(static_cast<hipError_t>(e)); }

int chx_malloc(void** p, uint64_t bytes) { return hipMalloc(p, bytes); }
int chx_free(void* p) { return hipFree(p); }
int chx_h2d(void* dst, const void* src, uint64_t bytes) { return hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice); }
int chx_d2h(void* dst, const void* src, uint64_t bytes) { return hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost); }
int chx_d2d(void* dst, const void* src, uint64_t bytes) { return hipMemcpy(dst, src, bytes, hipMemcpyDeviceToDevice); }
int chx_memset(void* p, int value, uint64_t bytes) { return hipMemset(p, value, bytes); }
int chx_sync() { return hipDeviceSynchronize(); }
int chx_last_error() { return hipGetLastError(); }

int chx_stream_create(void** s) { return hipStreamCreate(reinterpret_cast<hipStream_t*>(s)); }
int chx_stream_destroy(void* s) { return hipStreamDestroy(static_cast<hipStream_t>(s)); }
int chx_stream_sync(void* s) { return hipStreamSynchronize(static_cast<hipStream_t>(s)); }

int chx_event_create(void** e) { return hipEventCreate(reinterpret_cast<hipEvent_t*>(e)); }
int chx_event_destroy(void* e) { return hipEventDestroy(static_cast<hipEvent_t>(e)); }
int chx_event_record(void* e, void* s) { return hipEventRecord(static_cast<hipEvent_t>(e), static_cast<hipStream_t>(s)); }
int chx_event_sync(void* e) { return hipEventSynchronize(static_cast<hipEvent_t>(e)); }
int chx_event_elapsed_ms(float* ms, void* start, void* stop) {
    return hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop));
}

// Graphs: capture a stream's launches, then replay them.
int chx_capture_begin(void* s) {
    return hipStreamBeginCapture(static_cast<hipStream_t>(s), hipStreamCaptureModeThreadLocal);
}
// Global mode: while it lasts, an unsafe call (an allocation, a free, a
// synchronous copy) from any thread of the process fails the capture.
int chx_capture_begin_global(void* s) {
    return hipStreamBeginCapture(static_cast<hipStream_t>(s), hipStreamCaptureModeGlobal);
}
int chx_capture_end(void* s, void** exec) {
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(static_cast<hipStream_t>(s), &g);
    if (e != hipSuccess) return e;
    e = hipGraphInstantiate(reinterpret_cast<hipGraphExec_t*>(exec), g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    return e;
}
int chx_graph_launch(void* exec, void* s) {
    return hipGraphLaunch(static_cast<hipGraphExec_t>(exec), static_cast<hipStream_t>(s));
}
int chx_graph_destroy(void* exec) { return hipGraphExecDestroy(static_cast<hipGraphExec_t>(exec)); }

int chx_unpack(uint32_t type, const void* piece, uint64_t blocks_in_piece, uint64_t groups, float* out, void* s) {
    if (reinterpret_cast<uintptr_t>(piece) % 16 != 0) return hipErrorInvalidValue;
    const dim3 grid(static_cast<uint32_t>((groups + 63) / 64));
    const auto* p = static_cast<const uint8_t*>(piece);
    const auto stream = static_cast<hipStream_t>(s);
    switch (type) {
        case chm::kF32:
            hipLaunchKernelGGL((unpack_kernel<chm::kF32>), grid, dim3(64), 0, stream, p, blocks_in_piece, groups, out);
            break;
        case chm::kF16:
            hipLaunchKernelGGL((unpack_kernel<chm::kF16>), grid, dim3(64), 0, stream, p, blocks_in_piece, groups, out);
            break;
        case chm::kBF16:
            hipLaunchKernelGGL((unpack_kernel<chm::kBF16>), grid, dim3(64), 0, stream, p, blocks_in_piece, groups, out);
            break;
        case chm::kQ4_0:
            hipLaunchKernelGGL((unpack_kernel<chm::kQ4_0>), grid, dim3(64), 0, stream, p, blocks_in_piece, groups, out);
            break;
        case chm::kQ4_1:
            hipLaunchKernelGGL((unpack_kernel<chm::kQ4_1>), grid, dim3(64), 0, stream, p, blocks_in_piece, groups, out);
            break;
        case chm::kQ8_0:
            hipLaunchKernelGGL((unpack_kernel<chm::kQ8_0>), grid, dim3(64), 0, stream, p, blocks_in_piece, groups, out);
            break;
        case chm::kQ6_K:
            hipLaunchKernelGGL((unpack_kernel<chm::kQ6_K>), grid, dim3(64), 0, stream, p, blocks_in_piece, groups, out);
            break;
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

int chx_copy(const void* src, void* dst, uint64_t bytes, void* s) {
    if (bytes % 16 != 0) return hipErrorInvalidValue;
    const uint64_t n = bytes / 16;
    const uint32_t blocks = static_cast<uint32_t>(std::min<uint64_t>((n + 255) / 256, 65536));
    hipLaunchKernelGGL(copy_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(s),
                       static_cast<const float4*>(src), static_cast<float4*>(dst), n);
    return hipGetLastError();
}

// Reads `bytes` (whole KB, 16-byte aligned) at `src` with read_kernel on
// two workgroups of four waves a CU; `sink` holds a word a thread
// (chx_read_sink_bytes).
int chx_read_sink_bytes(uint64_t* bytes) {
    int device = 0, cus = 0;
    hipError_t e = hipGetDevice(&device);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
    if (e != hipSuccess) return e;
    *bytes = static_cast<uint64_t>(2 * cus) * 64 * kReadWaves * 4;
    return hipSuccess;
}

int chx_read(const void* src, uint64_t bytes, void* sink, uint64_t sink_bytes, void* s) {
    uint64_t need = 0;
    const int e = chx_read_sink_bytes(&need);
    if (e != hipSuccess) return e;
    if (bytes % 1024 != 0 || reinterpret_cast<uintptr_t>(src) % 16 != 0 || sink_bytes < need) return hipErrorInvalidValue;
    const uint32_t blocks = static_cast<uint32_t>(need / (64 * kReadWaves * 4));
    hipLaunchKernelGGL(read_kernel, dim3(blocks), dim3(64 * kReadWaves), 0, static_cast<hipStream_t>(s),
                       static_cast<const uint8_t*>(src), bytes / 1024, static_cast<uint32_t*>(sink));
    return hipGetLastError();
}

// One form of the read sweep over `bytes` (whole KB, 16-byte aligned) at
// `src`: form 0 registers grid-strided, 1 registers a chunk a workgroup
// (u loads in flight a lane: 4, 8 or 16; nt: non-temporal loads), both with
// `blocks` workgroups of `threads` lanes (64..1024, whole waves); form 2 the
// LDS copy (u KB a step: 4, 9 or 16; depth steps in flight: 1 or 2; nt:
// non-temporal copies), `blocks` four-wave workgroups. `sink` must hold a
// word a lane of the grid.
int chx_read_sweep(int form, int u, int nt, int depth, uint32_t blocks, uint32_t threads, const void* src,
                   uint64_t bytes, void* sink, uint64_t sink_bytes, void* s) {
    const auto stream = static_cast<hipStream_t>(s);
    if (form == 2) threads = 256;
    if (blocks == 0 || threads == 0 || threads > 1024 || threads % 64 != 0 || bytes % 1024 != 0 ||
        reinterpret_cast<uintptr_t>(src) % 16 != 0 || sink_bytes < static_cast<uint64_t>(blocks) * threads * 4)
        return hipErrorInvalidValue;
    const auto* v = static_cast<const u32x4_t*>(src);
    auto* out = static_cast<uint32_t*>(sink);
    const uint64_t n16 = bytes / 16;
#define CHX_REGS(U, NT, CHUNK) \
    hipLaunchKernelGGL((sweep_regs<U, NT, CHUNK>), dim3(blocks), dim3(threads), 0, stream, v, n16, out)
    if (form == 0 || form == 1) {
        const bool chunk = form == 1;
        const int key = u * 4 + (nt ? 2 : 0) + (chunk ? 1 : 0);
        switch (key) {
            case 16: CHX_REGS(4, false, false); break;
            case 17: CHX_REGS(4, false, true); break;
            case 18: CHX_REGS(4, true, false); break;
            case 19: CHX_REGS(4, true, true); break;
            case 32: CHX_REGS(8, false, false); break;
            case 33: CHX_REGS(8, false, true); break;
            case 34: CHX_REGS(8, true, false); break;
            case 35: CHX_REGS(8, true, true); break;
            case 64: CHX_REGS(16, false, false); break;
            case 65: CHX_REGS(16, false, true); break;
            case 66: CHX_REGS(16, true, false); break;
            case 67: CHX_REGS(16, true, true); break;
            default: return hipErrorInvalidValue;
        }
    } else if (form == 2) {
        const auto* b = static_cast<const uint8_t*>(src);
        const uint64_t chunks = bytes / 1024;
        const int key = u * 4 + depth + (nt ? 1000 : 0);
#define CHX_LDS(CH, D, P) \
    hipLaunchKernelGGL((sweep_lds<CH, D, P>), dim3(blocks), dim3(256), 0, stream, b, chunks, out)
        switch (key) {
            case 17: CHX_LDS(4, 1, 0); break;
            case 18: CHX_LDS(4, 2, 0); break;
            case 37: CHX_LDS(9, 1, 0); break;
            case 38: CHX_LDS(9, 2, 0); break;
            case 65: CHX_LDS(16, 1, 0); break;
            case 66: CHX_LDS(16, 2, 0); break;
            case 1017: CHX_LDS(4, 1, 2); break;
            case 1018: CHX_LDS(4, 2, 2); break;
            case 1037: CHX_LDS(9, 1, 2); break;
            case 1038: CHX_LDS(9, 2, 2); break;
            case 1065: CHX_LDS(16, 1, 2); break;
            case 1066: CHX_LDS(16, 2, 2); break;
            default: return hipErrorInvalidValue;
        }
#undef CHX_LDS
    } else {
        return hipErrorInvalidValue;
    }
#undef CHX_REGS
    return hipGetLastError();
}

// The matrix-core rate probe: `blocks` four-wave workgroups each issuing
// `iters` rounds of `chains` independent instructions of `shape` (see
// mfma_rate_kernel) a wave. The operations a launch does: blocks x 4 x
// iters x chains x the shape's 2 M N K. `sink` holds a word a lane.
int chx_mfma_rate(int shape, int chains, uint32_t blocks, uint32_t iters, void* sink, uint64_t sink_bytes, void* s) {
    if (blocks == 0 || sink_bytes < static_cast<uint64_t>(blocks) * 256 * 4) return hipErrorInvalidValue;
    const auto stream = static_cast<hipStream_t>(s);
    auto* out = static_cast<uint32_t*>(sink);
#define CHX_MFMA(S, C) hipLaunchKernelGGL((mfma_rate_kernel<S, C>), dim3(blocks), dim3(256), 0, stream, iters, out)
#define CHX_SHAPE(S)                  \
    switch (chains) {                 \
        case 1: CHX_MFMA(S, 1); break; \
        case 2: CHX_MFMA(S, 2); break; \
        case 4: CHX_MFMA(S, 4); break; \
        case 8: if (S == 5) return hipErrorInvalidValue; CHX_MFMA(S, 8); break; \
        default: return hipErrorInvalidValue; \
    }
    switch (shape) {
        case 0: CHX_SHAPE(0); break;
        case 1: CHX_SHAPE(1); break;
        case 2: CHX_SHAPE(2); break;
        case 3: CHX_SHAPE(3); break;
        case 4: CHX_SHAPE(4); break;
        case 5: CHX_SHAPE(5); break;
        case 6: CHX_SHAPE(6); break;
        case 7: CHX_SHAPE(7); break;
        case 8: CHX_SHAPE(8); break;
        default: return hipErrorInvalidValue;
    }
#undef CHX_SHAPE
#undef CHX_MFMA
    return hipGetLastError();
}

// mfma_fma_check_kernel<shape> (5 or 6) over `pairs` pairs (ab: 2 floats a
// pair; c: 2,048 floats a pair), `blocks` one-wave workgroups; out: 2 + 4 x
// 64 words, cleared here.
int chx_mfma_fma_check(int shape, const void* ab, const void* c, uint32_t pairs, uint32_t blocks, void* out,
                       void* s) {
    if (pairs == 0 || blocks == 0 || (shape != 5 && shape != 6)) return hipErrorInvalidValue;
    const auto stream = static_cast<hipStream_t>(s);
    hipError_t e = hipMemsetAsync(out, 0, (2 + 4 * 64) * 4, stream);
    if (e != hipSuccess) return e;
    const auto* abf = static_cast<const float*>(ab);
    const auto* cf = static_cast<const float*>(c);
    auto* o = static_cast<uint32_t*>(out);
    if (shape == 5)
        hipLaunchKernelGGL(mfma_fma_check_kernel<5>, dim3(blocks), dim3(64), 0, stream, abf, cf, pairs, o);
    else
        hipLaunchKernelGGL(mfma_fma_check_kernel<6>, dim3(blocks), dim3(64), 0, stream, abf, cf, pairs, o);
    return hipGetLastError();
}

// mfma_c_probe_kernel<shape>: c and out hold 2,048 floats.
int chx_mfma_c_probe(int shape, const void* c, void* out, void* s) {
    const auto stream = static_cast<hipStream_t>(s);
    const auto* ci = static_cast<const float*>(c);
    auto* o = static_cast<float*>(out);
    switch (shape) {
        case 1: hipLaunchKernelGGL(mfma_c_probe_kernel<1>, dim3(1), dim3(64), 0, stream, ci, o); break;
        case 5: hipLaunchKernelGGL(mfma_c_probe_kernel<5>, dim3(1), dim3(64), 0, stream, ci, o); break;
        case 6: hipLaunchKernelGGL(mfma_c_probe_kernel<6>, dim3(1), dim3(64), 0, stream, ci, o); break;
        case 7: hipLaunchKernelGGL(mfma_c_probe_kernel<7>, dim3(1), dim3(64), 0, stream, ci, o); break;
        case 8: hipLaunchKernelGGL(mfma_c_probe_kernel<8>, dim3(1), dim3(64), 0, stream, ci, o); break;
        case 9: hipLaunchKernelGGL(mfma_c_probe_kernel<9>, dim3(1), dim3(64), 0, stream, ci, o); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// mfma_chain_check_kernel<k> (k = 2 or 4) over `pairs`: ab 2 k floats a
// pair, c 1,024 (k = 2) or 256 (k = 4) floats a pair; out as
// chx_mfma_fma_check's, cleared here.
int chx_mfma_chain_check(int k, const void* ab, const void* c, uint32_t pairs, uint32_t blocks, void* out, void* s) {
    if (pairs == 0 || blocks == 0 || (k != 2 && k != 4)) return hipErrorInvalidValue;
    const auto stream = static_cast<hipStream_t>(s);
    hipError_t e = hipMemsetAsync(out, 0, (2 + 4 * 64) * 4, stream);
    if (e != hipSuccess) return e;
    const auto* abf = static_cast<const float*>(ab);
    const auto* cf = static_cast<const float*>(c);
    auto* o = static_cast<uint32_t*>(out);
    if (k == 2)
        hipLaunchKernelGGL(mfma_chain_check_kernel<2>, dim3(blocks), dim3(64), 0, stream, abf, cf, pairs, o);
    else
        hipLaunchKernelGGL(mfma_chain_check_kernel<4>, dim3(blocks), dim3(64), 0, stream, abf, cf, pairs, o);
    return hipGetLastError();
}

// mfma_layout_kernel<shape> (5 or 6): out holds 2 x 2,048 floats.
int chx_mfma_layout(int shape, void* out, void* s) {
    const auto stream = static_cast<hipStream_t>(s);
    if (shape == 5) hipLaunchKernelGGL(mfma_layout_kernel<5>, dim3(1), dim3(64), 0, stream, static_cast<float*>(out));
    else if (shape == 6)
        hipLaunchKernelGGL(mfma_layout_kernel<6>, dim3(1), dim3(64), 0, stream, static_cast<float*>(out));
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

// `waves` one-wave workgroups reading `kib` KB each from `src` (16-byte
// aligned, waves * kib KB long); `sink` holds 64 words a wave.
int chx_touch(const void* src, uint32_t waves, uint32_t kib, void* sink, uint64_t sink_bytes, void* s) {
    if (waves == 0 || kib == 0 || reinterpret_cast<uintptr_t>(src) % 16 != 0 ||
        sink_bytes < static_cast<uint64_t>(waves) * 64 * 4)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(touch_kernel, dim3(waves), dim3(64), 0, static_cast<hipStream_t>(s),
                       static_cast<const u32x4_t*>(src), kib, static_cast<uint32_t*>(sink));
    return hipGetLastError();
}

}  // extern "C"
