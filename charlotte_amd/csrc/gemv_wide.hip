// Decode of Q4_0 rows of K = 9,216 to 16,384 in whole 1,024-weight blocks
// (G = 32 S groups, S = 9 .. 16 groups a range) — the down projections of
// the 7-8B models (Llama 3 8B and Mistral 7B: 4,096 x 14,336) — streamed
// through LDS.
//
// Why: a range here is S groups, so the reference's mapping (lane r of a
// half-wave owns range r, matmul.wgsl:207-243) has each lane load 16 bytes
// at a stride of 16 S bytes — 32 cache lines a load instruction — and the
// chunked kernel built on it (gemv.hip, gemv_chunked) reads 4,096 x 14,336
// at 1.5 TB/s. The mapping itself is what the order of addition fixes: a
// range's sum is one chain over its groups in order, so a range belongs to
// one lane and a row to 32 lanes. What changes is how the bytes arrive: a
// wave copies its step's two rows into its LDS stage with
// global_load_lds_dwordx4, eight lanes reading one range's eight consecutive
// groups (128 bytes) an instruction slot, and each lane then reads its own
// range's groups out of LDS.
//
// Stage layout: a row's codes in segments of 8 groups a range — 16-byte slot
// 256 q + 8 r + (e xor r mod 8) holds range r's group 8 q + e — so that the
// lanes reading group i of their ranges fall in different banks; the row's
// 2 G bytes of scales in order. x is staged once a workgroup, range-
// interleaved as gemv_ranges stages it (float4 v of a range's group i at
// 256 i + 32 v + r). Two steps a wave are never in flight: the next step's
// copy is issued once this one is out of the stage, as in gemv_stream4.hip.
// A row's 32 range sums meet in LDS and lane 0 or 1 adds them in order; the
// bits are every other kernel's.
#include <algorithm>

#include "decode.hpp"
#include "plan.hpp"
#include "product.hpp"
#include "stream.hpp"

namespace chm {

namespace {

constexpr uint32_t kWideWaves = 4;  // one workgroup a CU: x and four stages fill LDS
constexpr uint32_t kWideMinSpan = 9, kWideMaxSpan = 16;
constexpr uint32_t kWideSumPad = 36;  // a row's 32 range sums, 16-byte aligned

// A lane's share of a step: its range's S groups of its row, codes and fp16
// scales.
template <uint32_t S>
struct WideRun {
    u32x4s_t codes[S];
    uint32_t d[S];
};

// A wave's 16-byte DMA copy: lane l's 16 bytes from `from` to `to` + 16 l.
// (A function of its own: written inline in the kernel template's lambda,
// the builtin loses the kernel's host launch stub in this compiler.)
__device__ __forceinline__ void copy16(const uint8_t* from, u32x4s_t* to) {
    __builtin_amdgcn_global_load_lds(from, (lds_void)to, 16, 0, kStreamPolicy);
}

}  // namespace

template <uint32_t S, bool FULL>
__global__ __launch_bounds__(64 * kWideWaves) void gemv_wide(Product a, uint32_t steps) {
    constexpr uint32_t G = 32 * S;
    constexpr uint32_t kSegs = (S + 7) / 8;   // 8-group segments a range
    constexpr uint32_t kRowSlots = 256 * kSegs;  // 16-byte slots of a row's codes in the stage
    constexpr uint32_t kScSlots = G / 8;          // 16-byte slots of a row's scales
    __shared__ u32x4s_t x_stage[S * 256];
    __shared__ u32x4s_t codes_a[kWideWaves][2 * kRowSlots];
    __shared__ u32x4s_t scales_a[kWideWaves][2 * kScSlots];
    __shared__ float sums_a[kWideWaves][2 * kWideSumPad];
    const float4* const xs = reinterpret_cast<const float4*>(x_stage);

    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t h = lane >> 5, r = lane & 31u;
    const uint32_t waves = gridDim.x * kWideWaves;
    const uint32_t token = a.last_token ? a.tokens - 1 : 0;
    u32x4s_t *const codes_s = codes_a[wave], *const scales_s = scales_a[wave];
    float* const sums_s = sums_a[wave];

    // The copy: instruction k of a row fills its slots 64 k .. 64 k + 63, lane
    // l slot 64 k + l = 256 q + 8 rr + e', i.e. range rr's group 8 q + (e' xor
    // rr mod 8). Slots past a range's S groups copy nothing.
    uint32_t src_group[kSegs * 4];
#pragma unroll
    for (uint32_t k = 0; k < kSegs * 4; ++k) {
        const uint32_t slot = 64 * k + lane, q = slot >> 8, rr = (slot >> 3) & 31u;
        const uint32_t i = 8 * q + ((slot & 7u) ^ (rr & 7u));
        src_group[k] = i < S ? S * rr + i : ~0u;
    }
    auto issue = [&](uint32_t step) {
#pragma unroll
        for (uint32_t hh = 0; hh < 2; ++hh) {
            const uint32_t p = 2 * step + hh;
            if (p >= a.rows) break;
            const Piece w = piece_of(a, p);
            const uint8_t* codes = w.piece + 16 * (static_cast<uint64_t>(w.row) * G);
#pragma unroll
            for (uint32_t k = 0; k < kSegs * 4; ++k)
                if (src_group[k] != ~0u) copy16(codes + 16 * src_group[k], codes_s + hh * kRowSlots + 64 * k);
            copy_stream<kScSlots>(w.piece + 16 * w.blocks + 2 * (static_cast<uint64_t>(w.row) * G),
                                  scales_s + hh * kScSlots, lane);
        }
    };
    // A lane's share of a step (WideRun), read by instructions the compiler
    // does not look into (it would wait for the copy in flight into the
    // stage); their wait is explicit.
    const uint32_t c_at = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(codes_s + h * kRowSlots)) + 128 * r;
    const uint32_t s_at = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(scales_s + h * kScSlots)) + 2 * S * r;
    auto take = [&](WideRun<S>& run) {
#pragma unroll
        for (uint32_t i = 0; i < S; ++i) {
            const uint32_t at = c_at + 4096 * (i / 8) + 16 * ((i % 8) ^ (r & 7u));
            __asm__ __volatile__("ds_read_b128 %0, %1" : "=v"(run.codes[i]) : "v"(at));
            __asm__ __volatile__("ds_read_u16 %0, %1 offset:%2" : "=v"(run.d[i]) : "v"(s_at), "i"(2 * i));
        }
        __asm__ __volatile__("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (uint32_t i = 0; i < S; ++i) __asm__ __volatile__("" : "+v"(run.codes[i]), "+v"(run.d[i]));
    };
    const uint32_t out_token = a.last_token ? a.tokens - 1 : 0;
    // The range's chain over its groups, its sum to LDS, then lanes 0 and 1
    // add rows 2 step and 2 step + 1's 32 sums in order (matmul.h:34-50).
    auto decode = [&](uint32_t step, const WideRun<S>& run) {
        float s = 0.0f;
#pragma unroll
        for (uint32_t i = 0; i < S; ++i) {
            float xg[32];
#pragma unroll
            for (uint32_t v = 0; v < 8; ++v) {
                const float4 q = xs[256 * i + 32 * v + r];
                xg[4 * v] = q.x, xg[4 * v + 1] = q.y, xg[4 * v + 2] = q.z, xg[4 * v + 3] = q.w;
            }
            const uint32_t w[4] = {run.codes[i][0], run.codes[i][1], run.codes[i][2], run.codes[i][3]};
            s = chain_q4_0(w, run.d[i], xg, s);
        }
        sums_s[kWideSumPad * h + r] = s;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        float total = 0.0f;
        if (lane < 2) total = ordered_total(sums_s + kWideSumPad * lane);
        float partner = 0.0f;
        if (FULL && a.epilogue == kGated) partner = __shfl_xor(total, 1);
        const uint32_t p = 2 * step + lane;
        if (lane < 2 && p < a.rows) emit<FULL>(a, p, 0, out_token, total, partner);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };

    // The first step's copy goes out before x is staged (the barrier below
    // waits for both round trips at once).
    uint32_t step = blockIdx.x * kWideWaves + wave;
    if (step < steps) issue(step);
    {
        // Thread t stages range t % 32, float4 t / 32 of each of its groups,
        // clamped where the product is clipped; every load before any store.
        // The stores are instructions the compiler does not look into (it
        // would wait for the copy just issued); their wait is explicit.
        const float4* src = reinterpret_cast<const float4*>(a.x + static_cast<uint64_t>(token) * G * 32);
        const uint32_t sr = threadIdx.x & 31u, sv = threadIdx.x >> 5;
        float4 xv[S];
#pragma unroll
        for (uint32_t i = 0; i < S; ++i) xv[i] = clamp_input(a, src[(S * sr + i) * 8 + sv]);
        const uint32_t base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(x_stage));
#pragma unroll
        for (uint32_t i = 0; i < S; ++i) {
            const u32x4s_t bits = {__float_as_uint(xv[i].x), __float_as_uint(xv[i].y), __float_as_uint(xv[i].z),
                                   __float_as_uint(xv[i].w)};
            __asm__ __volatile__("ds_write_b128 %0, %1" : : "v"(base + 16 * (256 * i + threadIdx.x)), "v"(bits));
        }
        __asm__ __volatile__("s_waitcnt lgkmcnt(0)" ::: "memory");
        __syncthreads();
    }
    if (step >= steps) return;
    while (true) {
        __builtin_amdgcn_s_waitcnt(kVmcnt0);
        __asm__ __volatile__("" ::: "memory");
        WideRun<S> run;
        take(run);
        const uint32_t next = step + waves;
        if (next < steps) issue(next);
        decode(step, run);
        if (next >= steps) break;
        step = next;
    }
}

// Whether this kernel takes the product: Q4_0, K a whole number of 1,024-
// weight blocks from 9,216 to 16,384 (every range S groups). Rows are copied
// one at a time, so members and gated products take any rows.
bool gemv_wide_takes(const Product& a, uint32_t format) {
    if (format != kQ4_0 || a.groups % 32 != 0) return false;
    const uint32_t span = a.groups / 32;
    return span >= kWideMinSpan && span <= kWideMaxSpan;
}

uint64_t gemv_wide_workgroups(uint32_t compute_units, uint64_t steps) {
    return std::min<uint64_t>(compute_units, (steps + kWideWaves - 1) / kWideWaves);
}

template <uint32_t S>
static void go_wide(const Product& a, uint32_t compute_units, hipStream_t stream) {
    const uint32_t steps = (a.rows + 1) / 2;
    const uint32_t blocks = static_cast<uint32_t>(gemv_wide_workgroups(compute_units, steps));
    if (plain_epilogue(a))
        hipLaunchKernelGGL((gemv_wide<S, false>), dim3(blocks), dim3(64 * kWideWaves), 0, stream, a, steps);
    else
        hipLaunchKernelGGL((gemv_wide<S, true>), dim3(blocks), dim3(64 * kWideWaves), 0, stream, a, steps);
}

hipError_t launch_gemv_wide(const Product& a, uint32_t compute_units, hipStream_t stream) {
    switch (a.groups / 32) {
        case 9: go_wide<9>(a, compute_units, stream); break;
        case 10: go_wide<10>(a, compute_units, stream); break;
        case 11: go_wide<11>(a, compute_units, stream); break;
        case 12: go_wide<12>(a, compute_units, stream); break;
        case 13: go_wide<13>(a, compute_units, stream); break;
        case 14: go_wide<14>(a, compute_units, stream); break;
        case 15: go_wide<15>(a, compute_units, stream); break;
        case 16: go_wide<16>(a, compute_units, stream); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace chm
