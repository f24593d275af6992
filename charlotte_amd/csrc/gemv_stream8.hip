// Decode of Q6_K rows of K = 1,024 and 2,048 (G = 32, 64 groups) — the LM
// heads of Qwen3 0.6B (151,936 x 1,024) and Llama 3.2 1B (128,256 x 2,048)
// among them — streamed through LDS as gemv_stream.hip streams K = 1,152.
//
// Here every lane owns exactly 8 groups, one whole super-block, so a lane's
// d is one value: L = G / 8 lanes a row (4 or 8), 64 / L rows a step (16 or
// 8), and a step is 512 groups (64 super-blocks) whatever G — lo 8,192
// bytes, hi 4,096, scales 1,024, d 128, contiguous in the piece since a step
// starts on a super-block. Lane j of a row owns ranges (32 / L) j ..
// (32 / L)(j + 1) - 1, G / 32 groups each (floor(rG/32) is exact here). A
// wave copies a step into its LDS stage with global_load_lds_dwordx4, reads
// its lanes' share into registers once it has landed, starts the next
// step's copy, and decodes from registers, as gemv_stream.hip does; two
// workgroups of four waves a CU.
//
// Canonical form: a lane's range sums, then the row's chain over its L lanes
// by DPP row shifts — ((0 + sums of lane 0) + sums of lane 1) + ... — the
// order of matmul.h:34-50, the bits of every other kernel. LIMBS form (the
// INT8_LIMBS path, limbs.hpp): the lane's 8 groups into one sum from zero,
// the row's L sums added pairwise.
#include <algorithm>

#include "plan.hpp"
#include "product.hpp"
#include "stream.hpp"

namespace chm {

namespace {

constexpr int kWaves8 = 4;
constexpr uint32_t kLo8 = 512, kHi8 = 256, kSc8 = 64, kD8 = 8;  // 16-byte chunks a stream a step
constexpr uint32_t kSlice8 = 65;  // x slice stride, float4 or u32x4 (8 groups of 8, one of padding)

// A lane's share of a step: its 8 groups' lo and hi, their scale pairs, d.
struct StepRun8 {
    u32x4s_t lo[8];
    u32x2s_t hi[8];
    uint32_t sc[8];
    uint32_t d;
};

}  // namespace

template <uint32_t G, bool FULL, bool LIMBS>
__global__ __launch_bounds__(256, 2) void gemv_stream8(Product a, uint32_t steps, uint32_t common) {
    constexpr uint32_t L = G / 8;              // lanes a row
    constexpr uint32_t kRows = 64 / L;         // rows a step
    constexpr uint32_t kRanges = 32 / L;       // ranges a lane
    constexpr uint32_t kPerRange = G / 32;     // groups a range
    __shared__ u32x4s_t lo_a[kWaves8][kLo8];
    __shared__ u32x4s_t hi_a[kWaves8][kHi8];
    __shared__ u32x4s_t sc_a[kWaves8][kSc8];
    __shared__ u32x4s_t d_a[kWaves8][kD8];
    // x: L slices of 64 float4 and one of padding; or (LIMBS) L slices of 8
    // group records and 4 dwords of padding (the same size)
    __shared__ u32x4s_t x_stage[kSlice8 * L];
    float4* const xs = reinterpret_cast<float4*>(x_stage);

    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t rho = lane / L, j = lane % L;
    const uint32_t waves = gridDim.x * kWaves8;
    const uint32_t token = a.last_token ? a.tokens - 1 : 0;
    u32x4s_t *const lo_s = lo_a[wave], *const hi_s = hi_a[wave], *const sc_s = sc_a[wave], *const d_s = d_a[wave];

    auto issue = [&](uint32_t step) {
        const Piece w = piece_of(a, step * kRows);
        const uint64_t n = w.blocks, g0 = static_cast<uint64_t>(w.row) * G;  // the step's first group
        copy_stream<kLo8>(w.piece + 16 * g0, lo_s, lane);
        copy_stream<kHi8>(w.piece + 128 * n + 8 * g0, hi_s, lane);
        copy_stream<kSc8>(w.piece + 192 * n + 2 * g0, sc_s, lane);
        copy_stream<kD8>(w.piece + 208 * n + 2 * (g0 / 8), d_s, lane);
    };
    const uint32_t lg = G * rho + 8 * j;  // the lane's first group within a step (a super-block's first)
    // The stage's reads are instructions the compiler does not look into (it
    // would wait for the copy in flight into the same stage); their waits
    // are explicit, as in gemv_stream.hip.
    auto take = [&](StepRun8& run) {
        const uint32_t lo_at = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lo_s)) + 16 * lg;
        const uint32_t hi_at = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(hi_s)) + 8 * lg;
        const uint32_t sc_at = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(sc_s)) + 2 * lg;
        const uint32_t d_at = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(d_s)) + 2 * (lg >> 3);
#define CHM_LDS_B128(dst, off) __asm__ __volatile__("ds_read_b128 %0, %1 offset:" #off : "=v"(dst) : "v"(lo_at))
#define CHM_LDS_B64(dst, off) __asm__ __volatile__("ds_read_b64 %0, %1 offset:" #off : "=v"(dst) : "v"(hi_at))
#define CHM_LDS_U16(dst, addr, off) __asm__ __volatile__("ds_read_u16 %0, %1 offset:" #off : "=v"(dst) : "v"(addr))
        CHM_LDS_B128(run.lo[0], 0);
        CHM_LDS_B128(run.lo[1], 16);
        CHM_LDS_B128(run.lo[2], 32);
        CHM_LDS_B128(run.lo[3], 48);
        CHM_LDS_B128(run.lo[4], 64);
        CHM_LDS_B128(run.lo[5], 80);
        CHM_LDS_B128(run.lo[6], 96);
        CHM_LDS_B128(run.lo[7], 112);
        CHM_LDS_B64(run.hi[0], 0);
        CHM_LDS_B64(run.hi[1], 8);
        CHM_LDS_B64(run.hi[2], 16);
        CHM_LDS_B64(run.hi[3], 24);
        CHM_LDS_B64(run.hi[4], 32);
        CHM_LDS_B64(run.hi[5], 40);
        CHM_LDS_B64(run.hi[6], 48);
        CHM_LDS_B64(run.hi[7], 56);
        CHM_LDS_U16(run.sc[0], sc_at, 0);
        CHM_LDS_U16(run.sc[1], sc_at, 2);
        CHM_LDS_U16(run.sc[2], sc_at, 4);
        CHM_LDS_U16(run.sc[3], sc_at, 6);
        CHM_LDS_U16(run.sc[4], sc_at, 8);
        CHM_LDS_U16(run.sc[5], sc_at, 10);
        CHM_LDS_U16(run.sc[6], sc_at, 12);
        CHM_LDS_U16(run.sc[7], sc_at, 14);
        CHM_LDS_U16(run.d, d_at, 0);
        __asm__ __volatile__("s_waitcnt lgkmcnt(0)"
                             : "+v"(run.lo[0]), "+v"(run.lo[1]), "+v"(run.lo[2]), "+v"(run.lo[3]), "+v"(run.lo[4]),
                               "+v"(run.lo[5]), "+v"(run.lo[6]), "+v"(run.lo[7])
                             :
                             : "memory");
        __asm__ __volatile__(""
                             : "+v"(run.hi[0]), "+v"(run.hi[1]), "+v"(run.hi[2]), "+v"(run.hi[3]), "+v"(run.hi[4]),
                               "+v"(run.hi[5]), "+v"(run.hi[6]), "+v"(run.hi[7]));
        __asm__ __volatile__(""
                             : "+v"(run.sc[0]), "+v"(run.sc[1]), "+v"(run.sc[2]), "+v"(run.sc[3]), "+v"(run.sc[4]),
                               "+v"(run.sc[5]), "+v"(run.sc[6]), "+v"(run.sc[7]), "+v"(run.d));
#undef CHM_LDS_B128
#undef CHM_LDS_B64
#undef CHM_LDS_U16
    };
    const uint32_t out_token = a.last_token ? a.tokens - 1 : 0;
    // Canonical: the lane's range sums, then the chain over the row's lanes
    // (row_shr:1 hands lane j - 1's partial total to lane j).
    auto decode_exact = [&](uint32_t step, const StepRun8& run) {
        float sums[kRanges];
        float s = 0.0f;
        float4 xa[2][8];
#pragma unroll
        for (int v = 0; v < 8; ++v) xa[0][v] = xs[kSlice8 * j + v];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if (i + 1 < 8) {
#pragma unroll
                for (int v = 0; v < 8; ++v) xa[(i + 1) & 1][v] = xs[kSlice8 * j + 8 * (i + 1) + v];
            }
            float xg[32];
#pragma unroll
            for (int v = 0; v < 8; ++v) {
                const float4 q = xa[i & 1][v];
                xg[4 * v] = q.x, xg[4 * v + 1] = q.y, xg[4 * v + 2] = q.z, xg[4 * v + 3] = q.w;
            }
            const uint32_t lw[4] = {run.lo[i][0], run.lo[i][1], run.lo[i][2], run.lo[i][3]};
            const uint32_t hw[2] = {run.hi[i][0], run.hi[i][1]};
            s = chain_q6_k(lw, hw, run.sc[i], run.d, xg, s);
            if ((i + 1) % kPerRange == 0) {
                sums[i / kPerRange] = s;
                s = 0.0f;
            }
        }
        float total = 0.0f;
#pragma unroll
        for (uint32_t step_lane = 0; step_lane < L; ++step_lane) {
            float t = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, total), 0x111, 0xF, 0xF,
                                                                           false));  // row_shr:1
            if (step_lane == 0) t = 0.0f;
#pragma unroll
            for (uint32_t k = 0; k < kRanges; ++k) t = t + sums[k];
            if (j == step_lane) total = t;
        }
        const uint32_t p = step * kRows + rho;
        if (j == L - 1 && p < a.rows) emit<FULL>(a, p, 0, out_token, total, 0.0f);
    };
    // LIMBS: the lane's 8 groups into one sum; the row's L sums pairwise
    // (lanes xor 1, xor 2, then xor 4 for L = 8): every lane the same total.
    auto decode_limbs = [&](uint32_t step, const StepRun8& run) {
        const u32x4s_t* records = x_stage + kSlice8 * j;
        const float d = half_to_float(run.d);
        u32x4s_t g[2][8];
#pragma unroll
        for (int v = 0; v < 8; ++v) g[0][v] = records[v];
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if (i + 1 < 8) {
#pragma unroll
                for (int v = 0; v < 8; ++v) g[(i + 1) & 1][v] = records[8 * (i + 1) + v];
            }
            const uint32_t lw[4] = {run.lo[i][0], run.lo[i][1], run.lo[i][2], run.lo[i][3]};
            const uint32_t hw[2] = {run.hi[i][0], run.hi[i][1]};
            s = group_limbs_q6_k(lw, hw, run.sc[i], d, g[i & 1], s);
        }
        float total = s + __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, s), 0xB1, 0xF, 0xF,
                                                                              false));  // quad_perm [1, 0, 3, 2]
        total = total + __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, total), 0x4E, 0xF,
                                                                           0xF, false));  // quad_perm [2, 3, 0, 1]
        if constexpr (L == 8) total = total + __shfl_xor(total, 4);
        const uint32_t p = step * kRows + rho;
        if (j == L - 1 && p < a.rows) emit<FULL>(a, p, 0, out_token, total, 0.0f);
    };

    // The first step's copy goes out before x is staged (the barrier below
    // waits for both round trips at once).
    uint32_t step = blockIdx.x * kWaves8 + wave;
    if (step < steps) issue(step);
    if constexpr (LIMBS) {
        // group g's record: slice g / 8, record g % 8; four lanes a group
        const uint32_t t = threadIdx.x;
        if (t < 4 * G) {
            const uint32_t group = t >> 2, part = t & 3u;
            const float4* src =
                reinterpret_cast<const float4*>(a.x + static_cast<uint64_t>(token) * G * 32 + 32 * group + 8 * part);
            const uint32_t base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(x_stage));
            stage_limbs(clamp_input(a, src[0]), clamp_input(a, src[1]), part,
                        base + 16 * (kSlice8 * (group / 8) + 8 * (group % 8)));
        }
        __asm__ __volatile__("s_waitcnt lgkmcnt(0)" ::: "memory");
        __syncthreads();
    } else {
        // float4 v of x sits at v + v / 64 (slice v / 64 of 64, one of padding)
        constexpr uint32_t kPer = G * 8 / 256;  // float4 a thread: 1 or 2
        const float4* src = reinterpret_cast<const float4*>(a.x + static_cast<uint64_t>(token) * G * 32);
        const uint32_t base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(x_stage));
        float4 xv[kPer];
#pragma unroll
        for (uint32_t k = 0; k < kPer; ++k) xv[k] = clamp_input(a, src[threadIdx.x + 256 * k]);
#pragma unroll
        for (uint32_t k = 0; k < kPer; ++k) {
            const uint32_t v = threadIdx.x + 256 * k;
            const u32x4s_t bits = {__float_as_uint(xv[k].x), __float_as_uint(xv[k].y), __float_as_uint(xv[k].z),
                                   __float_as_uint(xv[k].w)};
            __asm__ __volatile__("ds_write_b128 %0, %1" : : "v"(base + 16 * (v + v / 64)), "v"(bits));
        }
        __asm__ __volatile__("s_waitcnt lgkmcnt(0)" ::: "memory");
        __syncthreads();
    }
    if (step >= steps) return;
    while (true) {
        __builtin_amdgcn_s_waitcnt(kVmcnt0);
        __asm__ __volatile__("" ::: "memory");
        StepRun8 run;
        take(run);
        // Steps below `common` are dealt to every wave in turn; the rest to
        // the first half of the grid alone (w < waves / 2), the CUs' first
        // workgroups, which win the SIMDs' issue arbitration and finish
        // sooner when dealt the same (as in gemv_stream.hip).
        uint32_t next = step + waves;
        if (next >= common) {
            const uint32_t fast = waves / 2, w = blockIdx.x * kWaves8 + wave;
            next = step < common ? (w < fast ? common + w : steps) : step + fast;
        }
        if (next < steps) issue(next);
        if constexpr (LIMBS)
            decode_limbs(step, run);
        else
            decode_exact(step, run);
        if (next >= steps) break;
        step = next;
    }
}

// Whether this kernel takes the product: Q6_K, K = 1,024 or 2,048, every
// member's rows and first row a whole number of steps, not gated.
bool gemv_stream8_takes(const Product& a, uint32_t format) {
    if (format != kQ6_K || (a.groups != 32 && a.groups != 64)) return false;
    const uint32_t rows = 64 / (a.groups / 8);
    for (uint32_t m = 0; m < a.members; ++m)
        if (a.m[m].rows % rows != 0 || a.m[m].row_offset % rows != 0) return false;
    return a.epilogue != kGated;
}

template <uint32_t G>
static void go8(const Product& a, uint32_t compute_units, bool limbs, hipStream_t stream) {
    const uint32_t steps = a.rows / (64 / (G / 8));
    const uint32_t blocks = std::min<uint32_t>(2 * compute_units, (steps + kWaves8 - 1) / kWaves8);
    // The last round's worth of steps on the first half of the grid: Q6_K
    // heads 151,936 x 1,024 32.5 -> 31.6 us, 128,256 x 2,048 47.5 -> 46.6,
    // 262,144 x 1,024 48.1 -> 47.6 (two rounds A/B on one box).
    const uint32_t waves = blocks * kWaves8;
    const uint32_t common = steps >= 2 * waves ? steps - waves : steps;
    const bool plain = plain_epilogue(a);
    if (limbs) {
        if (plain)
            hipLaunchKernelGGL((gemv_stream8<G, false, true>), dim3(blocks), dim3(256), 0, stream, a, steps, common);
        else
            hipLaunchKernelGGL((gemv_stream8<G, true, true>), dim3(blocks), dim3(256), 0, stream, a, steps, common);
    } else if (plain) {
        hipLaunchKernelGGL((gemv_stream8<G, false, false>), dim3(blocks), dim3(256), 0, stream, a, steps, common);
    } else {
        hipLaunchKernelGGL((gemv_stream8<G, true, false>), dim3(blocks), dim3(256), 0, stream, a, steps, common);
    }
}

hipError_t launch_gemv_stream8(const Product& a, uint32_t compute_units, bool limbs, hipStream_t stream) {
    if (a.groups == 32)
        go8<32>(a, compute_units, limbs, stream);
    else
        go8<64>(a, compute_units, limbs, stream);
    return hipGetLastError();
}

}  // namespace chm
