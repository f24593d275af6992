// Decode of Q4_0 rows of K = 1,024, 2,048, 4,096 and 8,192 (G = 32, 64, 128,
// 256 groups) — vocabulary heads, down projections and the wide products of
// larger models — streamed through LDS.
//
// Why: the reference's mapping (gemv.hip, lane r of a half-wave owns range
// r) gives a lane G / 32 contiguous groups, so past K = 1,024 each load
// instruction's lanes read 16 bytes at a stride of G / 2 bytes: 64 cache
// lines an instruction at K = 8,192 against 8 at K = 1,024, and the
// measured rate falls with it (32,768 x 8,192: 2.5 TB/s; 262,144 x 1,024:
// 4.0). Here a wave copies a step of rows into its LDS stage with
// global_load_lds_dwordx4 — the step's 8 KB of codes and 1 KB of scales are
// contiguous in the piece, so every copy instruction reads 1 KB in a row —
// and each lane then reads its own groups out of LDS, as gemv_stream8.hip
// does for Q6_K. At K = 1,024 the reference's mapping reads coalesced, but
// with one group a lane a row it spends 4.2 VALU instructions a weight on
// its loads' addresses and each row's reduction, against 2.9 here (the
// Q4_0 head, 151,936 x 1,024: 22.3-24.3 -> 21.6-23.3 us).
//
// Mapping: every lane owns 8 groups (128 code bytes, 16 scale bytes): L = G /
// 8 lanes a row (4, 8, 16, 32), 64 / L rows a step (16, 8, 4, 2). Lane j of
// a row owns ranges (32 / L) j .. (32 / L)(j + 1) - 1, G / 32 groups each.
// Its range sums wait in the wave's LDS for a batch of steps, and lane t
// then adds row t's 32 sums in order from zero. The bits are every other
// kernel's.
//
// The LIMBS form (the GEMV path INT8_LIMBS at K = 1,024 and 2,048,
// limbs.hpp) stages x as int8 limb records in the places of its float4 and
// decodes a group with 24 v_dot4_i32_i8: about half the VALU work a step.
// With plain weight copies it ran within noise of the canonical form (Q4_0
// head 20.2-21.1 us either way); with non-temporal copies it is ~10% faster
// there (19.6 against 21.7 us). At K = 4,096 and 8,192 it measured slower
// than the canonical decode and is not used there. Not the canonical bits:
// within 1e-5 of them.
#include <algorithm>

#include "decode.hpp"
#include "plan.hpp"
#include "product.hpp"
#include "stream.hpp"

namespace chm {

namespace {

// Waves a workgroup and workgroups a CU, by G = 32, 64, 128, 256.
constexpr uint32_t kS4Waves[4] = {4, 4, 4, 4};
constexpr uint32_t kS4Blocks[4] = {2, 2, 2, 2};
constexpr uint32_t s4_index(uint32_t G) { return G == 32 ? 0 : G == 64 ? 1 : G == 128 ? 2 : 3; }
// Rows whose range sums wait in LDS for one ordered pass, by G: as many as
// two workgroups a CU leave LDS for beside the stage and x (64 rows' sums, 8.4
// KB a wave, at G = 32 and 64; 32 at 128; 16 at 256, where x takes 33 KB).
// Fewer, fuller passes: 131,072 x 2,048 34.0 -> 31.2 us, 262,144 x 1,024
// 34.4 -> 31.8 us against 16 rows a pass.
constexpr uint32_t kSumRows[4] = {64, 64, 32, 16};
constexpr uint32_t kCodeChunks = 512, kScaleChunks = 64;  // 16-byte chunks a step: 8 KB codes, 1 KB scales
constexpr uint32_t kSlice4 = 65;                          // x slice stride in float4: 8 groups of 8, one of padding

// A lane's share of a step: its 8 groups' codes and their 8 fp16 scales.
struct StepRun4 {
    u32x4s_t codes[8];
    u32x4s_t scales;
};

}  // namespace

template <uint32_t G, bool FULL, uint32_t W, bool LIMBS>
__global__ __launch_bounds__(64 * W) void gemv_stream4(Product a, uint32_t steps, uint32_t common) {
    constexpr uint32_t L = G / 8;           // lanes a row
    constexpr uint32_t kRows = 64 / L;      // rows a step
    constexpr uint32_t kRanges = 32 / L;    // ranges a lane
    constexpr uint32_t kPerRange = G / 32;  // groups a range
    __shared__ u32x4s_t codes_a[W][kCodeChunks];
    __shared__ u32x4s_t scales_a[W][kScaleChunks];
    __shared__ u32x4s_t x_stage[kSlice4 * L];
    constexpr uint32_t kSums = kSumRows[s4_index(G)];
    constexpr uint32_t kBatch = kSums / kRows;  // steps whose range sums wait for one ordered pass
    __shared__ float sums_a[W][33 * kSums];     // a row's 32 range sums and one of padding
    const float4* const xs = reinterpret_cast<const float4*>(x_stage);

    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t rho = lane / L, j = lane % L;
    const uint32_t waves = gridDim.x * W;
    const uint32_t token = a.last_token ? a.tokens - 1 : 0;
    u32x4s_t *const codes_s = codes_a[wave], *const scales_s = scales_a[wave];
    float* const sums_s = sums_a[wave];

    // Codes land swizzled: stage chunk 8l + k holds the step's chunk 8l + (k
    // xor l mod 8), so the eight lanes that read one 128-byte row each (lane
    // l, its group i at chunk 8l + (i xor l mod 8)) fall in eight different
    // sets of four banks. A copy instruction still reads 1 KB in a row.
    const uint32_t swizzled = (lane & ~7u) | ((lane ^ (lane >> 3)) & 7u);
    auto issue = [&](uint32_t step) {
        const Piece w = piece_of(a, step * kRows);
        const uint64_t g0 = static_cast<uint64_t>(w.row) * G;  // the step's first group
        const uint8_t* from = w.piece + 16 * g0;
#pragma unroll
        for (uint32_t i = 0; i < kCodeChunks / 64; ++i)
            __builtin_amdgcn_global_load_lds(from + 16 * (64 * i + swizzled), (lds_void)(codes_s + 64 * i), 16, 0,
                                             kStreamPolicy);
        copy_stream<kScaleChunks>(w.piece + 16 * w.blocks + 2 * g0, scales_s, lane);
    };
    // The stage's reads are instructions the compiler does not look into (it
    // would wait for the copy in flight into the same stage); their wait is
    // explicit, as in gemv_stream.hip. Lane l's groups are the step's 8l ..
    // 8l + 7.
    const uint32_t c_at = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(codes_s)) + 128 * lane;
    const uint32_t s_at = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(scales_s)) + 16 * lane;
    auto take = [&](StepRun4& run) {
#pragma unroll
        for (uint32_t i = 0; i < 8; ++i)
            __asm__ __volatile__("ds_read_b128 %0, %1" : "=v"(run.codes[i]) : "v"(c_at + 16 * (i ^ (lane & 7u))));
        __asm__ __volatile__("ds_read_b128 %0, %1" : "=v"(run.scales) : "v"(s_at));
        __asm__ __volatile__("s_waitcnt lgkmcnt(0)"
                             : "+v"(run.codes[0]), "+v"(run.codes[1]), "+v"(run.codes[2]), "+v"(run.codes[3]),
                               "+v"(run.codes[4]), "+v"(run.codes[5]), "+v"(run.codes[6]), "+v"(run.codes[7]),
                               "+v"(run.scales)
                             :
                             : "memory");
    };
    const uint32_t out_token = a.last_token ? a.tokens - 1 : 0;
    // A step's range sums go to the wave's LDS, the step's rows at slot
    // `slot` of kBatch.
    auto decode = [&](uint32_t slot, const StepRun4& run) {
        float s = 0.0f;
        // x a group ahead: group i + 1's words are read before group i's
        // products, so the reads' latency runs under them.
        float4 xa[2][8];
#pragma unroll
        for (int v = 0; v < 8; ++v) xa[0][v] = xs[kSlice4 * j + v];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if (i + 1 < 8) {
#pragma unroll
                for (int v = 0; v < 8; ++v) xa[(i + 1) & 1][v] = xs[kSlice4 * j + 8 * (i + 1) + v];
            }
            float xg[32];
#pragma unroll
            for (int v = 0; v < 8; ++v) {
                const float4 q = xa[i & 1][v];
                xg[4 * v] = q.x, xg[4 * v + 1] = q.y, xg[4 * v + 2] = q.z, xg[4 * v + 3] = q.w;
            }
            const uint32_t cw[4] = {run.codes[i][0], run.codes[i][1], run.codes[i][2], run.codes[i][3]};
            const uint32_t d = (run.scales[i >> 1] >> (16 * (i & 1))) & 0xFFFFu;
            if constexpr (LIMBS) {
                // the record's words, as staged: the float4 reads carry them
                u32x4s_t g[8];
#pragma unroll
                for (int v = 0; v < 8; ++v) {
                    const float4 q = xa[i & 1][v];
                    g[v] = u32x4s_t{__float_as_uint(q.x), __float_as_uint(q.y), __float_as_uint(q.z),
                                    __float_as_uint(q.w)};
                }
                s = group_limbs_q4_0(cw, half_to_float(d), g, s);
            } else {
                s = chain_q4_0_wide(cw, d, xg, s);
            }
            if ((i + 1) % kPerRange == 0) {
                sums_s[33 * (slot * kRows + rho) + kRanges * j + i / kPerRange] = s;
                s = 0.0f;
            }
        }
    };
    // Every kBatch steps (and after the last): lane t adds row t's 32 sums in
    // order from zero — ((0 + s0) + s1) + ... + s31, the order of
    // matmul.h:34-50 — and emits it. The serial adds run once for kSums rows
    // instead of once a step. The sums are this wave's own: a wave barrier
    // orders the writes before the reads, and the reads before the next
    // batch's writes. `first` is the batch's first step; its steps are
    // `waves` apart.
    auto flush = [&](uint32_t first, uint32_t count, uint32_t stride) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (lane < count * kRows) {
            float total = 0.0f;
#pragma unroll
            for (int k = 0; k < 32; ++k) total = total + sums_s[33 * lane + k];
            const uint32_t p = (first + (lane / kRows) * stride) * kRows + lane % kRows;
            if (p < a.rows) emit<FULL>(a, p, 0, out_token, total, 0.0f);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };

    // The first step's copy goes out before x is staged (the barrier below
    // waits for both round trips at once).
    uint32_t step = blockIdx.x * W + wave;
    if (step < steps) issue(step);
    if constexpr (LIMBS) {
        // Group g's limb record (limbs.hpp, bias 8) in the place of its
        // eight float4, at 8 g + g / 8; four lanes a group, a quad.
        // Every pass's loads before any record is worked out: one round trip.
        constexpr uint32_t kThreads = 64 * W, kPasses = (4 * G + kThreads - 1) / kThreads;
        const float* xrow = a.x + static_cast<uint64_t>(token) * G * 32;
        const uint32_t base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(x_stage));
        float4 xv[kPasses][2];
#pragma unroll
        for (uint32_t k = 0; k < kPasses; ++k) {
            const uint32_t t = threadIdx.x + kThreads * k;
            if (t < 4 * G) {
                const float4* src = reinterpret_cast<const float4*>(xrow + 8 * t);
                xv[k][0] = clamp_input(a, src[0]), xv[k][1] = clamp_input(a, src[1]);
            }
        }
#pragma unroll
        for (uint32_t k = 0; k < kPasses; ++k) {
            const uint32_t t = threadIdx.x + kThreads * k, group = t >> 2;
            if (t < 4 * G) stage_limbs<8>(xv[k][0], xv[k][1], t & 3u, base + 16 * (8 * group + group / 8));
        }
        __asm__ __volatile__("s_waitcnt lgkmcnt(0)" ::: "memory");
        __syncthreads();
    } else {
        // float4 v of x sits at v + v / 64 (slice v / 64 of 64, one of
        // padding), clamped where the product is clipped. The stores are
        // instructions the compiler does not look into (it would wait for
        // the copy just issued); their wait is explicit.
        constexpr uint32_t kThreads = 64 * W, kPer = (G * 8 + kThreads - 1) / kThreads;  // float4 a thread
        const float4* src = reinterpret_cast<const float4*>(a.x + static_cast<uint64_t>(token) * G * 32);
        const uint32_t base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(x_stage));
        float4 xv[kPer];
#pragma unroll
        for (uint32_t k = 0; k < kPer; ++k)
            if (threadIdx.x + kThreads * k < G * 8) xv[k] = clamp_input(a, src[threadIdx.x + kThreads * k]);
#pragma unroll
        for (uint32_t k = 0; k < kPer; ++k) {
            const uint32_t v = threadIdx.x + kThreads * k;
            if (v >= G * 8) break;
            const u32x4s_t bits = {__float_as_uint(xv[k].x), __float_as_uint(xv[k].y), __float_as_uint(xv[k].z),
                                   __float_as_uint(xv[k].w)};
            __asm__ __volatile__("ds_write_b128 %0, %1" : : "v"(base + 16 * (v + v / 64)), "v"(bits));
        }
        __asm__ __volatile__("s_waitcnt lgkmcnt(0)" ::: "memory");
        __syncthreads();
    }
    if (step >= steps) return;
    uint32_t slot = 0, first = step, stride = waves;
    while (true) {
        __builtin_amdgcn_s_waitcnt(kVmcnt0);
        __asm__ __volatile__("" ::: "memory");
        StepRun4 run;
        take(run);
        // Steps below `common` are dealt to every wave in turn; the rest to
        // the first half of the grid alone (the CUs' first workgroups, which
        // finish sooner when dealt the same). A batch's steps are `stride`
        // apart, so a batch ends where the dealing changes.
        uint32_t next = step + waves;
        bool turn = false;
        if (next >= common) {
            const uint32_t fast = waves / 2, w = blockIdx.x * W + wave;
            turn = step < common;
            next = turn ? (w < fast ? common + w : steps) : step + fast;
        }
        if (next < steps) issue(next);
        decode(slot, run);
        if (++slot == kBatch || next >= steps || turn) {
            flush(first, slot, stride);
            slot = 0;
            first = next;
            if (turn) stride = waves / 2;
        }
        if (next >= steps) break;
        step = next;
    }
}

// Whether this kernel takes the product: Q4_0, K = 1,024, 2,048, 4,096 or
// 8,192, 2^20 groups or more, every member's rows and first row a whole number of
// steps (so a step lies in one member), not gated (a gated product
// interleaves its members' rows). A smaller product is bound by dispatch and
// one memory round trip, and goes to the 32-lane mapping's one-wave
// workgroups, which spread over every CU (Qwen3 0.6B's o projection, 1,024 x
// 2,048: its decode step 590 -> 559 us).
bool gemv_stream4_takes(const Product& a, uint32_t format) {
    if (format != kQ4_0 || (a.groups != 32 && a.groups != 64 && a.groups != 128 && a.groups != 256)) return false;
    if (static_cast<uint64_t>(a.rows) * a.groups < (1u << 20)) return false;
    const uint32_t rows = 64 / (a.groups / 8);
    for (uint32_t m = 0; m < a.members; ++m)
        if (a.m[m].rows % rows != 0 || a.m[m].row_offset % rows != 0) return false;
    return a.epilogue != kGated;
}

uint64_t gemv_stream4_workgroups(uint32_t groups, uint32_t compute_units, uint64_t steps) {
    const uint32_t i = s4_index(groups);
    return std::min<uint64_t>(uint64_t{kS4Blocks[i]} * compute_units, (steps + kS4Waves[i] - 1) / kS4Waves[i]);
}

template <uint32_t G, bool LIMBS>
static void go4(const Product& a, uint32_t compute_units, hipStream_t stream) {
    constexpr uint32_t W = kS4Waves[s4_index(G)];
    const uint32_t steps = a.rows / (64 / (G / 8));
    const uint32_t blocks = static_cast<uint32_t>(gemv_stream4_workgroups(G, compute_units, steps));
    // The last round's worth of steps on the first half of the grid: Q4_0
    // head 151,936 x 1,024 21.6 -> 20.3 us, 65,536 x 2,048 18.4 -> 17.9,
    // 32,768 x 8,192 32.4 -> 32.1 (two rounds A/B on one box).
    const uint32_t waves = blocks * W;
    const uint32_t common = steps >= 2 * waves ? steps - waves : steps;
    if (plain_epilogue(a))
        hipLaunchKernelGGL((gemv_stream4<G, false, W, LIMBS>), dim3(blocks), dim3(64 * W), 0, stream, a, steps, common);
    else
        hipLaunchKernelGGL((gemv_stream4<G, true, W, LIMBS>), dim3(blocks), dim3(64 * W), 0, stream, a, steps, common);
}

template <bool LIMBS>
static hipError_t launch4(const Product& a, uint32_t compute_units, hipStream_t stream) {
    switch (a.groups) {
        case 32: go4<32, LIMBS>(a, compute_units, stream); break;
        case 64: go4<64, LIMBS>(a, compute_units, stream); break;
        case 128: go4<128, LIMBS>(a, compute_units, stream); break;
        case 256: go4<256, LIMBS>(a, compute_units, stream); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_gemv_stream4(const Product& a, uint32_t compute_units, bool limbs, hipStream_t stream) {
    return limbs ? launch4<true>(a, compute_units, stream) : launch4<false>(a, compute_units, stream);
}

}  // namespace chm
