// Prefill of a short step: the canonical tile with K split inside the workgroup.
//
// gemm_short — VALU, the canonical order, bit-exact with every other kernel.
// A step too short to give the GPU's compute units a 128-row tile each (a few
// tokens through a product, gated or with options, which the reference never
// splits along K: matmul.cpp:166-172) leaves most CUs idle in gemm_canonical:
// 32 tokens through a 2,048 x 8,192 product are 16 workgroups, each walking
// all of K. Here a workgroup takes a tile of RT rows x 32 tokens (RT = 16 or
// 8, so a step makes 8-16 times the workgroups), and its four waves split K
// between them: wave w computes ranges 8w .. 8w + 7 of every output of the
// tile, each range an fma chain from zero in k order, and keeps the 8 range
// sums in registers. Every wave stages its own groups in its own LDS, so the
// K loop needs no workgroup barrier. At the end the 32 range sums of each
// output meet in LDS and are added in order from zero, skipping empty ranges
// (G < 32) — the order of addition of gemm_canonical and of the split form's
// combine (matmul.wgsl:592-695), so the bits are theirs.
//
// A lane's micro-tile: rows 2r and 2r + 1 (a gated product's gate and up
// totals meet in one lane) by TT tokens; per k one float2 of weights and one
// float2 or float4 of inputs from LDS for 2 TT multiply-adds.
#include "plan.hpp"
#include "product.hpp"

namespace chm {

namespace {

constexpr uint32_t kTokens = 32;  // tokens a tile
constexpr uint32_t kWaves = 4;    // waves a workgroup: eight of the 32 ranges each

__device__ __forceinline__ uint32_t pick4(const uint32_t* w, uint32_t i) {
    return i == 0 ? w[0] : i == 1 ? w[1] : i == 2 ? w[2] : w[3];
}

// Weight l (0..31, known only at run time) of a group: the arithmetic of
// formats.hpp's weight(), its words picked by selects, so nothing is indexed
// in registers by a run-time value. Exact, the same bits.
__device__ __forceinline__ float weight_at(const Q4_0Group& g, uint32_t l) {
    const uint32_t q = (pick4(g.w, (l & 15u) >> 2) >> (8 * (l & 3u) + 4 * (l >> 4))) & 0xFu;
    return __builtin_fmaf(static_cast<float>(q), g.d, g.minus_8d);
}

__device__ __forceinline__ float weight_at(const Q4_1Group& g, uint32_t l) {
    const uint32_t q = (pick4(g.w, (l & 15u) >> 2) >> (8 * (l & 3u) + 4 * (l >> 4))) & 0xFu;
    return __builtin_fmaf(static_cast<float>(q), g.d, g.m);
}

__device__ __forceinline__ float weight_at(const Q6_KGroup& g, uint32_t l) {
    const uint32_t low = (pick4(g.lo, (l & 15u) >> 2) >> (8 * (l & 3u) + 4 * (l >> 4))) & 0xFu;
    const uint32_t pair = ((((l & 7u) >> 2) ? g.hi[1] : g.hi[0]) >> (8 * (l & 3u) + 2 * (l >> 3))) & 3u;
    const float q = static_cast<float>(low | (pair << 4));
    return l < 16 ? __builtin_fmaf(q, g.first, g.minus_32_first) : __builtin_fmaf(q, g.second, g.minus_32_second);
}

__device__ __forceinline__ float weight_at(const Q8_0Group& g, uint32_t l) {
    const uint32_t i = l >> 2;
    const uint32_t word = i < 4 ? pick4(g.w, i) : pick4(g.w + 4, i - 4);
    const int32_t q = static_cast<int8_t>((word >> (8 * (l & 3u))) & 0xFFu);
    return static_cast<float>(q) * g.d;
}

// Weights first .. first + N - 1 of an unquantized group, loaded as they lie
// (F32 N words, F16 and BF16 N / 2), so no value is picked by a run-time index.
template <uint32_t F, uint32_t N>
struct ValuesRun {
    uint32_t w[F == kF32 ? N : N / 2];
};

template <uint32_t F, uint32_t N>
__device__ __forceinline__ ValuesRun<F, N> fetch_values_run(const uint8_t* piece, uint64_t gi, uint32_t first) {
    constexpr uint32_t bytes = F == kF32 ? 4 : 2;
    constexpr uint32_t words = F == kF32 ? N : N / 2;
    const uint8_t* at = piece + 32 * bytes * gi + bytes * first;
    ValuesRun<F, N> out;
    if constexpr (words % 4 == 0) {
#pragma unroll
        for (uint32_t v = 0; v < words / 4; ++v) {
            const uint4 q = reinterpret_cast<const uint4*>(at)[v];
            out.w[4 * v] = q.x, out.w[4 * v + 1] = q.y, out.w[4 * v + 2] = q.z, out.w[4 * v + 3] = q.w;
        }
    } else {
        const uint2 q = *reinterpret_cast<const uint2*>(at);
        out.w[0] = q.x, out.w[1] = q.y;
    }
    return out;
}

// Value j of a run, exact (formats.hpp's value()).
template <uint32_t F, uint32_t N>
__device__ __forceinline__ float value_of(const ValuesRun<F, N>& r, int j) {
    if constexpr (F == kF32) return __uint_as_float(r.w[j]);
    else if constexpr (F == kF16) return half_to_float((j & 1) ? r.w[j >> 1] >> 16 : r.w[j >> 1] & 0xFFFFu);
    else return (j & 1) ? bf16_high(r.w[j >> 1]) : bf16_low(r.w[j >> 1]);
}

template <uint32_t F, uint32_t N>
__device__ __forceinline__ auto fetch_short(const uint8_t* piece, uint64_t n, uint64_t gi, uint32_t first) {
    if constexpr (F == kQ4_0) return fetch_q4_0(piece, n, gi);
    else if constexpr (F == kQ4_1) return fetch_q4_1(piece, n, gi);
    else if constexpr (F == kQ8_0) return fetch_q8_0(piece, n, gi);
    else if constexpr (plain_values(F)) return fetch_values_run<F, N>(piece, gi, first);
    else return fetch_q6_k(piece, n, gi);
}

}  // namespace

// RT rows x 32 tokens a workgroup; tile (token tile first, then row tile) by
// blockIdx.x. LDS: each wave's two staging buffers ([32 k][RT] weights, then
// [32 k][32] inputs), reused after the K loop for the range sums [32][RT][32].
template <uint32_t F, uint32_t RT, bool FULL>
__global__ __launch_bounds__(256) void gemm_short(Product a, uint32_t token_tiles) {
    constexpr uint32_t kPairs = RT / 2;          // a wave's lanes along rows (row pairs)
    constexpr uint32_t kTq = 64 / kPairs;        // lanes along tokens: 8 (RT = 16) or 16 (RT = 8)
    constexpr uint32_t TT = kTokens / kTq;       // a lane's tokens: 4 or 2
    constexpr uint32_t kParts = 64 / RT;         // lanes staging one row's group: 4 or 8
    constexpr uint32_t kRun = 32 / kParts;       // weights each stages: 8 or 4
    constexpr uint32_t kBuf = 32 * (RT + kTokens);  // floats a staging buffer
    constexpr uint32_t kStage = kWaves * 2 * kBuf;
    constexpr uint32_t kSums = 32 * RT * kTokens;
    __shared__ float lds[kStage > kSums ? kStage : kSums];

    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t tile_t = blockIdx.x % token_tiles, tile_r = blockIdx.x / token_tiles;
    const uint32_t m0 = tile_t * kTokens, n0 = tile_r * RT;
    const uint32_t G = a.groups, K = G * 32;
    const uint32_t g_lo = range_lo(8 * wave, G), g_hi = range_lo(8 * wave + 8, G);

    // Staging roles. Weights: row lane % RT of the tile, its group's weights
    // kRun (lane / RT) .. + kRun - 1. Inputs: token lane % 32, floats
    // 16 (lane / 32) .. + 15 of the group.
    const uint32_t srow = lane % RT, spart = lane / RT;
    const uint32_t sp = n0 + srow;
    const bool slive = sp < a.rows;
    const Piece spiece = piece_of(a, slive ? sp : 0);
    const uint32_t xtok = lane & 31u, xhalf = lane >> 5;
    const bool xlive = m0 + xtok < a.tokens;
    const float* xsrc = a.x + static_cast<uint64_t>(xlive ? m0 + xtok : 0) * K + 16 * xhalf;

    // The lane's micro-tile: rows n0 + 2 pr, + 1; tokens m0 + TT tq + i.
    const uint32_t pr = lane % kPairs, tq = lane / kPairs;

    decltype(fetch_short<F, kRun>(nullptr, 0, 0, 0)) staged{};
    float4 xnext[4];
    auto fetch = [&](uint32_t g) {
        if (slive)
            staged = fetch_short<F, kRun>(spiece.piece, spiece.blocks, static_cast<uint64_t>(spiece.row) * G + g,
                                          kRun * spart);
        if (xlive) {
            const float4* src = reinterpret_cast<const float4*>(xsrc + g * 32);
#pragma unroll
            for (int v = 0; v < 4; ++v) xnext[v] = src[v];
        }
    };
    float* const mine = lds + wave * 2 * kBuf;
    auto stage = [&](uint32_t b) {
        float* ws = mine + b * kBuf;         // [32 k][RT]
        float* xs = ws + 32 * RT;            // [32 k][32 tokens]
        if constexpr (plain_values(F)) {
#pragma unroll
            for (uint32_t j = 0; j < kRun; ++j)
                ws[(kRun * spart + j) * RT + srow] = slive ? value_of(staged, j) : 0.0f;
        } else {
            const auto grp = group_of(staged);
#pragma unroll
            for (uint32_t j = 0; j < kRun; ++j)
                ws[(kRun * spart + j) * RT + srow] = slive ? weight_at(grp, kRun * spart + j) : 0.0f;
        }
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const float4 q = xlive ? clamp_input(a, xnext[v]) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            xs[(16 * xhalf + 4 * v) * kTokens + xtok] = q.x;
            xs[(16 * xhalf + 4 * v + 1) * kTokens + xtok] = q.y;
            xs[(16 * xhalf + 4 * v + 2) * kTokens + xtok] = q.z;
            xs[(16 * xhalf + 4 * v + 3) * kTokens + xtok] = q.w;
        }
    };
    // LDS operations of one wave complete in the order issued, so a wave
    // reading what its own lanes wrote needs no barrier; these keep the
    // compiler from moving LDS accesses across the hand-off.
    auto wave_sync = [] {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };

    float rs[8][2 * TT];
    if (g_lo < g_hi) {
        fetch(g_lo);
        stage(0);
    }
    if (g_lo + 1 < g_hi) fetch(g_lo + 1);
    uint32_t g = g_lo;
#pragma unroll
    for (int lr = 0; lr < 8; ++lr) {
        const uint32_t g_end = range_lo(8 * wave + lr + 1, G);
        float s[2 * TT];
#pragma unroll
        for (int o = 0; o < 2 * static_cast<int>(TT); ++o) s[o] = 0.0f;
        for (; g < g_end; ++g) {
            const uint32_t b = (g - g_lo) & 1u;
            wave_sync();
            const float* ws = mine + b * kBuf;
            const float* xs = ws + 32 * RT;
#pragma unroll 8
            for (int k = 0; k < 32; ++k) {
                const float2 w = reinterpret_cast<const float2*>(ws + k * RT)[pr];
                float x[TT];
                if constexpr (TT == 4) {
                    const float4 v = reinterpret_cast<const float4*>(xs + k * kTokens)[tq];
                    x[0] = v.x, x[1] = v.y, x[2] = v.z, x[3] = v.w;
                } else {
                    const float2 v = reinterpret_cast<const float2*>(xs + k * kTokens)[tq];
                    x[0] = v.x, x[1] = v.y;
                }
#pragma unroll
                for (uint32_t i = 0; i < TT; ++i) {
                    s[2 * i] = __builtin_fmaf(w.x, x[i], s[2 * i]);
                    s[2 * i + 1] = __builtin_fmaf(w.y, x[i], s[2 * i + 1]);
                }
            }
            wave_sync();
            if (g + 1 < g_hi) stage(b ^ 1u);
            if (g + 2 < g_hi) fetch(g + 2);
        }
#pragma unroll
        for (int o = 0; o < 2 * static_cast<int>(TT); ++o) rs[lr][o] = s[o];
    }

    // The range sums meet in LDS, [range][row][token], over the staging.
    __syncthreads();
#pragma unroll
    for (int lr = 0; lr < 8; ++lr)
#pragma unroll
        for (uint32_t i = 0; i < TT; ++i)
#pragma unroll
            for (uint32_t h = 0; h < 2; ++h)
                lds[((8 * wave + lr) * RT + 2 * pr + h) * kTokens + TT * tq + i] = rs[lr][2 * i + h];
    __syncthreads();

    // Lane c adds rows 2 (c / 32), + 1 of token c % 32: each output's 32 range
    // sums in order from zero, the empty ranges skipped.
    const uint32_t c = threadIdx.x;
    if (c >= kPairs * kTokens) return;
    const uint32_t token = m0 + (c & 31u), p0 = n0 + 2 * (c >> 5);
    float tot[2] = {0.0f, 0.0f};
#pragma unroll
    for (uint32_t r = 0; r < 32; ++r) {
        if (range_lo(r, G) == range_lo(r + 1, G)) continue;
#pragma unroll
        for (uint32_t h = 0; h < 2; ++h) tot[h] = tot[h] + lds[(r * RT + 2 * (c >> 5) + h) * kTokens + (c & 31u)];
    }
    if (token >= a.tokens) return;
#pragma unroll
    for (uint32_t h = 0; h < 2; ++h)
        if (p0 + h < a.rows) emit<FULL>(a, p0 + h, token, token, tot[h], h ? 0.0f : tot[1]);
}

template <uint32_t F, uint32_t RT>
static void go_short(const Product& a, const Plan& plan, hipStream_t stream) {
    const dim3 grid(plan.token_tiles * plan.row_tiles);
    if (plain_epilogue(a))
        hipLaunchKernelGGL((gemm_short<F, RT, false>), grid, dim3(256), 0, stream, a, plan.token_tiles);
    else
        hipLaunchKernelGGL((gemm_short<F, RT, true>), grid, dim3(256), 0, stream, a, plan.token_tiles);
}

template <uint32_t F>
static void go_short_format(const Product& a, const Plan& plan, hipStream_t stream) {
    if (plan.tile_rows == 16)
        go_short<F, 16>(a, plan, stream);
    else
        go_short<F, 8>(a, plan, stream);
}

// A short step's tile: 16 rows where that gives every CU two workgroups,
// else 8; 32 tokens.
void plan_gemm_short(const Product& a, uint32_t compute_units, Plan* plan) {
    *plan = Plan{};
    const uint32_t token_tiles = (a.tokens + kTokens - 1) / kTokens;
    const uint32_t rt = static_cast<uint64_t>(token_tiles) * ((a.rows + 15) / 16) >= 2ull * compute_units ? 16 : 8;
    plan->kernel = kGemmShort;
    plan->launches = 1;
    plan->tile_tokens = kTokens;
    plan->tile_rows = rt;
    plan->token_tiles = token_tiles;
    plan->row_tiles = (a.rows + rt - 1) / rt;
    plan->chunks = 1;
    plan->tiles = static_cast<uint64_t>(token_tiles) * plan->row_tiles;
    plan->workgroups = plan->tiles;
}

hipError_t launch_gemm_short(const Product& a, uint32_t format, const Plan& plan, hipStream_t stream) {
    switch (format) {
        case kQ4_0: go_short_format<kQ4_0>(a, plan, stream); break;
        case kQ4_1: go_short_format<kQ4_1>(a, plan, stream); break;
        case kQ8_0: go_short_format<kQ8_0>(a, plan, stream); break;
        case kQ6_K: go_short_format<kQ6_K>(a, plan, stream); break;
        case kF32: go_short_format<kF32>(a, plan, stream); break;
        case kF16: go_short_format<kF16>(a, plan, stream); break;
        case kBF16: go_short_format<kBF16>(a, plan, stream); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace chm
