// Prefill: the tiled matrix product over a step's tokens.
//
// gemm_canonical — VALU, the canonical order, bit-exact with decode and the
// CPU restatement (matmul.wgsl:395-533 restated for CDNA4). A workgroup of
// 256 lanes takes a tile of BM tokens x 128 rows and walks K one 32-weight
// group at a time: the group's 128 rows are decoded once into LDS (exact
// f32), the tokens' 32 inputs staged beside them, then each lane runs its
// micro-tile of TM tokens x 8 rows (BM = 32, 64 or 128: TM = 2, 4 or 8),
// 32 multiply-adds in k order per output, each output keeping its range sum
// and its total: at a range's last group
// the total adds the range sum and the range sum restarts from zero. So every
// output's order of addition is decode's, whatever BM. Workgroups are
// numbered token tile first, so the tiles that read one weight tile run
// together and find it in L2 (matmul.wgsl:480-482).
//
// Split along K (matmul.wgsl:592-695): the same tile over a chunk of the 32
// ranges only, each range sum written to `range_sums` range first,
// [32][tokens][rows]; the combine adds a row's 32 sums in order from zero.
// Range sums are the same bits either way, so split and tiled outputs agree.
#include "plan.hpp"
#include "product.hpp"

namespace chm {

constexpr int kRowsATile = 128;

// Where range r's sum of product row p for `token` lies (matmul.wgsl:603-605).
__device__ __forceinline__ uint64_t range_sum_at(const Product& a, uint32_t r, uint32_t token, uint32_t p) {
    return (static_cast<uint64_t>(r) * a.tokens + token) * a.rows + p;
}

// A group's bytes as loaded; group_of() makes the group weight() decodes.
// The unquantized formats load only the half (`half`, 16 values) the lane
// stages: their values are their bytes, 64 or 32 of them a half.
template <uint32_t F>
__device__ __forceinline__ auto fetch_group(const uint8_t* piece, uint64_t n, uint64_t gi, uint32_t half) {
    if constexpr (F == kQ4_0) return fetch_q4_0(piece, n, gi);
    else if constexpr (F == kQ4_1) return fetch_q4_1(piece, n, gi);
    else if constexpr (F == kQ8_0) return fetch_q8_0(piece, n, gi);
    else if constexpr (plain_values(F)) return fetch_values_half<F>(piece, gi, half);
    else return fetch_q6_k(piece, n, gi);
}

// SPLIT: `chunks` workgroups a tile, chunk c taking ranges [32c / chunks,
// 32(c + 1) / chunks) and writing their sums to `range_sums`; else one a
// tile, writing the outputs.
template <uint32_t F, int BM, bool SPLIT, bool FULL>
__global__ __launch_bounds__(256) void gemm_canonical(Product a, uint32_t token_tiles, uint32_t row_tiles,
                                                      uint32_t chunks, float* range_sums) {
    constexpr int TM = BM / 16;  // a lane's tokens
    // Token i of a lane's micro-tile: 2 ty + i (BM = 32); 4 ty + i % 4, and
    // + 64 for i >= 4 (BM = 64, 128).
    auto token_at = [&](uint32_t ty, int i) -> uint32_t {
        return TM == 2 ? 2 * ty + i : 4 * ty + (i & 3) + 64 * (i >> 2);
    };
    __shared__ float4 Ws[2][32][kRowsATile / 4];
    __shared__ float4 Xs[2][32][BM / 4];
    const uint32_t t = threadIdx.x, tx = t & 15u, ty = t >> 4;
    const uint32_t tile_t = blockIdx.x % token_tiles, tile_r = (blockIdx.x / token_tiles) % row_tiles;
    const uint32_t chunk = blockIdx.x / (token_tiles * row_tiles);
    const uint32_t r_begin = 32 * chunk / chunks, r_end = 32 * (chunk + 1) / chunks;
    const uint32_t m0 = tile_t * BM, n0 = tile_r * kRowsATile;
    const uint32_t G = a.groups, K = G * 32;

    // Staging roles: weights — row t % 128, weights 16 (t / 128) .. + 15 of
    // its group; inputs — BM tokens x 32 floats, BM / 8 floats a lane.
    const uint32_t srow = t & 127u, shalf = t >> 7;
    const uint32_t sp = n0 + srow;
    const bool slive = sp < a.rows;
    const Piece spiece = piece_of(a, slive ? sp : 0);
    constexpr int XPer = BM / 8;                 // floats a lane stages: 16, 8 or 4
    const uint32_t xtok = t % BM, xpart = t / BM;
    const bool xlive = m0 + xtok < a.tokens;
    const float* xsrc = a.x + static_cast<uint64_t>(m0 + xtok) * K + xpart * XPer;

    float s[TM][8], tot[TM][8];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) s[i][j] = tot[i][j] = 0.0f;

    // The range that ends after group g is the one before `next_r`'s first
    // group; ranges with no groups hold zero and add nothing to a total, which
    // is never -0.
    uint32_t next_r = r_begin + 1;
    const uint32_t g_begin = range_lo(r_begin, G), g_end = range_lo(r_end, G);
    while (next_r < r_end && range_lo(next_r, G) <= g_begin) ++next_r;

    // Two tiles in LDS: group g's products read one while group g + 1 is
    // staged into the other, one barrier a group. Group g + 2's stored bytes
    // and inputs are loaded into registers behind that barrier, so their round
    // trip overlaps group g + 1's arithmetic.
    decltype(fetch_group<F>(nullptr, 0, 0, 0)) staged{};
    float4 xnext[XPer / 4];
    auto fetch = [&](uint32_t g) {
        if (slive)
            staged = fetch_group<F>(spiece.piece, spiece.blocks, static_cast<uint64_t>(spiece.row) * G + g, shalf);
        if (xlive) {
            const float4* src = reinterpret_cast<const float4*>(xsrc + g * 32);
#pragma unroll
            for (int v = 0; v < XPer / 4; ++v) xnext[v] = src[v];
        }
    };
    auto stage = [&](int b) {
        float* wflat = reinterpret_cast<float*>(Ws[b]);
        float* xflat = reinterpret_cast<float*>(Xs[b]);
        if constexpr (plain_values(F)) {
#pragma unroll
            for (int j = 0; j < 16; ++j)
                wflat[(16 * shalf + j) * kRowsATile + srow] = slive ? value<F>(staged, j) : 0.0f;
        } else if constexpr (F == kQ8_0) {
            // The lane's half of the codes chosen by a select, so every index
            // below is a constant (an index by shalf would go through scratch).
            const auto grp = group_of(staged);
            uint32_t hw[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) hw[k] = shalf ? grp.w[4 + k] : grp.w[k];
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int32_t q = static_cast<int8_t>((hw[j >> 2] >> (8 * (j & 3))) & 0xFFu);
                wflat[(16 * shalf + j) * kRowsATile + srow] = slive ? static_cast<float>(q) * grp.d : 0.0f;
            }
        } else {
            const auto grp = group_of(staged);
#pragma unroll
            for (int j = 0; j < 16; ++j)
                wflat[(16 * shalf + j) * kRowsATile + srow] = slive ? weight(grp, 16 * shalf + j) : 0.0f;
        }
#pragma unroll
        for (int v = 0; v < XPer / 4; ++v) {
            const float4 q = xlive ? clamp_input(a, xnext[v]) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            xflat[(xpart * XPer + 4 * v) * BM + xtok] = q.x;
            xflat[(xpart * XPer + 4 * v + 1) * BM + xtok] = q.y;
            xflat[(xpart * XPer + 4 * v + 2) * BM + xtok] = q.z;
            xflat[(xpart * XPer + 4 * v + 3) * BM + xtok] = q.w;
        }
    };
    if (g_begin < g_end) {
        fetch(g_begin);
        stage(0);
    }
    __syncthreads();
    if (g_begin + 1 < g_end) fetch(g_begin + 1);

    for (uint32_t g = g_begin; g < g_end; ++g) {
        const int b = (g - g_begin) & 1;
#pragma unroll 4
        for (int k = 0; k < 32; ++k) {
            const float4 wa = Ws[b][k][tx], wb = Ws[b][k][16 + tx];
            const float w[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
            float x[TM];
            if constexpr (TM == 2) {
                const float2 xa = reinterpret_cast<const float2*>(Xs[b][k])[ty];
                x[0] = xa.x;
                x[1] = xa.y;
            } else {
                const float4 xa = Xs[b][k][ty];
                x[0] = xa.x;
                x[1] = xa.y;
                x[2] = xa.z;
                x[3] = xa.w;
            }
            if constexpr (TM == 8) {
                const float4 xb = Xs[b][k][16 + ty];
                x[4] = xb.x;
                x[5] = xb.y;
                x[6] = xb.z;
                x[7] = xb.w;
            }
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < 8; ++j) s[i][j] = __builtin_fmaf(w[j], x[i], s[i][j]);
        }
        if (g + 1 == range_lo(next_r, G)) {  // range next_r - 1 ends
            if constexpr (SPLIT) {
#pragma unroll
                for (int i = 0; i < TM; ++i) {
                    const uint32_t token = m0 + token_at(ty, i);
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const uint32_t p = n0 + 4 * tx + (j & 3) + 64 * (j >> 2);
                        if (token < a.tokens && p < a.rows) range_sums[range_sum_at(a, next_r - 1, token, p)] = s[i][j];
                        s[i][j] = 0.0f;
                    }
                }
            } else {
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        tot[i][j] = tot[i][j] + s[i][j];
                        s[i][j] = 0.0f;
                    }
            }
            while (next_r < r_end && range_lo(next_r, G) <= g + 1) ++next_r;
        }
        // Group g + 1 into the other tile, last read by group g - 1's products
        // before the previous barrier.
        if (g + 1 < g_end) stage(b ^ 1);
        __syncthreads();
        if (g + 2 < g_end) fetch(g + 2);
    }
    if constexpr (SPLIT) return;

    // Rows p, p + 1 of a micro-tile (j, j + 1 for even j) are adjacent, so a
    // gated product's gate and up totals meet in one lane.
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const uint32_t token = m0 + token_at(ty, i);
        if (token >= a.tokens) continue;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t p = n0 + 4 * tx + (j & 3) + 64 * (j >> 2);
            if (p < a.rows) emit<FULL>(a, p, token, token, tot[i][j], (j & 1) ? 0.0f : tot[i][j ^ 1]);
        }
    }
}

// The combine (matmul.wgsl:621-695): a lane an output of each token, its 32
// range sums added in order to a total from zero, then the epilogue. Empty
// ranges (G < 32) are never written by the split form and add nothing.
__global__ __launch_bounds__(256) void combine_ranges(Product a, const float* range_sums) {
    const uint64_t id = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (id >= static_cast<uint64_t>(a.tokens) * a.rows) return;
    const uint32_t token = static_cast<uint32_t>(id / a.rows), p = static_cast<uint32_t>(id % a.rows);
    // All 32 loads issued before the first add — every range's slot lies in
    // the buffer, written or not — then the non-empty ranges added in order.
    float sums[32];
#pragma unroll
    for (uint32_t r = 0; r < 32; ++r) sums[r] = range_sums[range_sum_at(a, r, token, p)];
    float total = 0.0f;
#pragma unroll
    for (uint32_t r = 0; r < 32; ++r)
        if (range_lo(r, a.groups) < range_lo(r + 1, a.groups)) total = total + sums[r];
    emit<true>(a, p, token, token, total, 0.0f);
}

template <uint32_t F, int BM>
static void go(const Product& a, const Plan& plan, float* range_sums, hipStream_t stream) {
    const dim3 grid(plan.token_tiles * plan.row_tiles * plan.chunks);
    if (range_sums)
        hipLaunchKernelGGL((gemm_canonical<F, BM, true, false>), grid, dim3(256), 0, stream, a, plan.token_tiles,
                           plan.row_tiles, plan.chunks, range_sums);
    else if (plain_epilogue(a))
        hipLaunchKernelGGL((gemm_canonical<F, BM, false, false>), grid, dim3(256), 0, stream, a, plan.token_tiles,
                           plan.row_tiles, 1u, nullptr);
    else
        hipLaunchKernelGGL((gemm_canonical<F, BM, false, true>), grid, dim3(256), 0, stream, a, plan.token_tiles,
                           plan.row_tiles, 1u, nullptr);
}

template <uint32_t F>
static void go_format(const Product& a, const Plan& plan, float* range_sums, hipStream_t stream) {
    if (plan.tile_tokens == 128)
        go<F, 128>(a, plan, range_sums, stream);
    else if (plan.tile_tokens == 32)
        go<F, 32>(a, plan, range_sums, stream);
    else
        go<F, 64>(a, plan, range_sums, stream);
}

// The tile: 128 tokens where that still gives every CU two workgroups, 32
// for a short step (no lanes on absent tokens), else 64. Split along K, the
// ranges cut into as few chunks as still give every CU two workgroups.
void plan_gemm_canonical(const Product& a, uint32_t compute_units, bool split, Plan* plan) {
    *plan = Plan{};
    const uint32_t row_tiles = (a.rows + kRowsATile - 1) / kRowsATile;
    const bool wide = static_cast<uint64_t>((a.tokens + 127) / 128) * row_tiles >= 2ull * compute_units;
    const bool narrow = a.tokens <= 32;
    const uint32_t bm = wide ? 128 : narrow ? 32 : 64;
    const uint32_t token_tiles = (a.tokens + bm - 1) / bm;
    uint32_t chunks = 1;
    if (split) {
        chunks = 2;
        while (chunks < 32 && static_cast<uint64_t>(token_tiles) * row_tiles * chunks < 2ull * compute_units)
            chunks *= 2;
    }
    plan->kernel = split ? kGemmSplit : kGemmTiled;
    plan->launches = split ? 2 : 1;
    plan->tile_tokens = bm;
    plan->tile_rows = kRowsATile;
    plan->token_tiles = token_tiles;
    plan->row_tiles = row_tiles;
    plan->chunks = chunks;
    plan->tiles = static_cast<uint64_t>(token_tiles) * row_tiles;
    plan->workgroups = plan->tiles * chunks;
}

// The combine of a split product's range sums (every output of every token).
hipError_t launch_combine_ranges(const Product& a, const float* range_sums, hipStream_t stream) {
    const uint64_t outputs = static_cast<uint64_t>(a.tokens) * a.rows;
    hipLaunchKernelGGL(combine_ranges, dim3(static_cast<uint32_t>((outputs + 255) / 256)), dim3(256), 0, stream, a,
                       range_sums);
    return hipGetLastError();
}

// The tiled form; with `range_sums` (room for 32 x tokens x rows floats), the
// split form and its combine.
hipError_t launch_gemm_canonical(const Product& a, uint32_t format, const Plan& plan, float* range_sums,
                                 hipStream_t stream) {
    switch (format) {
        case kQ4_0: go_format<kQ4_0>(a, plan, range_sums, stream); break;
        case kQ4_1: go_format<kQ4_1>(a, plan, range_sums, stream); break;
        case kQ8_0: go_format<kQ8_0>(a, plan, range_sums, stream); break;
        case kQ6_K: go_format<kQ6_K>(a, plan, range_sums, stream); break;
        case kF32: go_format<kF32>(a, plan, range_sums, stream); break;
        case kF16: go_format<kF16>(a, plan, range_sums, stream); break;
        case kBF16: go_format<kBF16>(a, plan, range_sums, stream); break;
        default: return hipErrorInvalidValue;
    }
    if (range_sums) return launch_combine_ranges(a, range_sums, stream);
    return hipGetLastError();
}

}  // namespace chm
