// Prefill on the matrix cores (the SPLIT_F16_MFMA path): within the stated
// tolerance, not bit-exact — the canonical VALU tile keeps the reference's
// order; this one trades it for throughput.
//
// The weights' codes are exact in binary16 (Q4_0 q - 8, Q6_K q - 32); the
// block scale stays out of the product and is applied in f32 after it. The
// input is split in two binary16 parts per token: x 2^s = hi + lo with
// hi = f16(x 2^s), lo = f16(x 2^s - hi), s a power of two per token putting
// its largest |x| in [2^14, 2^15) — so neither part overflows, and lo keeps
// the bits hi drops (about 22 bits of x in all, relative to the token's
// largest). Each group's product is two matrix-core multiplies into f32,
//   P = codes . hi + codes . lo       (products of f16 values are exact in f32)
// and the output row accumulates total = fma(scale, P, total) a group at a
// time, then y = total 2^-s. The error is that of f32 accumulation, far
// inside max |err| / max |y| <= 1e-5.
//
// Layout: prepare_x writes the split input once a step into the workspace,
// [G][tokens][4 quarters][hi 8 halves | lo 8 halves]: quarter q of group g
// holds x[4q .. 4q+3] and x[16+4q .. 16+4q+3] — the weights a lane of
// quarter q decodes from code dword q of a Q4_0 group (low nibbles, then
// high), and the two 16-weight halves of a Q6_K group. A wave takes R x 16
// weight rows by T x 16 tokens; v_mfma_f32_16x16x32_f16 (Q4_0) and
// v_mfma_f32_16x16x16_f16 (Q6_K, one a half: its scale differs) with the
// input as the A operand, so a lane's four outputs are four tokens of one
// weight row and need one scale. A workgroup's four waves share its tokens:
// their split input is staged once through LDS; each wave's codes go from the
// piece straight into registers. Both are loaded four groups ahead.
#include <type_traits>

#include "decode.hpp"
#include "product.hpp"

namespace chm {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr uint32_t kTokenPad = 64;  // prepared tokens: a multiple of the widest wave tile

uint64_t mfma_padded_tokens(uint32_t tokens) { return (uint64_t{tokens} + kTokenPad - 1) / kTokenPad * kTokenPad; }

uint64_t mfma_workspace_bytes(uint32_t tokens, uint32_t groups) {
    const uint64_t m = mfma_padded_tokens(tokens);
    return m * groups * 128 + m * 4;
}

// One workgroup a token (padded tokens get zeros): the token's scale 2^s,
// then its groups split into hi and lo, clamped first where the product is
// clipped.
__global__ __launch_bounds__(256) void prepare_x(Product a, uint8_t* __restrict__ xp, float* __restrict__ inv) {
    __shared__ float largest[4];
    const uint32_t t = blockIdx.x, G = a.groups;
    const bool live = t < a.tokens;
    const float4* x = reinterpret_cast<const float4*>(a.x + static_cast<uint64_t>(live ? t : 0) * G * 32);
    float m = 0.0f;
    if (live) {
        for (uint32_t v = threadIdx.x; v < G * 8; v += 256) {
            const float4 q = clamp_input(a, x[v]);
            m = fmaxf(m, fmaxf(fmaxf(fabsf(q.x), fabsf(q.y)), fmaxf(fabsf(q.z), fabsf(q.w))));
        }
    }
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if ((threadIdx.x & 63u) == 0) largest[threadIdx.x >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(largest[0], largest[1]), fmaxf(largest[2], largest[3]));
    int s = 0;
    if (m > 0.0f && m <= 3.4e38f) {
        int e = 0;
        (void)frexpf(m, &e);  // m in [2^(e-1), 2^e)
        s = min(max(15 - e, -126), 126);
    }
    if (threadIdx.x == 0) inv[t] = ldexpf(1.0f, -s);
    for (uint32_t v = threadIdx.x; v < G * 4; v += 256) {
        const uint32_t g = v >> 2, q = v & 3u;
        float e[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        if (live) {
            const float4 a0 = clamp_input(a, x[8 * g + q]), a1 = clamp_input(a, x[8 * g + 4 + q]);
            e[0] = a0.x, e[1] = a0.y, e[2] = a0.z, e[3] = a0.w;
            e[4] = a1.x, e[5] = a1.y, e[6] = a1.z, e[7] = a1.w;
        }
        half8_t hi, lo;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float xs = ldexpf(e[i], s);
            hi[i] = static_cast<_Float16>(xs);
            lo[i] = static_cast<_Float16>(xs - static_cast<float>(hi[i]));
        }
        half8_t* out = reinterpret_cast<half8_t*>(xp + ((static_cast<uint64_t>(g) * gridDim.x + t) * 4 + q) * 32);
        out[0] = hi;
        out[1] = lo;
    }
}

// A lane's weights of one group, as loaded: Q4_0 one code dword and the fp16
// scale; Q6_K a lo dword, a hi dword, the group's two int8 scales and d.
template <uint32_t F>
struct Codes;

template <>
struct Codes<kQ4_0> {
    uint32_t code;
    uint32_t d;
};

template <>
struct Codes<kQ6_K> {
    uint32_t lo, hi;
    uint32_t sc;  // two int8, low byte first
    uint32_t d;
};

// Where a lane's row of a wave's row block reads: the piece and the row's
// first group.
struct RowAt {
    const uint8_t* piece;
    uint64_t blocks;
    uint64_t gi0;
};

template <uint32_t F>
__device__ __forceinline__ Codes<F> load_codes(const RowAt& w, uint32_t g, uint32_t q) {
    const uint64_t gi = w.gi0 + g;
    Codes<F> c;
    if constexpr (F == kQ4_0) {
        c.code = *reinterpret_cast<const uint32_t*>(w.piece + 16 * gi + 4 * q);
        c.d = *reinterpret_cast<const uint16_t*>(w.piece + 16 * w.blocks + 2 * gi);
    } else {
        const uint64_t n = w.blocks;
        c.lo = *reinterpret_cast<const uint32_t*>(w.piece + 16 * gi + 4 * q);
        c.hi = *reinterpret_cast<const uint32_t*>(w.piece + 128 * n + 8 * gi + 4 * (q & 1u));
        c.sc = *reinterpret_cast<const uint16_t*>(w.piece + 192 * n + 2 * gi);
        c.d = *reinterpret_cast<const uint16_t*>(w.piece + 208 * n + 2 * (gi >> 3));
    }
    return c;
}

__device__ __forceinline__ half2_t lift_less(uint32_t codes, uint32_t selector, _Float16 bias) {
    half2_t v = lift(codes, selector);
    const half2_t b = {bias, bias};
    return v - b;  // (1024 + q) - (1024 + bias) = q - bias, exact in binary16
}

// A workgroup's four waves share its T x 16 tokens and take R x 16 rows
// each. The tokens' split input moves through LDS, two buffers of one group
// each: a group's 128 bytes a token are loaded into registers kDepth groups
// ahead (all 256 lanes, 16 bytes each), written to the buffer the group after
// next will not need, and read back as A operands. Each wave loads its rows'
// codes into registers kDepth groups ahead too. 16-byte chunk k of token t
// sits at chunk k ^ (t & 7), so the 16 tokens a read takes spread over the
// banks.
constexpr int kDepth = 4;

template <uint32_t F, int R, int T, bool FULL>
__global__ __launch_bounds__(256, 2) void gemm_mfma(Product a, const uint8_t* __restrict__ xp,
                                                   const float* __restrict__ inv, uint32_t token_tiles,
                                                   uint32_t padded_tokens) {
    constexpr int BM = T * 16;
    constexpr int XC = BM * 8 / 256;  // 16-byte chunks a lane stages a group
    __shared__ u32x4_t xs[2][BM * 8];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t q = lane >> 4, c = lane & 15u;
    const uint32_t tile_t = blockIdx.x % token_tiles, tile_r = blockIdx.x / token_tiles;
    const uint32_t tok0 = tile_t * BM, row0 = (tile_r * 4 + wave) * R * 16;
    const uint32_t G = a.groups;

    RowAt rows[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t p = min(row0 + 16 * r + c, a.rows - 1);
        const Piece w = piece_of(a, p);
        rows[r] = {w.piece, w.blocks, static_cast<uint64_t>(w.row) * G};
    }
    // Staging: chunk j = threadIdx.x + 256 i of the tile's group: token j / 8,
    // chunk j % 8 of its 128 bytes.
    const u32x4_t* xsrc = reinterpret_cast<const u32x4_t*>(xp + static_cast<uint64_t>(tok0) * 128);
    const uint64_t group_chunks = static_cast<uint64_t>(padded_tokens) * 8;
    uint32_t slot[XC];
#pragma unroll
    for (int i = 0; i < XC; ++i) {
        const uint32_t j = threadIdx.x + 256 * i, t = j >> 3;
        slot[i] = t * 8 + ((j & 7u) ^ (t & 7u));
    }
    auto load_x = [&](u32x4_t (&v)[XC], uint32_t g) {
#pragma unroll
        for (int i = 0; i < XC; ++i) v[i] = xsrc[g * group_chunks + threadIdx.x + 256 * i];
    };
    auto store_x = [&](const u32x4_t (&v)[XC], uint32_t buf) {
#pragma unroll
        for (int i = 0; i < XC; ++i) xs[buf][slot[i]] = v[i];
    };

    float4_t tot[R][T];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int t = 0; t < T; ++t) tot[r][t] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};

    u32x4_t xr[kDepth][XC];
    Codes<F> wr[kDepth][R];
#pragma unroll
    for (int d = 0; d < kDepth; ++d) {
        const uint32_t g = d < G ? d : G - 1;
        load_x(xr[d], g);
#pragma unroll
        for (int r = 0; r < R; ++r) wr[d][r] = load_codes<F>(rows[r], g, q);
    }
    store_x(xr[0], 0);

    // One group's step; d = g % kDepth names the register slots at compile
    // time, so they stay registers.
    auto step = [&](uint32_t g0, auto slot_d) {
        constexpr int d = decltype(slot_d)::value;
        {
            const uint32_t g = g0 + d;
            __syncthreads();  // buffer g & 1 is written; buffer (g + 1) & 1 is read no more
            if (g + 1 < G) store_x(xr[(d + 1) % kDepth], (g + 1) & 1u);
            const uint32_t ahead = g + kDepth < G ? g + kDepth : G - 1;
            load_x(xr[d], ahead);
            if (g < G) {
                const u32x4_t* buf = xs[g & 1u];
                half8_t xh[T], xl[T];
#pragma unroll
                for (int t = 0; t < T; ++t) {
                    const uint32_t tok = 16 * t + c;
                    xh[t] = __builtin_bit_cast(half8_t, buf[tok * 8 + ((2 * q) ^ (tok & 7u))]);
                    xl[t] = __builtin_bit_cast(half8_t, buf[tok * 8 + ((2 * q + 1) ^ (tok & 7u))]);
                }
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const Codes<F>& cw = wr[d][r];
                    if constexpr (F == kQ4_0) {
                        const uint32_t lo = cw.code & 0x0F0F0F0Fu, hi = (cw.code >> 4) & 0x0F0F0F0Fu;
                        const half2_t b0 = lift_less(lo, kLowPair, 1032.0f16), b1 = lift_less(lo, kHighPair, 1032.0f16);
                        const half2_t b2 = lift_less(hi, kLowPair, 1032.0f16), b3 = lift_less(hi, kHighPair, 1032.0f16);
                        const half8_t b = {b0.x, b0.y, b1.x, b1.y, b2.x, b2.y, b3.x, b3.y};
                        const float s = half_to_float(cw.d);
#pragma unroll
                        for (int t = 0; t < T; ++t) {
                            float4_t p = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh[t], b, float4_t{0.0f, 0.0f, 0.0f, 0.0f},
                                                                                0, 0, 0);
                            p = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl[t], b, p, 0, 0, 0);
#pragma unroll
                            for (int k = 0; k < 4; ++k) tot[r][t][k] = __builtin_fmaf(s, p[k], tot[r][t][k]);
                        }
                    } else {
                        // Codes of weights 4q .. 4q+3 (half 0) and 16+4q .. 16+4q+3
                        // (half 1): low nibbles from lo, high pairs from hi.
                        const uint32_t up = q >> 1;
                        const uint32_t h0 = (cw.hi >> (2 * up)) & 0x03030303u;
                        const uint32_t h1 = (cw.hi >> (2 * (2 + up))) & 0x03030303u;
                        const uint32_t c0 = (cw.lo & 0x0F0F0F0Fu) | (h0 << 4);
                        const uint32_t c1 = ((cw.lo >> 4) & 0x0F0F0F0Fu) | (h1 << 4);
                        const half2_t a0 = lift_less(c0, kLowPair, 1056.0f16), a1 = lift_less(c0, kHighPair, 1056.0f16);
                        const half2_t a2 = lift_less(c1, kLowPair, 1056.0f16), a3 = lift_less(c1, kHighPair, 1056.0f16);
                        const half4_t b0 = {a0.x, a0.y, a1.x, a1.y}, b1 = {a2.x, a2.y, a3.x, a3.y};
                        const float dd = half_to_float(cw.d);
                        const float s0 = dd * static_cast<float>(static_cast<int8_t>(cw.sc & 0xFFu));
                        const float s1 = dd * static_cast<float>(static_cast<int8_t>((cw.sc >> 8) & 0xFFu));
#pragma unroll
                        for (int t = 0; t < T; ++t) {
                            const half4_t h0x = {xh[t][0], xh[t][1], xh[t][2], xh[t][3]};
                            const half4_t l0x = {xl[t][0], xl[t][1], xl[t][2], xl[t][3]};
                            const half4_t h1x = {xh[t][4], xh[t][5], xh[t][6], xh[t][7]};
                            const half4_t l1x = {xl[t][4], xl[t][5], xl[t][6], xl[t][7]};
                            const float4_t z = {0.0f, 0.0f, 0.0f, 0.0f};
                            float4_t p0 = __builtin_amdgcn_mfma_f32_16x16x16f16(h0x, b0, z, 0, 0, 0);
                            float4_t p1 = __builtin_amdgcn_mfma_f32_16x16x16f16(h1x, b1, z, 0, 0, 0);
                            p0 = __builtin_amdgcn_mfma_f32_16x16x16f16(l0x, b0, p0, 0, 0, 0);
                            p1 = __builtin_amdgcn_mfma_f32_16x16x16f16(l1x, b1, p1, 0, 0, 0);
#pragma unroll
                            for (int k = 0; k < 4; ++k) {
                                tot[r][t][k] = __builtin_fmaf(s0, p0[k], tot[r][t][k]);
                                tot[r][t][k] = __builtin_fmaf(s1, p1[k], tot[r][t][k]);
                            }
                        }
                    }
                }
            }
#pragma unroll
            for (int r = 0; r < R; ++r) wr[d][r] = load_codes<F>(rows[r], ahead, q);
        }
    };
    for (uint32_t g0 = 0; g0 < G; g0 += kDepth) {
        step(g0, std::integral_constant<int, 0>{});
        step(g0, std::integral_constant<int, 1>{});
        step(g0, std::integral_constant<int, 2>{});
        step(g0, std::integral_constant<int, 3>{});
    }
    static_assert(kDepth == 4, "one step call a slot");

    // Lane (c, q) holds tokens 4q .. 4q+3 of each token block for row c of
    // each row block; rows c and c ^ 1 (a gated product's gate and up) are
    // adjacent lanes.
#pragma unroll
    for (int t = 0; t < T; ++t) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t token = tok0 + 16 * t + 4 * q + k;
            const float unscale = inv[token];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float v = tot[r][t][k] * unscale;
                float partner = 0.0f;
                if (FULL && a.epilogue == kGated) partner = __shfl_xor(v, 1);
                const uint32_t p = row0 + 16 * r + c;
                if (token < a.tokens && p < a.rows) emit<FULL>(a, p, token, token, v, partner);
            }
        }
    }
}

template <uint32_t F, int R, int T>
static void go(const Product& a, const uint8_t* xp, const float* inv, hipStream_t stream) {
    const uint32_t token_tiles = (a.tokens + T * 16 - 1) / (T * 16);
    const uint32_t row_tiles = (a.rows + 64 * R - 1) / (64 * R);
    const uint32_t m = static_cast<uint32_t>(mfma_padded_tokens(a.tokens));
    const dim3 grid(token_tiles * row_tiles);
    if (plain_epilogue(a))
        hipLaunchKernelGGL((gemm_mfma<F, R, T, false>), grid, dim3(256), 0, stream, a, xp, inv, token_tiles, m);
    else
        hipLaunchKernelGGL((gemm_mfma<F, R, T, true>), grid, dim3(256), 0, stream, a, xp, inv, token_tiles, m);
}

// The widest wave tile that still gives every SIMD two waves, else the
// smallest. Q6_K's 4 x 4 tile would not fit two waves' registers.
template <uint32_t F>
static void launch_format(const Product& a, const uint8_t* xp, const float* inv, uint32_t compute_units,
                          hipStream_t stream) {
    const auto waves = [&](int r, int t) {
        return uint64_t{(a.tokens + 16u * t - 1) / (16u * t)} * ((a.rows + 16u * r - 1) / (16u * r));
    };
    const uint64_t want = uint64_t{compute_units} * 8;
    if constexpr (F == kQ4_0) {
        if (waves(4, 4) >= want) return go<F, 4, 4>(a, xp, inv, stream);
    }
    if (waves(2, 4) >= want)
        go<F, 2, 4>(a, xp, inv, stream);
    else
        go<F, 2, 2>(a, xp, inv, stream);
}

hipError_t launch_gemm_mfma(const Product& a, uint32_t format, uint32_t compute_units, void* workspace,
                            hipStream_t stream) {
    const uint64_t m = mfma_padded_tokens(a.tokens);
    uint8_t* xp = static_cast<uint8_t*>(workspace);
    float* inv = reinterpret_cast<float*>(xp + m * a.groups * 128);
    hipLaunchKernelGGL(prepare_x, dim3(static_cast<uint32_t>(m)), dim3(256), 0, stream, a, xp, inv);
    if (format == kQ4_0)
        launch_format<kQ4_0>(a, xp, inv, compute_units, stream);
    else
        launch_format<kQ6_K>(a, xp, inv, compute_units, stream);
    return hipGetLastError();
}

}  // namespace chm
