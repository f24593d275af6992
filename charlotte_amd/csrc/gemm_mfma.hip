// Prefill on the matrix cores (the SPLIT_F16_MFMA path): within the stated
// tolerance, not bit-exact — the canonical VALU tile keeps the reference's
// order; this one trades it for throughput.
//
// The weights' codes are exact in binary16 (Q4_0 q - 8, Q6_K q - 32, Q8_0 q,
// Q4_1 q); the block scale stays out of the product and is applied in f32
// after it. Q4_1's minimum m multiplies the group's sum of inputs, which one
// more product against all-ones codes gives for every row at once:
// total = fma(d, P, fma(m, S, total)), S = ones . hi + ones . lo. The
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
// weight row and need one scale. Q8_0 and Q4_1 go as Q4_0 does, their codes
// group by group. A workgroup's four waves share its tokens: their split
// input is copied once a batch from the workspace straight into LDS
// (global_load_lds, no register round trip); each wave's codes go from the
// piece straight into registers. Both are loaded a batch of groups ahead.
#include <type_traits>

#include "decode.hpp"
#include "stream.hpp"
#include "plan.hpp"
#include "product.hpp"

namespace chm {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr uint32_t kTokenPad = 64;  // prepared tokens: a multiple of the widest wave tile
constexpr int kBatch = 4;          // groups a batch of the matrix-core loop

uint64_t mfma_padded_tokens(uint32_t tokens) { return (uint64_t{tokens} + kTokenPad - 1) / kTokenPad * kTokenPad; }

uint64_t mfma_workspace_bytes(uint32_t tokens, uint32_t groups) {
    const uint64_t m = mfma_padded_tokens(tokens);
    return m * groups * 128 + m * 4;
}

// A wave's 16-byte copy into LDS: lane L's 16 bytes from `from` land at
// to + 16 L (`to` the same for every lane).
__device__ __forceinline__ void dma16(const uint8_t* from, u32x4_t* to) {
    __builtin_amdgcn_global_load_lds(from, (lds_void)to, 16, 0, 0);
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

template <>
struct Codes<kQ8_0> {
    uint32_t c0, c1;  // codes 4q .. 4q+3 and 16+4q .. 16+4q+3
    uint32_t d;
};

template <>
struct Codes<kQ4_1> {
    uint32_t code;
    uint32_t dm;  // d low, m high
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
    } else if constexpr (F == kQ8_0) {
        c.c0 = *reinterpret_cast<const uint32_t*>(w.piece + 32 * gi + 4 * q);
        c.c1 = *reinterpret_cast<const uint32_t*>(w.piece + 32 * gi + 16 + 4 * q);
        c.d = *reinterpret_cast<const uint16_t*>(w.piece + 32 * w.blocks + 2 * gi);
    } else if constexpr (F == kQ4_1) {
        c.code = *reinterpret_cast<const uint32_t*>(w.piece + 16 * gi + 4 * q);
        c.dm = *reinterpret_cast<const uint32_t*>(w.piece + 16 * w.blocks + 4 * gi);
    } else {
        const uint64_t n = w.blocks;
        c.lo = *reinterpret_cast<const uint32_t*>(w.piece + 16 * gi + 4 * q);
        c.hi = *reinterpret_cast<const uint32_t*>(w.piece + 128 * n + 8 * gi + 4 * (q & 1u));
        c.sc = *reinterpret_cast<const uint16_t*>(w.piece + 192 * n + 2 * gi);
        c.d = *reinterpret_cast<const uint16_t*>(w.piece + 208 * n + 2 * (gi >> 3));
    }
    return c;
}

// A wave's codes for one batch of kBatch groups, as loaded.
//   Q4_0: lane (c, q) loads group b kBatch + q of its row whole (16 bytes;
//   the row's four groups are 64 contiguous bytes) and the four groups'
//   scales (8 bytes, when the row's first group is a multiple of 4, else one
//   load a group); a 4 x 4 transpose across the lane quarters (two
//   v_permlane32_swap, two v_permlane16_swap) then gives lane (c, q) code
//   dword q of each of the four groups — what group_product takes. One 16-byte
//   and one 8-byte load a row block a batch instead of eight narrow ones.
//   Q6_K, Q8_0, Q4_1: group by group, as load_codes reads them.
template <uint32_t F, int R>
struct Batch {
    Codes<F> c[kBatch][R];
    __device__ __forceinline__ void load(const RowAt (&rows)[R], uint32_t b, uint32_t G, uint32_t q, bool) {
#pragma unroll
        for (int j = 0; j < kBatch; ++j)
#pragma unroll
            for (int r = 0; r < R; ++r) c[j][r] = load_codes<F>(rows[r], min(b * kBatch + j, G - 1), q);
    }
    __device__ __forceinline__ void codes(Codes<F> (&wc)[kBatch][R]) const {
#pragma unroll
        for (int j = 0; j < kBatch; ++j)
#pragma unroll
            for (int r = 0; r < R; ++r) wc[j][r] = c[j][r];
    }
};

template <int R>
struct Batch<kQ4_0, R> {
    u32x4_t raw[R];
    uint32_t sc[R][2];
    __device__ __forceinline__ void load(const RowAt (&rows)[R], uint32_t b, uint32_t G, uint32_t q, bool aligned) {
        const uint32_t first = b * kBatch;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint64_t gi = rows[r].gi0 + min(first + q, G - 1);
            raw[r] = *reinterpret_cast<const u32x4_t*>(rows[r].piece + 16 * gi);
            const uint16_t* scales = reinterpret_cast<const uint16_t*>(rows[r].piece + 16 * rows[r].blocks);
            if (aligned) {
                const uint2 two = *reinterpret_cast<const uint2*>(scales + rows[r].gi0 + first);
                sc[r][0] = two.x;
                sc[r][1] = two.y;
            } else {
                const uint64_t g0 = rows[r].gi0;
                const uint32_t d0 = scales[g0 + min(first, G - 1)], d1 = scales[g0 + min(first + 1, G - 1)];
                const uint32_t d2 = scales[g0 + min(first + 2, G - 1)], d3 = scales[g0 + min(first + 3, G - 1)];
                sc[r][0] = d0 | (d1 << 16);
                sc[r][1] = d2 | (d3 << 16);
            }
        }
    }
    __device__ __forceinline__ void codes(Codes<kQ4_0> (&wc)[kBatch][R]) const {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            uint32_t v0 = raw[r][0], v1 = raw[r][1], v2 = raw[r][2], v3 = raw[r][3];
            const auto s02 = __builtin_amdgcn_permlane32_swap(v0, v2, false, false);
            const auto s13 = __builtin_amdgcn_permlane32_swap(v1, v3, false, false);
            v0 = s02[0], v2 = s02[1], v1 = s13[0], v3 = s13[1];
            const auto s01 = __builtin_amdgcn_permlane16_swap(v0, v1, false, false);
            const auto s23 = __builtin_amdgcn_permlane16_swap(v2, v3, false, false);
            wc[0][r].code = s01[0], wc[1][r].code = s01[1], wc[2][r].code = s23[0], wc[3][r].code = s23[1];
            wc[0][r].d = sc[r][0] & 0xFFFFu, wc[1][r].d = sc[r][0] >> 16;
            wc[2][r].d = sc[r][1] & 0xFFFFu, wc[3][r].d = sc[r][1] >> 16;
        }
    }
};

// One group's products for a wave: the codes of its R row blocks (decoded
// here to binary16) against the T token blocks' split input, each block's
// P = codes . hi + codes . lo scaled into its totals.
// A row block's products are issued hi parts first, then lo parts, then the
// scales: a block's lo multiply accumulates onto its hi result, and its scale
// waits for the lo, so the T blocks' independent multiplies sit between them.
template <uint32_t F, int R, int T>
__device__ __forceinline__ void group_product(float4_t (&tot)[R][T], const half8_t (&xh)[T], const half8_t (&xl)[T],
                                              const Codes<F> (&cw)[R], uint32_t q) {
    const float4_t z = {0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (F == kQ4_0 || F == kQ8_0 || F == kQ4_1) {
        // Codes of weights 4q .. 4q+3, then 16+4q .. 16+4q+3, as binary16.
        half8_t b[R];
        float s[R], m[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            uint32_t first, second;
            _Float16 bias;
            if constexpr (F == kQ8_0) {
                // int8 q with its sign bit flipped is q + 128: lifted to 1152 + q
                first = cw[r].c0 ^ 0x80808080u, second = cw[r].c1 ^ 0x80808080u, bias = 1152.0f16;
                s[r] = half_to_float(cw[r].d);
            } else if constexpr (F == kQ4_1) {
                first = cw[r].code & 0x0F0F0F0Fu, second = (cw[r].code >> 4) & 0x0F0F0F0Fu, bias = 1024.0f16;
                s[r] = half_to_float(cw[r].dm & 0xFFFFu);
                m[r] = half_to_float(cw[r].dm >> 16);
            } else {
                first = cw[r].code & 0x0F0F0F0Fu, second = (cw[r].code >> 4) & 0x0F0F0F0Fu, bias = 1032.0f16;
                s[r] = half_to_float(cw[r].d);
            }
            const half2_t b0 = lift_less(first, kLowPair, bias), b1 = lift_less(first, kHighPair, bias);
            const half2_t b2 = lift_less(second, kLowPair, bias), b3 = lift_less(second, kHighPair, bias);
            b[r] = half8_t{b0.x, b0.y, b1.x, b1.y, b2.x, b2.y, b3.x, b3.y};
        }
        if constexpr (F == kQ4_1) {
            // Each token's sum of the group's inputs, the same for every row.
            const half8_t ones = {1.0f16, 1.0f16, 1.0f16, 1.0f16, 1.0f16, 1.0f16, 1.0f16, 1.0f16};
            float4_t sum[T];
#pragma unroll
            for (int t = 0; t < T; ++t) sum[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh[t], ones, z, 0, 0, 0);
#pragma unroll
            for (int t = 0; t < T; ++t) sum[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl[t], ones, sum[t], 0, 0, 0);
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int t = 0; t < T; ++t)
#pragma unroll
                    for (int k = 0; k < 4; ++k) tot[r][t][k] = __builtin_fmaf(m[r], sum[t][k], tot[r][t][k]);
        }
        // every block's hi multiplies, then every lo, then the scales: each
        // scale waits behind R T independent multiplies, not T
        float4_t p[R][T];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int t = 0; t < T; ++t) p[r][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh[t], b[r], z, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int t = 0; t < T; ++t) p[r][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xl[t], b[r], p[r][t], 0, 0, 0);
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int t = 0; t < T; ++t)
#pragma unroll
                for (int k = 0; k < 4; ++k) tot[r][t][k] = __builtin_fmaf(s[r], p[r][t][k], tot[r][t][k]);
    } else {
        // Codes of weights 4q .. 4q+3 (half 0) and 16+4q .. 16+4q+3 (half
        // 1): low nibbles from lo, high pairs from hi.
        half4_t b0[R], b1[R];
        float s0[R], s1[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t up = q >> 1;
            const uint32_t h0 = (cw[r].hi >> (2 * up)) & 0x03030303u;
            const uint32_t h1 = (cw[r].hi >> (2 * (2 + up))) & 0x03030303u;
            const uint32_t c0 = (cw[r].lo & 0x0F0F0F0Fu) | (h0 << 4);
            const uint32_t c1 = ((cw[r].lo >> 4) & 0x0F0F0F0Fu) | (h1 << 4);
            const half2_t a0 = lift_less(c0, kLowPair, 1056.0f16), a1 = lift_less(c0, kHighPair, 1056.0f16);
            const half2_t a2 = lift_less(c1, kLowPair, 1056.0f16), a3 = lift_less(c1, kHighPair, 1056.0f16);
            b0[r] = half4_t{a0.x, a0.y, a1.x, a1.y};
            b1[r] = half4_t{a2.x, a2.y, a3.x, a3.y};
            const float d = half_to_float(cw[r].d);
            s0[r] = d * static_cast<float>(static_cast<int8_t>(cw[r].sc & 0xFFu));
            s1[r] = d * static_cast<float>(static_cast<int8_t>((cw[r].sc >> 8) & 0xFFu));
        }
        float4_t p0[R][T], p1[R][T];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const half4_t h0x = {xh[t][0], xh[t][1], xh[t][2], xh[t][3]};
                const half4_t h1x = {xh[t][4], xh[t][5], xh[t][6], xh[t][7]};
                p0[r][t] = __builtin_amdgcn_mfma_f32_16x16x16f16(h0x, b0[r], z, 0, 0, 0);
                p1[r][t] = __builtin_amdgcn_mfma_f32_16x16x16f16(h1x, b1[r], z, 0, 0, 0);
            }
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const half4_t l0x = {xl[t][0], xl[t][1], xl[t][2], xl[t][3]};
                const half4_t l1x = {xl[t][4], xl[t][5], xl[t][6], xl[t][7]};
                p0[r][t] = __builtin_amdgcn_mfma_f32_16x16x16f16(l0x, b0[r], p0[r][t], 0, 0, 0);
                p1[r][t] = __builtin_amdgcn_mfma_f32_16x16x16f16(l1x, b1[r], p1[r][t], 0, 0, 0);
            }
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int t = 0; t < T; ++t)
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    tot[r][t][k] = __builtin_fmaf(s0[r], p0[r][t][k], tot[r][t][k]);
                    tot[r][t][k] = __builtin_fmaf(s1[r], p1[r][t][k], tot[r][t][k]);
                }
    }
}

// A workgroup's four waves share its T x 16 tokens and take R x 16 rows
// each, and walk K a batch of kBatch groups at a time. The tokens' split
// input goes through LDS, two batch buffers: while a batch is multiplied out
// of one, the next batch's input is copied into the other by the LDS DMA
// (all 256 lanes, 16 bytes a chunk, nothing held in registers — measured
// against copying through registers: C4 +2-4%, C5 +7.5%, and 100 fewer
// registers a lane). Each wave's codes for the next batch are loaded into
// registers alongside. So every load has a whole batch of products to
// arrive in, and a workgroup meets at one barrier a batch. 16-byte chunk k of token t sits at a swizzled chunk
// (below), spreading the 16 tokens a read takes over the banks. (Codes two
// batches ahead, or the A operand read a group ahead, measured no better.)
constexpr uint32_t kMfmaWavesASimd = 2;

// The chunk a token's 16-byte chunk k sits at. With 64 banks (256 bytes a
// bank row), tokens t and t ^ 1 share a row, and t and t + 8 would collide
// under k ^ (t & 7); k ^ ((t >> 1) & 7) spreads the 16 tokens of a read over
// all 16 chunk positions of a bank row.
__device__ __forceinline__ uint32_t swizzle(uint32_t t, uint32_t k) { return k ^ ((t >> 1) & 7u); }

template <uint32_t F, int R, int T, bool FULL>
__global__ __launch_bounds__(256, 2) void gemm_mfma(Product a, const uint8_t* __restrict__ xp,
                                                   const float* __restrict__ inv, uint32_t token_tiles,
                                                   uint32_t padded_tokens) {
    constexpr int BM = T * 16;
    constexpr int XC = BM * 8 / 256;  // 16-byte chunks a lane stages a group
    __shared__ u32x4_t xs[2][kBatch][BM * 8];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t q = lane >> 4, c = lane & 15u;
    const uint32_t tile_t = blockIdx.x % token_tiles, tile_r = blockIdx.x / token_tiles;
    const uint32_t tok0 = tile_t * BM, row0 = (tile_r * 4 + wave) * R * 16;
    const uint32_t G = a.groups;
    const uint32_t batches = (G + kBatch - 1) / kBatch;

    RowAt rows[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t p = min(row0 + 16 * r + c, a.rows - 1);
        const Piece w = piece_of(a, p);
        rows[r] = {w.piece, w.blocks, static_cast<uint64_t>(w.row) * G};
    }
    // Staging: the tile's input for a batch goes straight from the workspace
    // into LDS (global_load_lds: nothing lands in registers), LDS chunk j =
    // threadIdx.x + 256 i of a group holding token j / 8's chunk
    // swizzle(j / 8, j % 8) — the swizzle is its own inverse, so chunk k of
    // token t sits at t * 8 + swizzle(t, k), as the reads expect.
    const uint8_t* xbase = xp + static_cast<uint64_t>(tok0) * 128;
    const uint64_t group_bytes = static_cast<uint64_t>(padded_tokens) * 128;
    uint32_t from[XC];
#pragma unroll
    for (int i = 0; i < XC; ++i) {
        const uint32_t j = threadIdx.x + 256 * i, t = j >> 3;
        from[i] = 16 * (t * 8 + swizzle(t, j & 7u));
    }
    const bool aligned = (G & 3u) == 0;
    // A batch's input copies into LDS buffer `buf`: groups past the last
    // copy the last (unused). Each wave instruction writes 1 KB of LDS, its
    // lane L at 16 L from the wave's base.
    auto copy_x = [&](uint32_t b, uint32_t buf) {
        const uint32_t wave_base = 64 * wave;
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            const uint8_t* g = xbase + min(b * kBatch + j, G - 1) * group_bytes;
#pragma unroll
            for (int i = 0; i < XC; ++i) dma16(g + from[i], &xs[buf][j][256 * i + wave_base]);
        }
    };

    float4_t tot[R][T];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int t = 0; t < T; ++t) tot[r][t] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};

    // Batch b: its input in LDS buffer b & 1 (copied during batch b - 1), its
    // codes in `wcur`; the next batch's copies and code loads are issued
    // before its products, so they have the whole batch to land.
    Batch<F, R> w0, w1;
    auto batch = [&](uint32_t b, const Batch<F, R>& wcur, Batch<F, R>& wahead) {
        // This wave's copies for batch b (and its code loads) have landed;
        // after the barrier every wave's have, and every wave is done reading
        // buffer (b + 1) & 1 (batch b - 1).
        __builtin_amdgcn_s_waitcnt(kVmcnt0);
        __builtin_amdgcn_s_barrier();
        __asm__ __volatile__("" ::: "memory");
        const bool more = b + 1 < batches;
        if (more) copy_x(b + 1, (b + 1) & 1u);
        if (more) wahead.load(rows, b + 1, G, q, aligned);
        Codes<F> wc[kBatch][R];
        wcur.codes(wc);
        const u32x4_t* buf = xs[b & 1u][0];
        // A operands of group j of the batch, two buffers in turn.
        half8_t ah[2][T], al[2][T];
        auto read = [&](int j, half8_t (&xh)[T], half8_t (&xl)[T]) {
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const uint32_t tok = 16 * t + c;
                xh[t] = __builtin_bit_cast(half8_t, buf[j * BM * 8 + tok * 8 + swizzle(tok, 2 * q)]);
                xl[t] = __builtin_bit_cast(half8_t, buf[j * BM * 8 + tok * 8 + swizzle(tok, 2 * q + 1)]);
            }
        };
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            read(j, ah[j & 1], al[j & 1]);
            if (b * kBatch + j < G) group_product<F, R, T>(tot, ah[j & 1], al[j & 1], wc[j], q);
        }
    };
    copy_x(0, 0);
    w0.load(rows, 0, G, q, aligned);
    for (uint32_t b = 0; b < batches; b += 2) {
        batch(b, w0, w1);
        if (b + 1 < batches) batch(b + 1, w1, w0);
    }

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
static void go(const Product& a, const Plan& plan, const uint8_t* xp, const float* inv, hipStream_t stream) {
    const uint32_t m = static_cast<uint32_t>(mfma_padded_tokens(a.tokens));
    const dim3 grid(plan.token_tiles * plan.row_tiles);
    if (plain_epilogue(a))
        hipLaunchKernelGGL((gemm_mfma<F, R, T, false>), grid, dim3(256), 0, stream, a, xp, inv, plan.token_tiles, m);
    else
        hipLaunchKernelGGL((gemm_mfma<F, R, T, true>), grid, dim3(256), 0, stream, a, xp, inv, plan.token_tiles, m);
}

template <uint32_t F>
static hipError_t launch_format(const Product& a, const Plan& plan, const uint8_t* xp, const float* inv,
                                hipStream_t stream) {
    if constexpr (F == kQ4_0) {
        if (plan.wave_rows == 4 && plan.wave_tokens == 4) return go<F, 4, 4>(a, plan, xp, inv, stream), hipSuccess;
    }
    if (plan.wave_rows == 2 && plan.wave_tokens == 4) return go<F, 2, 4>(a, plan, xp, inv, stream), hipSuccess;
    if (plan.wave_rows == 2 && plan.wave_tokens == 2) return go<F, 2, 2>(a, plan, xp, inv, stream), hipSuccess;
    return hipErrorInvalidValue;
}

bool mfma_reads(uint32_t format) {
    return format == kQ4_0 || format == kQ4_1 || format == kQ8_0 || format == kQ6_K;
}

// The widest wave tile (16-row blocks x 16-token blocks) that still gives
// every SIMD two waves, else the smallest. Q6_K's 4 x 4 tile would not fit
// two waves' registers.
void plan_gemm_mfma(const Product& a, uint32_t format, uint32_t compute_units, Plan* plan) {
    *plan = Plan{};
    const auto waves = [&](int r, int t) {
        return uint64_t{(a.tokens + 16u * t - 1) / (16u * t)} * ((a.rows + 16u * r - 1) / (16u * r));
    };
    const uint64_t want = uint64_t{compute_units} * 4 * kMfmaWavesASimd;
    int r = 2, t = 2;
    if (format == kQ4_0 && waves(4, 4) >= want)
        r = 4, t = 4;
    else if (waves(2, 4) >= want)
        r = 2, t = 4;
    plan->kernel = kGemmMfma;
    plan->launches = 2;  // prepare_x, then the product
    plan->canonical = false;
    plan->wave_rows = r;
    plan->wave_tokens = t;
    plan->tile_tokens = 16 * t;
    plan->tile_rows = 64 * r;
    plan->token_tiles = (a.tokens + 16 * t - 1) / (16 * t);
    plan->row_tiles = (a.rows + 64 * r - 1) / (64 * r);
    plan->tiles = static_cast<uint64_t>(plan->token_tiles) * plan->row_tiles;
    plan->workgroups = plan->tiles;
}

hipError_t launch_gemm_mfma(const Product& a, uint32_t format, const Plan& plan, void* workspace,
                            hipStream_t stream) {
    const uint64_t m = mfma_padded_tokens(a.tokens);
    uint8_t* xp = static_cast<uint8_t*>(workspace);
    float* inv = reinterpret_cast<float*>(xp + m * a.groups * 128);
    hipLaunchKernelGGL(prepare_x, dim3(static_cast<uint32_t>(m)), dim3(256), 0, stream, a, xp, inv);
    hipError_t e;
    switch (format) {
        case kQ4_0: e = launch_format<kQ4_0>(a, plan, xp, inv, stream); break;
        case kQ4_1: e = launch_format<kQ4_1>(a, plan, xp, inv, stream); break;
        case kQ8_0: e = launch_format<kQ8_0>(a, plan, xp, inv, stream); break;
        case kQ6_K: e = launch_format<kQ6_K>(a, plan, xp, inv, stream); break;
        default: return hipErrorInvalidValue;
    }
    if (e != hipSuccess) return e;
    return hipGetLastError();
}

}  // namespace chm
