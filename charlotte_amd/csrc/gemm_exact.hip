// Prefill on the matrix cores in the canonical order: bit-exact.
//
// gemm_exact — v_mfma_f32_32x32x1_2b_f32 (K = 1, two 32 x 32 blocks) rounds
// each element once, as a fused multiply-add: d = c + a b is fmaf(a, b, c)
// bit for bit (checked on the GPU by harness.hip's mfma_fma_check over
// random, cancelling, halfway, denormal, overflowing, infinite and NaN
// operands). So a range's chain s = fma(w_k, x_k, s), in k order from +0
// (matmul.wgsl:121-126, 224-230), runs as a chain of these instructions, one
// k at a time, for 2,048 outputs at once; a range's sums then add into the
// totals in order on the VALU (matmul.wgsl:134-137), as gemm_canonical adds
// them. Every output is gemm_canonical's bits, and decode's.
//
// A wave takes 64 rows x TT tokens. At each k lane l supplies row R + l's
// weight as the A operand (lanes 0-31 block 0's rows, 32-63 block 1's).
// TT = 64: lane l supplies token T + l's input as B (lanes 0-31 block 0's
// columns, 32-63 block 1's), and two instructions a k, each broadcasting one
// block's A to both blocks (CBSZ 1, ABID 0 and 1), give rows R .. R + 31 and
// R + 32 .. R + 63 against tokens T .. T + 63. TT = 32 (for steps too small
// to give every SIMD two waves of 64 x 64): lanes l and l + 32 both supply
// token T + l % 32, and one instruction a k gives rows R .. R + 63 against
// tokens T .. T + 31. Each lane decodes its row's group (32 exact f32 weights) and
// loads its token's 32 inputs into registers, a group ahead; nothing goes
// through LDS and the waves of a workgroup never wait for one another. The
// VALU's share — a group's decode, a range's adds — is small beside the 64
// matrix instructions a group, and runs while they do.
//
// Result layout of one instruction (register v of 32, lane l): block v / 16,
// in it column l % 32 and row 8 ((v % 16) / 4) + 4 (l / 32) + v % 4 — rows
// p, p + 1 (p even) in one lane, so a gated product's gate and up totals
// (rows 2r, 2r + 1) meet there.
#include "decode.hpp"
#include "plan.hpp"
#include "product.hpp"
#include "stream.hpp"

namespace chm {

namespace {

typedef float f32x32 __attribute__((ext_vector_type(32)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr uint32_t kWaveRows = 64;   // rows a wave
constexpr uint32_t kWaves = 4;       // waves a workgroup, each its own 64 rows

// Four weights from four code bytes as the decodes' chain4 makes them: two
// codes a v_perm_b32 as binary16 1024 + b, then one v_fma_mix_f32 a weight,
// fma(1024 + b, scale, offset) — one rounding of a value f32 holds exactly.
__device__ __forceinline__ void weights4(uint32_t codes, float scale, float offset, float* w) {
    const half2_t a = lift(codes, kLowPair), b = lift(codes, kHighPair);
    w[0] = __builtin_fmaf(static_cast<float>(a.x), scale, offset);
    w[1] = __builtin_fmaf(static_cast<float>(a.y), scale, offset);
    w[2] = __builtin_fmaf(static_cast<float>(b.x), scale, offset);
    w[3] = __builtin_fmaf(static_cast<float>(b.y), scale, offset);
}

// The 32 exact weights of a group as loaded: the values of formats.hpp's
// weight(), which the VALU tile stages. Q4_0, Q8_0 and Q6_K by the lift of
// decode.hpp's chain_q4_0, chain_q8_0 and chain_q6_k (1.75 instructions a
// weight against weight()'s 3: C4 105 -> 111 TFLOP/s), the others by weight().
template <uint32_t F>
__device__ __forceinline__ void weights_of(const Raw<F>& r, float* w) {
    if constexpr (F == kQ4_0) {
        // (1024 + q) d - 1032 d; high nibbles as bytes 16 q: (1024 + 16 q) (d / 16) - 72 d
        const float d = half_to_float(r.d);
        const float low_offset = -1032.0f * d, d16 = d * 0.0625f, high_offset = -72.0f * d;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            weights4(r.w[c] & 0x0F0F0F0Fu, d, low_offset, w + 4 * c);
            weights4(r.w[c] & 0xF0F0F0F0u, d16, high_offset, w + 16 + 4 * c);
        }
    } else if constexpr (F == kQ4_1) {
        const Q4_1Group g = group_of(Q4_1Bytes{make_uint4(r.w[0], r.w[1], r.w[2], r.w[3]), r.dm});
#pragma unroll
        for (int l = 0; l < 32; ++l) w[l] = weight(g, l);
    } else if constexpr (F == kQ8_0) {
        // q + 128 (the sign bit flipped) lifted: fma(1152 + q, d, -1152 d) = q d
        const float d = half_to_float(r.d), offset = -1152.0f * d;
#pragma unroll
        for (int c = 0; c < 8; ++c) weights4(r.w[c] ^ 0x80808080u, d, offset, w + 4 * c);
    } else if constexpr (F == kQ6_K) {
        // the 6-bit codes assembled as chain_q6_k assembles them, then
        // fma(1024 + q, scale, -1056 scale) = (q - 32) scale
        const float d = half_to_float(r.d);
        const float first = d * static_cast<float>(static_cast<int8_t>(r.sc & 0xFFu));
        const float second = d * static_cast<float>(static_cast<int8_t>((r.sc >> 8) & 0xFFu));
        const float first_offset = -1056.0f * first, second_offset = -1056.0f * second;
        const uint32_t a0 = r.hi[0] & 0x33333333u, a1 = r.hi[1] & 0x33333333u;
        const uint32_t b0 = (r.hi[0] >> 2) & 0x33333333u, b1 = (r.hi[1] >> 2) & 0x33333333u;
        constexpr uint32_t kNib = 0x0F0F0F0Fu;
        weights4(bitfield_insert(kNib, r.lo[0], a0 << 4), first, first_offset, w + 0);
        weights4(bitfield_insert(kNib, r.lo[1], a1 << 4), first, first_offset, w + 4);
        weights4(bitfield_insert(kNib, r.lo[2], b0 << 4), first, first_offset, w + 8);
        weights4(bitfield_insert(kNib, r.lo[3], b1 << 4), first, first_offset, w + 12);
        weights4(bitfield_insert(kNib, r.lo[0] >> 4, a0), second, second_offset, w + 16);
        weights4(bitfield_insert(kNib, r.lo[1] >> 4, a1), second, second_offset, w + 20);
        weights4(bitfield_insert(kNib, r.lo[2] >> 4, b0), second, second_offset, w + 24);
        weights4(bitfield_insert(kNib, r.lo[3] >> 4, b1), second, second_offset, w + 28);
    } else if constexpr (F == kF32) {
#pragma unroll
        for (int l = 0; l < 32; ++l) w[l] = __uint_as_float(r.w[l]);
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            w[2 * i] = F == kF16 ? half_to_float(r.w[i] & 0xFFFFu) : bf16_low(r.w[i]);
            w[2 * i + 1] = F == kF16 ? half_to_float(r.w[i] >> 16) : bf16_high(r.w[i]);
        }
    }
}

// SPLIT (the split along K, matmul.wgsl:592-695): `chunks` workgroups a tile,
// chunk c taking ranges [32c / chunks, 32(c + 1) / chunks) and writing each
// range's sum to range_sums ([32][tokens][rows], range first) instead of
// adding it to a total; combine_ranges (gemm.hip) then adds a row's sums in
// order. The range sums are the VALU split's bits, so the outputs are too.
// `quads`: rows a multiple of 4 and range_sums 16-byte aligned, so a lane's
// four registers of consecutive rows go out as one 16-byte store (C6's split
// 20.9 -> 18.3 us against a store a register).
template <uint32_t F, uint32_t TT, bool FULL, bool CLIP, bool SPLIT = false>
__global__ __launch_bounds__(256, 2) void gemm_exact(Product a, uint32_t token_tiles, uint32_t row_tiles,
                                                     uint32_t chunks, float* range_sums, bool quads) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t tile_t = blockIdx.x % token_tiles, tile_r = (blockIdx.x / token_tiles) % row_tiles;
    const uint32_t chunk = blockIdx.x / (token_tiles * row_tiles);
    const uint32_t T = tile_t * TT, R = (tile_r * kWaves + wave) * kWaveRows;
    if (R >= a.rows) return;  // the whole wave: no barrier follows
    const uint32_t G = a.groups;
    const uint64_t K = static_cast<uint64_t>(G) * 32;
    const uint32_t r_begin = 32 * chunk / chunks, r_end = 32 * (chunk + 1) / chunks;
    const uint32_t g_begin = range_lo(r_begin, G), g_end = range_lo(r_end, G);
    if (g_begin >= g_end) return;  // a chunk of empty ranges (G < 32): nothing to write

    // Rows and tokens past the product read its last row or token; their
    // outputs are never stored.
    const Piece pc = piece_of(a, min(R + lane, a.rows - 1));
    const uint64_t row0 = static_cast<uint64_t>(pc.row) * G;
    const uint32_t my_token = T + (TT == 64 ? lane : lane & 31u);
    const float4* xrow = reinterpret_cast<const float4*>(a.x + static_cast<uint64_t>(min(my_token, a.tokens - 1)) * K);
    float lo = 0.0f, hi = 0.0f;
    if constexpr (CLIP) lo = *a.clip[0], hi = *a.clip[1];

    // Range sums (TT = 64: rows R .. R + 31 and R + 32 .. R + 63 against 64
    // tokens; TT = 32: s0 alone, rows R .. R + 63 against 32) and totals.
    constexpr int S = TT == 64 ? 2 : 1;
    f32x32 s0 = {}, s1 = {};
    float t[S][32];
#pragma unroll
    for (int v = 0; v < 32; ++v)
#pragma unroll
        for (int i = 0; i < S; ++i) t[i][v] = 0.0f;

    // The range that ends after group g is the one before `next_r`'s first
    // group; ranges with no groups (G < 32) hold zero and add nothing.
    uint32_t next_r = r_begin + 1;
    while (next_r < r_end && range_lo(next_r, G) <= g_begin) ++next_r;

    // A group's bytes and inputs are loaded a whole group ahead, into one of
    // two buffers (the loop takes groups in pairs, so each buffer keeps its
    // registers): at the top of group g every load of group g has been
    // waited for, and the loads of group g + 1 go out before its products,
    // so no wait inside them depends on a load issued in the same group.
    struct Buffer {
        Raw<F> raw;
        float4 xq[8];
    };
    auto fetch = [&](Buffer& b, uint32_t g) {
        b.raw.load(pc.piece, pc.blocks, row0 + g);
#pragma unroll
        for (int v = 0; v < 8; ++v) b.xq[v] = xrow[8 * g + v];
    };
    bool fresh = true;  // the next product starts a range: its chain from +0
    auto group = [&](const Buffer& b, uint32_t g) {
        float w[32], x[32];
        weights_of(b.raw, w);
#pragma unroll
        for (int v = 0; v < 8; ++v) {
            float4 q = b.xq[v];
            if constexpr (CLIP) {
                q.x = clamp_to(q.x, lo, hi);
                q.y = clamp_to(q.y, lo, hi);
                q.z = clamp_to(q.z, lo, hi);
                q.w = clamp_to(q.w, lo, hi);
            }
            x[4 * v] = q.x;
            x[4 * v + 1] = q.y;
            x[4 * v + 2] = q.z;
            x[4 * v + 3] = q.w;
        }
        // A range's first product takes +0 as its accumulator, so the chain
        // starts from +0 as fma(w, x, +0) does (the sums are never cleared).
        if (fresh) {
            const f32x32 zero = {};
            if constexpr (TT == 64) {
                s0 = __builtin_amdgcn_mfma_f32_32x32x1f32(w[0], x[0], zero, 1, 0, 0);
                s1 = __builtin_amdgcn_mfma_f32_32x32x1f32(w[0], x[0], zero, 1, 1, 0);
            } else {
                s0 = __builtin_amdgcn_mfma_f32_32x32x1f32(w[0], x[0], zero, 0, 0, 0);
            }
        } else {
            if constexpr (TT == 64) {
                s0 = __builtin_amdgcn_mfma_f32_32x32x1f32(w[0], x[0], s0, 1, 0, 0);
                s1 = __builtin_amdgcn_mfma_f32_32x32x1f32(w[0], x[0], s1, 1, 1, 0);
            } else {
                s0 = __builtin_amdgcn_mfma_f32_32x32x1f32(w[0], x[0], s0, 0, 0, 0);
            }
        }
#pragma unroll
        for (int k = 1; k < 32; ++k) {
            if constexpr (TT == 64) {
                s0 = __builtin_amdgcn_mfma_f32_32x32x1f32(w[k], x[k], s0, 1, 0, 0);
                s1 = __builtin_amdgcn_mfma_f32_32x32x1f32(w[k], x[k], s1, 1, 1, 0);
            } else {
                s0 = __builtin_amdgcn_mfma_f32_32x32x1f32(w[k], x[k], s0, 0, 0, 0);
            }
        }
        fresh = g + 1 == range_lo(next_r, G);
        if (fresh) {  // range next_r - 1 ends
            if constexpr (SPLIT) {
#pragma unroll
                for (int v = 0; v < 32; v += 4) {
                    const uint32_t in_block = 8 * ((v & 15) / 4) + 4 * (lane >> 5);  // rows in_block .. + 3
                    uint32_t token, p;
                    if constexpr (TT == 64) {
                        token = T + 32 * (v / 16) + (lane & 31u), p = R + in_block;
                    } else {
                        token = T + (lane & 31u), p = R + 32 * (v / 16) + in_block;
                    }
                    if (token >= a.tokens) continue;
                    float* at = range_sums + (static_cast<uint64_t>(next_r - 1) * a.tokens + token) * a.rows + p;
                    float q0[4] = {s0[v], s0[v + 1], s0[v + 2], s0[v + 3]};
                    if (quads) {
                        if (p < a.rows) *reinterpret_cast<float4*>(at) = make_float4(q0[0], q0[1], q0[2], q0[3]);
                    } else {
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            if (p + i < a.rows) at[i] = q0[i];
                    }
                    if constexpr (S == 2) {
                        float q1[4] = {s1[v], s1[v + 1], s1[v + 2], s1[v + 3]};
                        if (quads) {
                            if (p + 32 < a.rows)
                                *reinterpret_cast<float4*>(at + 32) = make_float4(q1[0], q1[1], q1[2], q1[3]);
                        } else {
#pragma unroll
                            for (int i = 0; i < 4; ++i)
                                if (p + 32 + i < a.rows) at[32 + i] = q1[i];
                        }
                    }
                }
            } else {
#pragma unroll
                for (int v = 0; v < 32; ++v) {
                    const float a0 = s0[v];
                    t[0][v] = t[0][v] + a0;
                    if constexpr (S == 2) {
                        const float a1 = s1[v];
                        t[S - 1][v] = t[S - 1][v] + a1;
                    }
                }
            }
            while (next_r < r_end && range_lo(next_r, G) <= g + 1) ++next_r;
        }
    };

    // Every fetch is issued on every path (past the last group it reads the
    // last group again, unused), so the count of loads in flight at each wait
    // is the same on every path: a wait for one buffer never waits for the
    // other's loads.
    Buffer A, B;
    fetch(A, g_begin);
    for (uint32_t g = g_begin; g < g_end; g += 2) {
        fetch(B, min(g + 1, g_end - 1));
        group(A, g);
        if (g + 1 >= g_end) break;
        fetch(A, min(g + 2, g_end - 1));
        group(B, g + 1);
    }
    if constexpr (SPLIT) return;

#pragma unroll
    for (int v = 0; v < 32; ++v) {
        const uint32_t in_block = 8 * ((v & 15) / 4) + 4 * (lane >> 5) + (v & 3);
        if constexpr (TT == 64) {
            const uint32_t token = T + 32 * (v / 16) + (lane & 31u), p = R + in_block;
            if (token < a.tokens) {
                if (p < a.rows) emit<FULL>(a, p, token, token, t[0][v], (v & 1) ? 0.0f : t[0][v ^ 1]);
                if (p + 32 < a.rows) emit<FULL>(a, p + 32, token, token, t[S - 1][v], (v & 1) ? 0.0f : t[S - 1][v ^ 1]);
            }
        } else {
            const uint32_t token = T + (lane & 31u), p = R + 32 * (v / 16) + in_block;
            if (token < a.tokens && p < a.rows) emit<FULL>(a, p, token, token, t[0][v], (v & 1) ? 0.0f : t[0][v ^ 1]);
        }
    }
}


// gemm_exact_short — a short step on the matrix cores: the canonical order
// with K split among a workgroup's waves, as gemm_short splits it on the
// VALU. A step of few tokens gives gemm_exact few waves, each walking all of
// K as one chain of dependent matrix instructions (C6's 2,048 x 8,192 at 32
// tokens: 32 waves); here a workgroup takes 32 rows x 32 tokens and its
// eight waves four of the 32 ranges each, as two pairs. A pair's two chains
// run in one v_mfma_f32_32x32x1_2b_f32 (K = 1, two 32 x 32 blocks, one fused
// multiply-add an element): block b is range r_begin + 2 p + b, its A (row R
// + l % 32) and B (token T + l % 32) from lanes 32 b .. 32 b + 31, each lane
// decoding its own range's group, and register v holds block v / 16's row 8
// ((v % 16) / 4) + 4 (l / 32) + v % 4, column l % 32. Step j of a pair is
// group j of both ranges; where one range is a group shorter than the other
// (the two differ by at most one), its block's lanes take -0 and +0 at the
// pair's last step: fma(-0, +0, acc) is acc for every acc (acc + -0 = acc).
//
// A step's inputs (two groups x 32 tokens x 128 bytes) reach the wave's LDS
// stage by eight copies (global_load_lds, 1 KB each: 8 tokens' whole lines of
// one group), where loading them into registers took eight loads a group
// touching 32 lines each; token t's 16-byte chunk c lies at position c ^ (t %
// 8) of its 128 bytes, so a read of one chunk for 32 tokens spreads over the
// banks. Two stages a wave: a step's loads are waited for (the compiler's
// wait, which covers its copies, issued before them) before the next step's
// go out, in flight under this step's chain. The pairs' sums stay in
// registers through K; then, after a barrier, the stages' LDS holds the range
// sums ([range][register][lane]: 128 KB, one workgroup a CU), and after a
// second each thread adds two registers' 32 range sums in order from zero,
// skipping empty ones (G < 32) — rows p, p + 1 of one token, so a gated pair's
// totals meet in the thread: gemm_canonical's order, its bits.
constexpr uint32_t kShortWaves = 8;  // waves a workgroup, two pairs of ranges each
constexpr uint32_t kShortTile = 32;  // rows, and tokens, a workgroup

template <uint32_t F, bool FULL, bool CLIP>
__global__ __launch_bounds__(64 * kShortWaves, 1) void gemm_exact_short(Product a, uint32_t token_tiles) {
    __shared__ float4 lds[32 * 16 * 64 / 4];  // the stages (16 KB a wave), then the range sums (128 KB)
    static_assert(kShortWaves * 2 * 512 == 32 * 16 * 64 / 4, "two stages of 8 KB a wave fill the range sums' LDS");
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6, half = lane >> 5;
    const uint32_t T = (blockIdx.x % token_tiles) * kShortTile, R = (blockIdx.x / token_tiles) * kShortTile;
    const uint32_t G = a.groups;
    const uint64_t K = static_cast<uint64_t>(G) * 32;
    const uint32_t r_begin = 4 * wave;
    // pair p's steps: its longer range's groups
    const uint32_t l0 = range_lo(r_begin, G), l1 = range_lo(r_begin + 1, G), l2 = range_lo(r_begin + 2, G),
                   l3 = range_lo(r_begin + 3, G), l4 = range_lo(r_begin + 4, G);
    const uint32_t n0 = max(l1 - l0, l2 - l1), steps = n0 + max(l3 - l2, l4 - l3);
    f32x32 held0 = {}, held1 = {};  // pair 0's sums, pair 1's

    if (steps) {
        // Rows and tokens past the product read its last row or token; their
        // outputs are never stored.
        const Piece pc = piece_of(a, min(R + (lane & 31u), a.rows - 1));
        const uint64_t row0 = static_cast<uint64_t>(pc.row) * G;
        // copy i of a group: token 8 i + lane / 8, its chunk (lane % 8) ^ (token % 8)
        const float4* src[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t tok = 8 * i + (lane >> 3);
            src[i] = reinterpret_cast<const float4*>(a.x + static_cast<uint64_t>(min(T + tok, a.tokens - 1)) * K) +
                     ((lane & 7u) ^ (tok & 7u));
        }
        const uint32_t my_tok = lane & 31u;
        float4* const stages = lds + wave * 1024;  // two stages of 2 x 256 chunks, [block][token][chunk]
        const uint32_t read_at =
            static_cast<uint32_t>(reinterpret_cast<uintptr_t>(stages)) + 4096 * half + 128 * my_tok;
        float lo = 0.0f, hi = 0.0f;
        if constexpr (CLIP) lo = *a.clip[0], hi = *a.clip[1];
        // Step t's group for block b, clamped into the product; `live` false
        // past the end of the block's range.
        auto group_of = [&](uint32_t t, uint32_t b, bool& live) {
            const bool second = t >= n0;
            const uint32_t j = second ? t - n0 : t;
            const uint32_t first = second ? (b ? l3 : l2) : (b ? l1 : l0), end = second ? (b ? l4 : l3) : (b ? l2 : l1);
            live = first + j < end;
            return min(first + j, G - 1);
        };
        // A step's copies go out before its weights' loads (and nothing may
        // move between them), so the wait for its weights covers its copies.
        auto fetch = [&](Raw<F>& raw, uint32_t stage, uint32_t t) {
            bool live;
            const uint32_t g0 = group_of(t, 0, live), g1 = group_of(t, 1, live);
#pragma unroll
            for (int i = 0; i < 4; ++i)
                __builtin_amdgcn_global_load_lds(src[i] + 8 * g0, (lds_void)(stages + 512 * stage + 64 * i), 16, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i)
                __builtin_amdgcn_global_load_lds(src[i] + 8 * g1, (lds_void)(stages + 512 * stage + 256 + 64 * i), 16,
                                                 0, 0);
            __asm__ __volatile__("" ::: "memory");
            raw.load(pc.piece, pc.blocks, row0 + (half ? g1 : g0));
        };
        f32x32 s = {};  // +0 at each pair's start: its first products are fma(w, x, +0)
        auto step = [&](const Raw<F>& raw, uint32_t stage, uint32_t t, auto&& next) {
            float w[32], x[32];
            weights_of(raw, w);
            // the stage's reads, after the weights (whose loads were waited
            // for): the last weight is an input the reads do not use
            u32x4s_t q[8];
            const uint32_t at = read_at + 8192 * stage;
            const uint32_t sw = my_tok & 7u;
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const uint32_t addr = at + 16 * (c ^ sw);
                __asm__ __volatile__("ds_read_b128 %0, %1" : "=v"(q[c]) : "v"(addr), "v"(w[31]));
            }
            __asm__ __volatile__("s_waitcnt lgkmcnt(0)"
                                 : "+v"(q[0]), "+v"(q[1]), "+v"(q[2]), "+v"(q[3]), "+v"(q[4]), "+v"(q[5]),
                                   "+v"(q[6]), "+v"(q[7]));
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                float4 v = make_float4(__uint_as_float(q[c][0]), __uint_as_float(q[c][1]),
                                       __uint_as_float(q[c][2]), __uint_as_float(q[c][3]));
                if constexpr (CLIP) {
                    v.x = clamp_to(v.x, lo, hi);
                    v.y = clamp_to(v.y, lo, hi);
                    v.z = clamp_to(v.z, lo, hi);
                    v.w = clamp_to(v.w, lo, hi);
                }
                x[4 * c] = v.x;
                x[4 * c + 1] = v.y;
                x[4 * c + 2] = v.z;
                x[4 * c + 3] = v.w;
            }
            bool live0, live1;
            group_of(t, 0, live0);
            group_of(t, 1, live1);
            if (!(half ? live1 : live0)) {  // past this block's range: products of -0 and +0
#pragma unroll
                for (int k = 0; k < 32; ++k) w[k] = -0.0f, x[k] = 0.0f;
            }
            next();  // the next step's loads, in flight under this chain
#pragma unroll
            for (int k = 0; k < 32; ++k) s = __builtin_amdgcn_mfma_f32_32x32x1f32(w[k], x[k], s, 0, 0, 0);
            if (t + 1 == n0) {  // pair 0 ends
                held0 = s;
                s = f32x32{};
            }
        };
        Raw<F> A, B;
        fetch(A, 0, 0);
        for (uint32_t t = 0; t < steps; t += 2) {
            step(A, 0, t, [&] {
                if (t + 1 < steps) fetch(B, 1, t + 1);
            });
            if (t + 1 >= steps) break;
            step(B, 1, t + 1, [&] {
                if (t + 2 < steps) fetch(A, 0, t + 2);
            });
        }
        held1 = s;
    }
    // Every copy has landed (each wave waited for its last step's weights,
    // loaded after its copies, and loads nothing past it) and every stage
    // read: the LDS takes the range sums, [range][register][lane].
    __syncthreads();
    float* const sums = reinterpret_cast<float*>(lds);
#pragma unroll
    for (int v = 0; v < 32; ++v) {
        const uint32_t r = r_begin + (v / 16);
        sums[r * 1024 + 64 * (v % 16) + lane] = held0[v];
        sums[(r + 2) * 1024 + 64 * (v % 16) + lane] = held1[v];
    }
    __syncthreads();

    // The ordered combine: registers 2 wave and 2 wave + 1 of a block, for `lane`.
    const uint32_t v0 = 2 * wave;
    float ta = 0.0f, tb = 0.0f;
#pragma unroll
    for (uint32_t r = 0; r < 32; ++r) {
        if (range_lo(r, G) < range_lo(r + 1, G)) {
            ta = ta + sums[r * 1024 + 64 * v0 + lane];
            tb = tb + sums[r * 1024 + 64 * (v0 + 1) + lane];
        }
    }
    const uint32_t token = T + (lane & 31u);
    const uint32_t p = R + 8 * (v0 / 4) + 4 * (lane >> 5) + (v0 & 3);
    if (token < a.tokens) {
        if (p < a.rows) emit<FULL>(a, p, token, token, ta, tb);
        if (p + 1 < a.rows) emit<FULL>(a, p + 1, token, token, tb, 0.0f);
    }
}

// gemm_exact_quad — the short-step tile for a step whose 32 x 32 tiles would
// leave compute units idle (C6's 2,048 x 8,192 at 32 tokens: 64 of them):
// 16 rows x 16 tokens a workgroup, four times the workgroups, at twice the
// decode a product (each instruction does half the products). Each of its
// eight waves takes four of the 32 ranges as the four blocks of one
// v_mfma_f32_16x16x1_4b_f32 (K = 1, one fused multiply-add an element): block
// b is range r_begin + b, its A (row R + l % 16) and B (token T + l % 16) from
// lanes 16 b .. 16 b + 15, each lane decoding its own range's group; register
// v holds block v / 4's row 4 (l / 16) + v % 4, column l % 16. Step j is group
// j of the four ranges; a range a group shorter than the wave's longest takes
// -0 and +0 at the last step (fma(-0, +0, acc) = acc for every acc). A
// step's inputs, four groups x 16 tokens x 128 bytes, reach the wave's LDS
// stage by eight whole-line copies as gemm_exact_short's do, two stages a
// wave; the accumulator ends as the wave's four range sums, which a barrier
// later the LDS holds ([range][register][lane]), and 128 threads add a
// token's rows p, p + 1 over the 32 ranges in order from zero: the bits of
// every other canonical tile.
constexpr uint32_t kQuadTile = 16;  // rows, and tokens, a workgroup

template <uint32_t F, bool FULL, bool CLIP>
__global__ __launch_bounds__(64 * kShortWaves, 1) void gemm_exact_quad(Product a, uint32_t token_tiles) {
    __shared__ float4 lds[kShortWaves * 2 * 512];  // the stages (16 KB a wave), then the range sums (32 KB)
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6, blk = lane >> 4, my_i = lane & 15u;
    const uint32_t T = (blockIdx.x % token_tiles) * kQuadTile, R = (blockIdx.x / token_tiles) * kQuadTile;
    const uint32_t G = a.groups;
    const uint64_t K = static_cast<uint64_t>(G) * 32;
    const uint32_t r_begin = 4 * wave;
    uint32_t lo_r[5];
#pragma unroll
    for (int b = 0; b < 5; ++b) lo_r[b] = range_lo(r_begin + b, G);
    uint32_t steps = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) steps = max(steps, lo_r[b + 1] - lo_r[b]);
    // this lane's range: its first group and its end
    const uint32_t my_first = blk == 0 ? lo_r[0] : blk == 1 ? lo_r[1] : blk == 2 ? lo_r[2] : lo_r[3];
    const uint32_t my_end = blk == 0 ? lo_r[1] : blk == 1 ? lo_r[2] : blk == 2 ? lo_r[3] : lo_r[4];
    f32x16 s = {};  // +0: each range's first product is fma(w, x, +0)

    if (steps) {
        // Rows and tokens past the product read its last row or token; their
        // outputs are never stored.
        const Piece pc = piece_of(a, min(R + my_i, a.rows - 1));
        const uint64_t row0 = static_cast<uint64_t>(pc.row) * G;
        // copy (b, h): block b's tokens 8 h + lane / 8, chunk (lane % 8) ^ (token % 8)
        const float4* src[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t tok = 8 * h + (lane >> 3);
            src[h] = reinterpret_cast<const float4*>(a.x + static_cast<uint64_t>(min(T + tok, a.tokens - 1)) * K) +
                     ((lane & 7u) ^ (tok & 7u));
        }
        float4* const stages = lds + wave * 1024;  // two stages of 4 x 128 chunks, [block][token][chunk]
        const uint32_t read_at =
            static_cast<uint32_t>(reinterpret_cast<uintptr_t>(stages)) + 2048 * blk + 128 * my_i;
        float lo = 0.0f, hi = 0.0f;
        if constexpr (CLIP) lo = *a.clip[0], hi = *a.clip[1];
        // A step's copies go out before its weights' loads (and nothing may
        // move between them), so the wait for its weights covers its copies.
        auto fetch = [&](Raw<F>& raw, uint32_t stage, uint32_t j) {
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const uint32_t g = min(lo_r[b] + j, G - 1);
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    __builtin_amdgcn_global_load_lds(src[h] + 8 * g, (lds_void)(stages + 512 * stage + 128 * b + 64 * h),
                                                     16, 0, 0);
            }
            __asm__ __volatile__("" ::: "memory");
            raw.load(pc.piece, pc.blocks, row0 + min(my_first + j, G - 1));
        };
        auto step = [&](const Raw<F>& raw, uint32_t stage, uint32_t j, auto&& next) {
            float w[32], x[32];
            weights_of(raw, w);
            // the stage's reads, after the weights (whose loads were waited
            // for): the last weight is an input the reads do not use
            u32x4s_t q[8];
            const uint32_t at = read_at + 8192 * stage;
            const uint32_t sw = my_i & 7u;
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const uint32_t addr = at + 16 * (c ^ sw);
                __asm__ __volatile__("ds_read_b128 %0, %1" : "=v"(q[c]) : "v"(addr), "v"(w[31]));
            }
            __asm__ __volatile__("s_waitcnt lgkmcnt(0)"
                                 : "+v"(q[0]), "+v"(q[1]), "+v"(q[2]), "+v"(q[3]), "+v"(q[4]), "+v"(q[5]),
                                   "+v"(q[6]), "+v"(q[7]));
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                float4 v = make_float4(__uint_as_float(q[c][0]), __uint_as_float(q[c][1]),
                                       __uint_as_float(q[c][2]), __uint_as_float(q[c][3]));
                if constexpr (CLIP) {
                    v.x = clamp_to(v.x, lo, hi);
                    v.y = clamp_to(v.y, lo, hi);
                    v.z = clamp_to(v.z, lo, hi);
                    v.w = clamp_to(v.w, lo, hi);
                }
                x[4 * c] = v.x;
                x[4 * c + 1] = v.y;
                x[4 * c + 2] = v.z;
                x[4 * c + 3] = v.w;
            }
            if (my_first + j >= my_end) {  // past this block's range: products of -0 and +0
#pragma unroll
                for (int k = 0; k < 32; ++k) w[k] = -0.0f, x[k] = 0.0f;
            }
            next();  // the next step's loads, in flight under this chain
#pragma unroll
            for (int k = 0; k < 32; ++k) s = __builtin_amdgcn_mfma_f32_16x16x1f32(w[k], x[k], s, 0, 0, 0);
        };
        Raw<F> A, B;
        fetch(A, 0, 0);
        for (uint32_t j = 0; j < steps; j += 2) {
            step(A, 0, j, [&] {
                if (j + 1 < steps) fetch(B, 1, j + 1);
            });
            if (j + 1 >= steps) break;
            step(B, 1, j + 1, [&] {
                if (j + 2 < steps) fetch(A, 0, j + 2);
            });
        }
    }
    // Every copy has landed (each wave waited for its last step's weights,
    // loaded after its copies, and loads nothing past it) and every stage
    // read: the LDS takes the range sums, [range][register][lane].
    __syncthreads();
    float* const sums = reinterpret_cast<float*>(lds);
#pragma unroll
    for (int v = 0; v < 16; ++v) sums[(r_begin + v / 4) * 256 + 64 * (v % 4) + lane] = s[v];
    __syncthreads();

    // The ordered combine: registers 2 h and 2 h + 1 of a block, for lane `l`.
    if (threadIdx.x < 128) {
        const uint32_t l = threadIdx.x & 63u, h = threadIdx.x >> 6;
        float ta = 0.0f, tb = 0.0f;
#pragma unroll
        for (uint32_t r = 0; r < 32; ++r) {
            if (range_lo(r, G) < range_lo(r + 1, G)) {
                ta = ta + sums[r * 256 + 64 * (2 * h) + l];
                tb = tb + sums[r * 256 + 64 * (2 * h + 1) + l];
            }
        }
        const uint32_t token = T + (l & 15u);
        const uint32_t p = R + 4 * (l >> 4) + 2 * h;
        if (token < a.tokens) {
            if (p < a.rows) emit<FULL>(a, p, token, token, ta, tb);
            if (p + 1 < a.rows) emit<FULL>(a, p + 1, token, token, tb, 0.0f);
        }
    }
}

template <uint32_t F>
void go_exact_short(const Product& a, const Plan& plan, hipStream_t stream) {
    const dim3 grid(static_cast<uint32_t>(plan.workgroups)), block(64 * kShortWaves);
    const uint32_t tt = plan.token_tiles;
    if (plan.tile_rows == kQuadTile) {
        if (plain_epilogue(a))
            hipLaunchKernelGGL((gemm_exact_quad<F, false, false>), grid, block, 0, stream, a, tt);
        else if (!clipped(a))
            hipLaunchKernelGGL((gemm_exact_quad<F, true, false>), grid, block, 0, stream, a, tt);
        else
            hipLaunchKernelGGL((gemm_exact_quad<F, true, true>), grid, block, 0, stream, a, tt);
        return;
    }
    if (plain_epilogue(a))
        hipLaunchKernelGGL((gemm_exact_short<F, false, false>), grid, block, 0, stream, a, tt);
    else if (!clipped(a))
        hipLaunchKernelGGL((gemm_exact_short<F, true, false>), grid, block, 0, stream, a, tt);
    else
        hipLaunchKernelGGL((gemm_exact_short<F, true, true>), grid, block, 0, stream, a, tt);
}

template <uint32_t F, uint32_t TT>
void go_exact_tile(const Product& a, const Plan& plan, float* range_sums, hipStream_t stream) {
    const dim3 grid(static_cast<uint32_t>(plan.workgroups)), block(64 * kWaves);
    const uint32_t tt = plan.token_tiles, rt = plan.row_tiles, ch = plan.chunks;
    if (range_sums) {  // a split product has no options and is not gated
        const bool quads = a.rows % 4 == 0 && reinterpret_cast<uintptr_t>(range_sums) % 16 == 0;
        hipLaunchKernelGGL((gemm_exact<F, TT, false, false, true>), grid, block, 0, stream, a, tt, rt, ch, range_sums,
                           quads);
    } else if (plain_epilogue(a)) {
        hipLaunchKernelGGL((gemm_exact<F, TT, false, false>), grid, block, 0, stream, a, tt, rt, 1u, nullptr, false);
    } else if (!clipped(a)) {
        hipLaunchKernelGGL((gemm_exact<F, TT, true, false>), grid, block, 0, stream, a, tt, rt, 1u, nullptr, false);
    } else {
        hipLaunchKernelGGL((gemm_exact<F, TT, true, true>), grid, block, 0, stream, a, tt, rt, 1u, nullptr, false);
    }
}

template <uint32_t F>
void go_exact(const Product& a, const Plan& plan, float* range_sums, hipStream_t stream) {
    if constexpr (F != kF32) {
        if (plan.tile_tokens == 64) return go_exact_tile<F, 64>(a, plan, range_sums, stream);
    }
    go_exact_tile<F, 32>(a, plan, range_sums, stream);
}

}  // namespace

// Tiles of 256 rows (four waves of 64) by 64 or 32 tokens, token tile first,
// so the tiles reading one row tile's weights run together. A wave's time is
// its walk through K, and a SIMD's waves share its matrix core, so a step
// takes as many rounds as its most loaded SIMD holds waves: 64 x 64 waves
// where they give no more rounds than 64 x 32 waves give half-length ones
// (one wave of 64 x 64 a SIMD, two chains of products, measured faster than
// two of 64 x 32, one chain each: C4 98.6 against 93.4 TFLOP/s), else 64 x
// 32 — Llama 3.2 1B's QKV at 2,048 tokens: 1,536 waves of 64 x 64 on 1,024
// SIMDs are two rounds, 3,072 of 64 x 32 one and a half. F32 always by 32 (its
// 32 dwords a group beside 64 tokens' sums would not fit two waves' registers).
void plan_gemm_exact(const Product& a, uint32_t format, uint32_t compute_units, bool split, Plan* plan) {
    *plan = Plan{};
    const uint64_t wave_rows = (a.rows + kWaveRows - 1) / kWaveRows;
    const uint64_t simds = 4ull * compute_units;
    const uint64_t rounds64 = (wave_rows * ((a.tokens + 63) / 64) + simds - 1) / simds;
    const uint64_t rounds32 = (wave_rows * ((a.tokens + 31) / 32) + simds - 1) / simds;  // half-length rounds
    uint32_t tt = format != kF32 && rounds32 >= 2 * rounds64 ? 64 : 32;
    if (split) tt = format != kF32 && a.tokens > 32 ? 64 : 32;
    plan->kernel = split ? kGemmExactSplit : kGemmExact;
    plan->launches = split ? 2 : 1;
    plan->tile_tokens = tt;
    plan->tile_rows = kWaves * kWaveRows;
    plan->token_tiles = (a.tokens + tt - 1) / tt;
    plan->row_tiles = (a.rows + plan->tile_rows - 1) / plan->tile_rows;
    plan->wave_rows = kWaveRows / 32;
    plan->wave_tokens = tt / 32;
    plan->tiles = static_cast<uint64_t>(plan->token_tiles) * plan->row_tiles;
    // Split: the ranges cut into as few chunks (a power of two, at most 32)
    // as still give every compute unit two workgroups where 32 can.
    uint32_t chunks = 1;
    if (split) {
        chunks = 2;
        while (chunks < 32 && plan->tiles * chunks < 2ull * compute_units) chunks *= 2;
    }
    plan->chunks = chunks;
    plan->workgroups = plan->tiles * chunks;
}

// The short-step form: workgroups of 32 rows x 32 tokens, token tile first.
void plan_gemm_exact_short(const Product& a, uint32_t compute_units, Plan* plan) {
    *plan = Plan{};
    plan->kernel = kGemmExactShort;
    plan->launches = 1;
    // 16 x 16 tiles (gemm_exact_quad) where they number at most two a
    // compute unit, else 32 x 32 (gemm_exact_short), a quarter as many:
    // measured on 256 compute units, 2,048 x 2,048 x 32 tokens (256 of 16 x
    // 16) 7.5 against 17.2 us, 4,096 x 2,048 x 32 (512) 13.6 against 17.8,
    // 6,144 x 2,048 x 32 (768) 19.8 against 18.0
    const uint64_t quads = uint64_t{(a.tokens + kQuadTile - 1) / kQuadTile} * ((a.rows + kQuadTile - 1) / kQuadTile);
    const uint32_t tile = quads <= 2ull * compute_units ? kQuadTile : kShortTile;
    plan->tile_tokens = tile;
    plan->tile_rows = tile;
    plan->token_tiles = (a.tokens + tile - 1) / tile;
    plan->row_tiles = (a.rows + tile - 1) / tile;
    plan->wave_rows = 1;
    plan->wave_tokens = 1;
    plan->tiles = static_cast<uint64_t>(plan->token_tiles) * plan->row_tiles;
    plan->workgroups = plan->tiles;
}

hipError_t launch_gemm_exact_short(const Product& a, uint32_t format, const Plan& plan, hipStream_t stream) {
    switch (format) {
        case kQ4_0: go_exact_short<kQ4_0>(a, plan, stream); break;
        case kQ4_1: go_exact_short<kQ4_1>(a, plan, stream); break;
        case kQ8_0: go_exact_short<kQ8_0>(a, plan, stream); break;
        case kQ6_K: go_exact_short<kQ6_K>(a, plan, stream); break;
        case kF32: go_exact_short<kF32>(a, plan, stream); break;
        case kF16: go_exact_short<kF16>(a, plan, stream); break;
        case kBF16: go_exact_short<kBF16>(a, plan, stream); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// The tile; with `range_sums` (the split plan: room for 32 x tokens x rows
// floats), the split form and then combine_ranges.
hipError_t launch_gemm_exact(const Product& a, uint32_t format, const Plan& plan, float* range_sums,
                             hipStream_t stream) {
    switch (format) {
        case kQ4_0: go_exact<kQ4_0>(a, plan, range_sums, stream); break;
        case kQ4_1: go_exact<kQ4_1>(a, plan, range_sums, stream); break;
        case kQ8_0: go_exact<kQ8_0>(a, plan, range_sums, stream); break;
        case kQ6_K: go_exact<kQ6_K>(a, plan, range_sums, stream); break;
        case kF32: go_exact<kF32>(a, plan, range_sums, stream); break;
        case kF16: go_exact<kF16>(a, plan, range_sums, stream); break;
        case kBF16: go_exact<kBF16>(a, plan, range_sums, stream); break;
        default: return hipErrorInvalidValue;
    }
    if (range_sums) return launch_combine_ranges(a, range_sums, stream);
    return hipGetLastError();
}

}  // namespace chm
