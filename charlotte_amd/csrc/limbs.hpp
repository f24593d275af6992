// The decode path that trades the canonical order for fewer instructions a
// weight (the GEMV path INT8_LIMBS): integer dot products on v_dot4_i32_i8,
// four weights an instruction, against the exact path's three f32-rate
// instructions a weight. No counterpart in the reference, whose one order is
// the canonical one (matmul.h:34-50); its results are within the tolerance
// max|err| / max|y| <= 1e-5 of that order, not its bits.
//
// x, a 32-weight group g at a time: with m the group's max |x| (after the
// clip) and e such that m < 2^e <= 2m, s = 22 - e, every x of the group is
// X = rint(x 2^s), |X| <= 2^22, so |x - X 2^-s| <= 2^(e-23) <= m 2^-22. X is
// cut into three signed bytes, X = 65536 a + 256 b + c (c and b the low
// bytes sign-extended, a in [-64, 64]), so a weight code q (0..63) times X is
// three byte products, summed exactly in int32 by v_dot4_i32_i8.
//
// A group record, 32 dwords in LDS (the order of a group's weights is the
// codes': dword c holds weights 4c .. 4c + 3, byte b weight 4c + b):
//   [0, 8)   the a bytes      [8, 16) the b bytes      [16, 24) the c bytes
//   [24, 27) -32 (sum of a, sum of b, sum of c) over weights 0..15
//   [27, 30) the same over weights 16..31
//   30       -s, an int
//   31       0.0f, or a NaN if the group holds a non-finite x (so every
//            total it enters is NaN)
// Each 16-weight half h (a Q6_K scale's span) sums, from the records' -32
// sums, A = sum (q - 32) a, B and C alike; |A| <= 16 * 32 * 64 = 2^15, so
// Z = 256 A + B is exact in int32 and in f32, and P_h = fma(Z, 256, C) =
// sum (q - 32) X rounded once. The group's contribution is
// d ldexp(fma(sc_1, P_1, sc_0 P_0), -s): the power of two applied to the
// group's sum, exact wherever that sum is a normal f32.
//
// Q4_0 (codes q in 0..15, weight (q - 8) d, one scale a group) stages its
// records with a bias of 8 over the whole group: [24, 27) hold -8 (sum of
// a, sum of b, sum of c) over weights 0..31 and [27, 30) zero. A = sum
// (q - 8) a has |A| <= 32 * 8 * 64 = 2^14, Z = 256 A + B is exact, P =
// fma(Z, 256, C) is sum (q - 8) X rounded once, and the contribution is
// d ldexp(P + poison, -s).
#pragma once

#include "decode.hpp"

namespace chm {

typedef uint32_t u32x4s_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2s_t __attribute__((ext_vector_type(2)));

constexpr uint32_t kLimbRecord = 32;  // dwords a group

// Lane `part` (0..3) of a group's four converts x[8 part .. 8 part + 7] (v0,
// v1) and writes its share of the record at LDS byte address `record`; the
// four lanes are a quad (the group's max and sums meet by DPP). Stores are
// inline ds_writes: the caller waits for them (lgkmcnt) before its barrier.
// kBias 32 (Q6_K): the sums over each 16-weight half; 8 (Q4_0): over the
// whole group.
template <int kBias = 32>
__device__ __forceinline__ void stage_limbs(float4 v0, float4 v1, uint32_t part, uint32_t record) {
    const float e[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    float m = 0.0f;
    int bad = 0;  // a NaN or an infinity among the lane's x (fmaxf would pass a NaN over)
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        m = fmaxf(m, fabsf(e[k]));
        bad |= __builtin_isfinite(e[k]) ? 0 : 1;
    }
    // quad_perm [1, 0, 3, 2] then [2, 3, 0, 1]: the quad's max and flag on every lane
    m = fmaxf(m, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, m), 0xB1, 0xF, 0xF, false)));
    m = fmaxf(m, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, m), 0x4E, 0xF, 0xF, false)));
    bad |= __builtin_amdgcn_mov_dpp(bad, 0xB1, 0xF, 0xF, false);
    bad |= __builtin_amdgcn_mov_dpp(bad, 0x4E, 0xF, 0xF, false);
    const bool finite = bad == 0;
    int exponent = 0;
    (void)frexpf(m, &exponent);  // m = f 2^exponent, f in [0.5, 1)
    const int shift = (m == 0.0f || !finite) ? 0 : 22 - exponent;
    uint32_t wa[2] = {0, 0}, wb[2] = {0, 0}, wc[2] = {0, 0};
    int sa = 0, sb = 0, sc = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int X = finite ? static_cast<int>(rintf(ldexpf(e[k], shift))) : 0;
        const int c = static_cast<int8_t>(X & 0xFF);
        const int r = (X - c) >> 8;
        const int b = static_cast<int8_t>(r & 0xFF);
        const int a = (r - b) >> 8;
        wa[k >> 2] |= (static_cast<uint32_t>(a) & 0xFFu) << (8 * (k & 3));
        wb[k >> 2] |= (static_cast<uint32_t>(b) & 0xFFu) << (8 * (k & 3));
        wc[k >> 2] |= (static_cast<uint32_t>(c) & 0xFFu) << (8 * (k & 3));
        sa += a, sb += b, sc += c;
    }
    // the half's sums: parts 0 and 1 (weights 0..15), 2 and 3 (16..31)
    sa += __builtin_amdgcn_mov_dpp(sa, 0xB1, 0xF, 0xF, false);
    sb += __builtin_amdgcn_mov_dpp(sb, 0xB1, 0xF, 0xF, false);
    sc += __builtin_amdgcn_mov_dpp(sc, 0xB1, 0xF, 0xF, false);
    if constexpr (kBias == 8) {
        // and the group's: the two halves' (quad_perm [2, 3, 0, 1])
        sa += __builtin_amdgcn_mov_dpp(sa, 0x4E, 0xF, 0xF, false);
        sb += __builtin_amdgcn_mov_dpp(sb, 0x4E, 0xF, 0xF, false);
        sc += __builtin_amdgcn_mov_dpp(sc, 0x4E, 0xF, 0xF, false);
    }
    __asm__ __volatile__("ds_write_b64 %0, %1" : : "v"(record + 8 * part), "v"(u32x2s_t{wa[0], wa[1]}));
    __asm__ __volatile__("ds_write_b64 %0, %1" : : "v"(record + 32 + 8 * part), "v"(u32x2s_t{wb[0], wb[1]}));
    __asm__ __volatile__("ds_write_b64 %0, %1" : : "v"(record + 64 + 8 * part), "v"(u32x2s_t{wc[0], wc[1]}));
    if (part == 0 || part == 2) {
        const uint32_t at = record + (part == 0 ? 96 : 108);
        const bool live = kBias == 32 || part == 0;
        __asm__ __volatile__("ds_write_b32 %0, %1" : : "v"(at), "v"(live ? static_cast<uint32_t>(-kBias * sa) : 0u));
        __asm__ __volatile__("ds_write_b32 %0, %1" : : "v"(at + 4), "v"(live ? static_cast<uint32_t>(-kBias * sb) : 0u));
        __asm__ __volatile__("ds_write_b32 %0, %1" : : "v"(at + 8), "v"(live ? static_cast<uint32_t>(-kBias * sc) : 0u));
    }
    if (part == 1) {
        const float poison = finite ? 0.0f : __builtin_nanf("");
        __asm__ __volatile__("ds_write_b64 %0, %1"
                             :
                             : "v"(record + 120), "v"(u32x2s_t{static_cast<uint32_t>(-shift), __float_as_uint(poison)}));
    }
}

// One Q6_K group against its record g (8 dwords x 4), added to the lane's
// sum: fma(d, ldexp(fma(sc_1, P_1, fma(sc_0, P_0, poison)), -s), sum). The
// codes are assembled as chain_q6_k's: low nibbles into bits 0-3, the high
// pairs into bits 4-5, so each byte is q in 0..63.
__device__ __forceinline__ float group_limbs_q6_k(const uint32_t lo[4], const uint32_t hi[2], uint32_t sc, float d,
                                                  const u32x4s_t g[8], float sum) {
    const uint32_t a0 = hi[0] & 0x33333333u, a1 = hi[1] & 0x33333333u;
    const uint32_t b0 = (hi[0] >> 2) & 0x33333333u, b1 = (hi[1] >> 2) & 0x33333333u;
    constexpr uint32_t kNib = 0x0F0F0F0Fu;
    const uint32_t code[8] = {
        bitfield_insert(kNib, lo[0], a0 << 4),      bitfield_insert(kNib, lo[1], a1 << 4),
        bitfield_insert(kNib, lo[2], b0 << 4),      bitfield_insert(kNib, lo[3], b1 << 4),
        bitfield_insert(kNib, lo[0] >> 4, a0),      bitfield_insert(kNib, lo[1] >> 4, a1),
        bitfield_insert(kNib, lo[2] >> 4, b0),      bitfield_insert(kNib, lo[3] >> 4, b1),
    };
    float part[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        int A = static_cast<int>(h == 0 ? g[6][0] : g[6][3]);
        int B = static_cast<int>(h == 0 ? g[6][1] : g[7][0]);
        int C = static_cast<int>(h == 0 ? g[6][2] : g[7][1]);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int q = static_cast<int>(code[4 * h + c]);
            const int v = 4 * h + c;  // dword v of each limb: g[v / 4][v % 4], g[2 + v / 4], g[4 + v / 4]
            A = __builtin_amdgcn_sdot4(q, static_cast<int>(g[v >> 2][v & 3]), A, false);
            B = __builtin_amdgcn_sdot4(q, static_cast<int>(g[2 + (v >> 2)][v & 3]), B, false);
            C = __builtin_amdgcn_sdot4(q, static_cast<int>(g[4 + (v >> 2)][v & 3]), C, false);
        }
        part[h] = __builtin_fmaf(static_cast<float>(A * 256 + B), 256.0f, static_cast<float>(C));
    }
    const float first = static_cast<float>(static_cast<int8_t>(sc & 0xFFu));
    const float second = static_cast<float>(static_cast<int8_t>((sc >> 8) & 0xFFu));
    const float t = __builtin_fmaf(second, part[1], __builtin_fmaf(first, part[0], __uint_as_float(g[7][3])));
    return __builtin_fmaf(d, __builtin_ldexpf(t, static_cast<int>(g[7][2])), sum);
}

// One Q4_0 group against its record g (staged with kBias 8), added to the
// lane's sum: fma(d, ldexp(P + poison, -s), sum). Byte b of code dword c
// holds weights 4c + b (low nibble) and 16 + 4c + b (high), so the low
// nibbles of dword c meet the record's dword c and the high ones dword 4 + c.
__device__ __forceinline__ float group_limbs_q4_0(const uint32_t w[4], float d, const u32x4s_t g[8], float sum) {
    constexpr uint32_t kNib = 0x0F0F0F0Fu;
    int A = static_cast<int>(g[6][0]), B = static_cast<int>(g[6][1]), C = static_cast<int>(g[6][2]);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int lo = static_cast<int>(w[c] & kNib), hi = static_cast<int>((w[c] >> 4) & kNib);
        A = __builtin_amdgcn_sdot4(lo, static_cast<int>(g[0][c]), A, false);
        B = __builtin_amdgcn_sdot4(lo, static_cast<int>(g[2][c]), B, false);
        C = __builtin_amdgcn_sdot4(lo, static_cast<int>(g[4][c]), C, false);
        A = __builtin_amdgcn_sdot4(hi, static_cast<int>(g[1][c]), A, false);
        B = __builtin_amdgcn_sdot4(hi, static_cast<int>(g[3][c]), B, false);
        C = __builtin_amdgcn_sdot4(hi, static_cast<int>(g[5][c]), C, false);
    }
    const float P = __builtin_fmaf(static_cast<float>(A * 256 + B), 256.0f, static_cast<float>(C));
    return __builtin_fmaf(d, __builtin_ldexpf(P + __uint_as_float(g[7][3]), static_cast<int>(g[7][2])), sum);
}

}  // namespace chm
