// Fast exact decode of one 32-weight group into the canonical fma chain.
//
// formats.hpp's weight() is one weight at a time; here a group's bytes are
// taken a dword — four codes — at a time:
//   - the four codes are assembled into the four bytes of a dword (Q4_0: a
//     mask; Q6_K: a bitfield insert of the low nibbles into the high pairs);
//   - v_perm_b32 lifts two code bytes into the low bytes of two binary16
//     values whose high byte is 0x64, i.e. 1024 + q, exactly;
//   - v_fma_mix_f32 takes one binary16 half as an f32 operand, so
//     w = fma(1024 + q, scale, -(1024 + bias) * scale) is the weight, exactly:
//     (1024 + q) * scale has at most 11 + 18 bits and the fma rounds once, and
//     the constant and the result are exact (q - bias is at most 6 bits, the
//     scale at most 18);
//   - the chain s = fma(w_l, x_l, s) runs in k order, as formats.hpp's.
// About 2.9 VALU operations a Q4_0 weight and 3.4 a Q6_K weight, against
// formats.hpp's 5 to 6. The bits are the same: each w is the exact weight
// (Q4_1's, q d + m, rounded once as the reference's).
#pragma once

#include "formats.hpp"

namespace chm {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

constexpr uint32_t kHalf1024 = 0x64646464u;    // 0x64 in every byte: binary16 1024 + q's high byte
constexpr uint32_t kLowPair = 0x04010400u;     // bytes 0, 1 of a dword -> halves (1024 + b0, 1024 + b1)
constexpr uint32_t kHighPair = 0x04030402u;    // bytes 2, 3 -> halves (1024 + b2, 1024 + b3)

__device__ __forceinline__ half2_t lift(uint32_t codes, uint32_t selector) {
    return __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(kHalf1024, codes, selector));
}

// Two code bytes as binary16 codes less their bias: (1024 + q) - (1024 +
// bias) = q - bias, exact (the matrix-core prefill's operands).
__device__ __forceinline__ half2_t lift_less(uint32_t codes, uint32_t selector, _Float16 bias) {
    const half2_t v = lift(codes, selector);
    const half2_t b = {bias, bias};
    return v - b;
}

// Four weights from four code bytes, continuing the chain over x[0..3].
__device__ __forceinline__ float chain4(uint32_t codes, float scale, float offset, const float* x, float s) {
    const half2_t a = lift(codes, kLowPair), b = lift(codes, kHighPair);
    s = __builtin_fmaf(__builtin_fmaf(static_cast<float>(a.x), scale, offset), x[0], s);
    s = __builtin_fmaf(__builtin_fmaf(static_cast<float>(a.y), scale, offset), x[1], s);
    s = __builtin_fmaf(__builtin_fmaf(static_cast<float>(b.x), scale, offset), x[2], s);
    s = __builtin_fmaf(__builtin_fmaf(static_cast<float>(b.y), scale, offset), x[3], s);
    return s;
}

// (a & mask) | (b & ~mask) in one v_bfi_b32: written out, the compiler emits
// an and and an and-or (Q6_K's unpack: a C2 step's VALU instructions a lane
// 1,111 -> 1,040; C2 49.9-51.3 -> 49.3-49.7 us).
__device__ __forceinline__ uint32_t bitfield_insert(uint32_t mask, uint32_t a, uint32_t b) {
    uint32_t r;
    __asm__("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "s"(mask), "v"(a), "v"(b));
    return r;
}

// A Q4_0 group: 4 code dwords, its fp16 scale bits.
__device__ __forceinline__ float chain_q4_0(const uint32_t w[4], uint32_t d_bits, const float* x, float s) {
    const float d = half_to_float(d_bits);
    // low nibbles: (1024 + q) d - 1032 d; high nibbles as bytes 16q:
    // (1024 + 16q) (d / 16) - 72 d. d / 16 is exact (f32 has the range).
    const float low_offset = -1032.0f * d, d16 = d * 0.0625f, high_offset = -72.0f * d;
#pragma unroll
    for (int c = 0; c < 4; ++c) s = chain4(w[c] & 0x0F0F0F0Fu, d, low_offset, x + 4 * c, s);
#pragma unroll
    for (int c = 0; c < 4; ++c) s = chain4(w[c] & 0xF0F0F0F0u, d16, high_offset, x + 16 + 4 * c, s);
    return s;
}

// (a & mask) | bits in one v_and_or_b32 (with both constants literals the
// compiler emits an and and an or).
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t mask, uint32_t bits) {
    uint32_t r;
    __asm__("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(mask), "v"(bits));
    return r;
}

// chain_q4_0's bits in fewer operations, for the throughput-bound streamed
// decode (the latency-bound ones keep chain_q4_0, whose first product starts
// sooner). A code dword's 8 nibbles become four binary16 pairs in 5
// operations instead of 6: with 0x54 for the high byte a half is 64 + m / 16
// for its low byte m, so
//   - (w & 0x000F000F) | 0x54005400: 64 + l0 / 16, 64 + l2 / 16;
//   - (w & 0x00F000F0) | 0x54005400: 64 + h0, 64 + h2;
//   - p = bytes 1 and 3 under 0x54 (one v_perm_b32), then p & 0xFF0FFF0F:
//     64 + l1 / 16, 64 + l3 / 16; p & 0xFFF0FFF0: 64 + h1, 64 + h3;
// all exact (binary16 steps by 1/16 in [64, 128)). The weights:
// (64 + l / 16) 16d - 1032 d = (l - 8) d and (64 + h) d - 72 d = (h - 8) d,
// each one fma of exact terms whose result is exact (16d, 1032d and 72d are
// exact in f32: d has 11 significant bits).
__device__ __forceinline__ float chain_q4_0_wide(const uint32_t w[4], uint32_t d_bits, const float* x, float s) {
    const float d = half_to_float(d_bits);
    const float d16 = 16.0f * d, low_offset = -1032.0f * d, high_offset = -72.0f * d;
    uint32_t a[4], b[4], c[4], e[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t p = __builtin_amdgcn_perm(0x54545454u, w[k], 0x04030401u);  // 0x54:b1, 0x54:b3
        a[k] = and_or(w[k], 0x000F000Fu, 0x54005400u);
        b[k] = p & 0xFF0FFF0Fu;
        c[k] = and_or(w[k], 0x00F000F0u, 0x54005400u);
        e[k] = p & 0xFFF0FFF0u;
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const half2_t u = __builtin_bit_cast(half2_t, a[k]), v = __builtin_bit_cast(half2_t, b[k]);
        s = __builtin_fmaf(__builtin_fmaf(static_cast<float>(u.x), d16, low_offset), x[4 * k], s);
        s = __builtin_fmaf(__builtin_fmaf(static_cast<float>(v.x), d16, low_offset), x[4 * k + 1], s);
        s = __builtin_fmaf(__builtin_fmaf(static_cast<float>(u.y), d16, low_offset), x[4 * k + 2], s);
        s = __builtin_fmaf(__builtin_fmaf(static_cast<float>(v.y), d16, low_offset), x[4 * k + 3], s);
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const half2_t u = __builtin_bit_cast(half2_t, c[k]), v = __builtin_bit_cast(half2_t, e[k]);
        s = __builtin_fmaf(__builtin_fmaf(static_cast<float>(u.x), d, high_offset), x[16 + 4 * k], s);
        s = __builtin_fmaf(__builtin_fmaf(static_cast<float>(v.x), d, high_offset), x[16 + 4 * k + 1], s);
        s = __builtin_fmaf(__builtin_fmaf(static_cast<float>(u.y), d, high_offset), x[16 + 4 * k + 2], s);
        s = __builtin_fmaf(__builtin_fmaf(static_cast<float>(v.y), d, high_offset), x[16 + 4 * k + 3], s);
    }
    return s;
}

// A Q6_K group: 4 lo dwords, 2 hi dwords, its two int8 scales (low 16 bits
// of sc), its super-block's fp16 d bits.
__device__ __forceinline__ float chain_q6_k(const uint32_t lo[4], const uint32_t hi[2], uint32_t sc, uint32_t d_bits,
                                            const float* x, float s) {
    const float d = half_to_float(d_bits);
    const float first = d * static_cast<float>(static_cast<int8_t>(sc & 0xFFu));
    const float second = d * static_cast<float>(static_cast<int8_t>((sc >> 8) & 0xFFu));
    const float first_offset = -1056.0f * first, second_offset = -1056.0f * second;
    // hi byte m: pairs of weights m, m + 8, m + 16, m + 24 at bits 0, 2, 4, 6.
    // a: pairs at bits 0 and 4 of each byte; b: the others, moved there.
    const uint32_t a0 = hi[0] & 0x33333333u, a1 = hi[1] & 0x33333333u;
    const uint32_t b0 = (hi[0] >> 2) & 0x33333333u, b1 = (hi[1] >> 2) & 0x33333333u;
    constexpr uint32_t kNib = 0x0F0F0F0Fu;
    // weights 0..15: low nibbles of lo, pairs at bits 0 (l < 8) or 2 (l >= 8), moved to bits 4-5
    s = chain4(bitfield_insert(kNib, lo[0], a0 << 4), first, first_offset, x + 0, s);
    s = chain4(bitfield_insert(kNib, lo[1], a1 << 4), first, first_offset, x + 4, s);
    s = chain4(bitfield_insert(kNib, lo[2], b0 << 4), first, first_offset, x + 8, s);
    s = chain4(bitfield_insert(kNib, lo[3], b1 << 4), first, first_offset, x + 12, s);
    // weights 16..31: high nibbles of lo, pairs at bits 4 (l < 24) or 6 (l >= 24), at bits 4-5
    s = chain4(bitfield_insert(kNib, lo[0] >> 4, a0), second, second_offset, x + 16, s);
    s = chain4(bitfield_insert(kNib, lo[1] >> 4, a1), second, second_offset, x + 20, s);
    s = chain4(bitfield_insert(kNib, lo[2] >> 4, b0), second, second_offset, x + 24, s);
    s = chain4(bitfield_insert(kNib, lo[3] >> 4, b1), second, second_offset, x + 28, s);
    return s;
}

// Four weights of unsigned byte codes: w = fma(code, scale, offset), the
// codes converted by v_cvt_f32_ubyte0..3, one instruction each.
__device__ __forceinline__ float chain4_bytes(uint32_t codes, float scale, float offset, const float* x, float s) {
    s = __builtin_fmaf(__builtin_fmaf(static_cast<float>(codes & 0xFFu), scale, offset), x[0], s);
    s = __builtin_fmaf(__builtin_fmaf(static_cast<float>((codes >> 8) & 0xFFu), scale, offset), x[1], s);
    s = __builtin_fmaf(__builtin_fmaf(static_cast<float>((codes >> 16) & 0xFFu), scale, offset), x[2], s);
    s = __builtin_fmaf(__builtin_fmaf(static_cast<float>(codes >> 24), scale, offset), x[3], s);
    return s;
}

// A Q4_1 group: 4 code dwords, its d (low 16 bits) and m (high) word.
// w = q d + m: low nibbles fma(q, d, m); high nibbles as bytes 16q,
// fma(16q, d / 16, m) — (16q)(d / 16) = q d exactly — so one rounding either
// way, the add's.
__device__ __forceinline__ float chain_q4_1(const uint32_t w[4], uint32_t dm, const float* x, float s) {
    const float d = half_to_float(dm & 0xFFFFu), m = half_to_float(dm >> 16);
    const float d16 = d * 0.0625f;
#pragma unroll
    for (int c = 0; c < 4; ++c) s = chain4_bytes(w[c] & 0x0F0F0F0Fu, d, m, x + 4 * c, s);
#pragma unroll
    for (int c = 0; c < 4; ++c) s = chain4_bytes(w[c] & 0xF0F0F0F0u, d16, m, x + 16 + 4 * c, s);
    return s;
}

// A Q8_0 group: 8 code dwords, its fp16 d bits. Each int8 code q biased to
// q + 128 (the sign bit flipped), lifted to 1024 + q + 128, and
// fma(1152 + q, d, -1152 d) = q d, exact (1152 d and q d are exact).
__device__ __forceinline__ float chain_q8_0(const uint32_t w[8], uint32_t d_bits, const float* x, float s) {
    const float d = half_to_float(d_bits);
    const float offset = -1152.0f * d;
#pragma unroll
    for (int c = 0; c < 8; ++c) s = chain4(w[c] ^ 0x80808080u, d, offset, x + 4 * c, s);
    return s;
}

// An F32 group: its 32 floats, the chain over them.
__device__ __forceinline__ float chain_f32(const uint32_t w[32], const float* x, float s) {
#pragma unroll
    for (int l = 0; l < 32; ++l) s = __builtin_fmaf(__uint_as_float(w[l]), x[l], s);
    return s;
}

// An F16 group: 16 dwords, two halves each, the lower first. Each half is
// converted exactly inside the multiply-add (v_fma_mix_f32 takes a binary16
// operand as its f32 value): one instruction a weight.
__device__ __forceinline__ float chain_f16(const uint32_t w[16], const float* x, float s) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const half2_t h = __builtin_bit_cast(half2_t, w[i]);
        s = __builtin_fmaf(static_cast<float>(h.x), x[2 * i], s);
        s = __builtin_fmaf(static_cast<float>(h.y), x[2 * i + 1], s);
    }
    return s;
}

// A BF16 group: 16 dwords, two values each, the lower first; a value is its
// 16 bits at the top of an f32 (a shift or a mask), exact.
__device__ __forceinline__ float chain_bf16(const uint32_t w[16], const float* x, float s) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        s = __builtin_fmaf(bf16_low(w[i]), x[2 * i], s);
        s = __builtin_fmaf(bf16_high(w[i]), x[2 * i + 1], s);
    }
    return s;
}

// A group's raw bytes as a kernel holds them between load and use.
template <uint32_t F>
struct Raw;

template <>
struct Raw<kF32> {
    uint32_t w[32];
    __device__ __forceinline__ void load(const uint8_t* piece, uint64_t, uint64_t gi) {
        const uint4* c = reinterpret_cast<const uint4*>(piece + 128 * gi);
#pragma unroll
        for (int v = 0; v < 8; ++v) {
            const uint4 q = c[v];
            w[4 * v] = q.x;
            w[4 * v + 1] = q.y;
            w[4 * v + 2] = q.z;
            w[4 * v + 3] = q.w;
        }
    }
    __device__ __forceinline__ float chain(const float* x, float s) const { return chain_f32(w, x, s); }
};

// F16 and BF16: 64 bytes a group.
template <uint32_t F>
struct RawHalves {
    uint32_t w[16];
    __device__ __forceinline__ void load(const uint8_t* piece, uint64_t, uint64_t gi) {
        const uint4* c = reinterpret_cast<const uint4*>(piece + 64 * gi);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const uint4 q = c[v];
            w[4 * v] = q.x;
            w[4 * v + 1] = q.y;
            w[4 * v + 2] = q.z;
            w[4 * v + 3] = q.w;
        }
    }
    __device__ __forceinline__ float chain(const float* x, float s) const {
        return F == kF16 ? chain_f16(w, x, s) : chain_bf16(w, x, s);
    }
};

template <>
struct Raw<kF16> : RawHalves<kF16> {};
template <>
struct Raw<kBF16> : RawHalves<kBF16> {};

// Dwords a group holds in registers between load and use.
template <uint32_t F>
constexpr int raw_dwords() {
    return F == kF32 ? 32 : F == kF16 || F == kBF16 ? 16 : F == kQ8_0 ? 9 : F == kQ6_K ? 8 : 5;
}

template <>
struct Raw<kQ4_0> {
    uint32_t w[4];
    uint32_t d;
    __device__ __forceinline__ void load(const uint8_t* piece, uint64_t n, uint64_t gi) {
        const uint4 c = *reinterpret_cast<const uint4*>(piece + 16 * gi);
        w[0] = c.x;
        w[1] = c.y;
        w[2] = c.z;
        w[3] = c.w;
        d = *reinterpret_cast<const uint16_t*>(piece + 16 * n + 2 * gi);
    }
    __device__ __forceinline__ float chain(const float* x, float s) const { return chain_q4_0(w, d, x, s); }
};

template <>
struct Raw<kQ4_1> {
    uint32_t w[4];
    uint32_t dm;
    __device__ __forceinline__ void load(const uint8_t* piece, uint64_t n, uint64_t gi) {
        const uint4 c = *reinterpret_cast<const uint4*>(piece + 16 * gi);
        w[0] = c.x;
        w[1] = c.y;
        w[2] = c.z;
        w[3] = c.w;
        dm = *reinterpret_cast<const uint32_t*>(piece + 16 * n + 4 * gi);
    }
    __device__ __forceinline__ float chain(const float* x, float s) const { return chain_q4_1(w, dm, x, s); }
};

template <>
struct Raw<kQ8_0> {
    uint32_t w[8];
    uint32_t d;
    __device__ __forceinline__ void load(const uint8_t* piece, uint64_t n, uint64_t gi) {
        const uint4* c = reinterpret_cast<const uint4*>(piece + 32 * gi);
        const uint4 a = c[0], b = c[1];
        w[0] = a.x;
        w[1] = a.y;
        w[2] = a.z;
        w[3] = a.w;
        w[4] = b.x;
        w[5] = b.y;
        w[6] = b.z;
        w[7] = b.w;
        d = *reinterpret_cast<const uint16_t*>(piece + 32 * n + 2 * gi);
    }
    __device__ __forceinline__ float chain(const float* x, float s) const { return chain_q8_0(w, d, x, s); }
};

template <>
struct Raw<kQ6_K> {
    uint32_t lo[4], hi[2], sc, d;
    __device__ __forceinline__ void load(const uint8_t* piece, uint64_t n, uint64_t gi) {
        const uint4 l = *reinterpret_cast<const uint4*>(piece + 16 * gi);
        const uint2 h = *reinterpret_cast<const uint2*>(piece + 128 * n + 8 * gi);
        lo[0] = l.x;
        lo[1] = l.y;
        lo[2] = l.z;
        lo[3] = l.w;
        hi[0] = h.x;
        hi[1] = h.y;
        sc = *reinterpret_cast<const uint16_t*>(piece + 192 * n + 2 * gi);
        d = *reinterpret_cast<const uint16_t*>(piece + 208 * n + 2 * (gi / 8));
    }
    __device__ __forceinline__ float chain(const float* x, float s) const { return chain_q6_k(lo, hi, sc, d, x, s); }
};

}  // namespace chm
