// The weight formats as the kernels read them from a piece's streams, and
// the one multiply-add order every canonical kernel shares.
//
// A piece of n blocks holds each stream whole, one after another
// (src/core/formats/device_layout.h:111-136):
//   Q4_0  codes   [0, 16n)      16 bytes a block: byte j = weight j (low nibble),
//                               weight j + 16 (high nibble)
//         scales  [16n, 18n)    fp16 d a block
//   Q6_K  lo      [0, 128n)     16 bytes a 32-weight group: byte j = weight j's low
//                               nibble (low half), weight j + 16's (high half)
//         hi      [128n, 192n)  8 bytes a group: byte m = the high bit pairs of
//                               weights m, m + 8, m + 16, m + 24 at bits 0, 2, 4, 6
//         scales  [192n, 208n)  int8, two a group: weights 0..15, then 16..31
//         d       [208n, 210n)  fp16 a super-block of 8 groups
//   Q4_1  codes   [0, 16n)      as Q4_0's
//         d, m    [16n, 20n)    fp16 d then fp16 m, one dword a block
//   Q8_0  codes   [0, 32n)      32 int8 a block, weight j at byte j
//         scales  [32n, 34n)    fp16 d a block
//   F32   floats  [0, 4n)       a "block" is one weight
//   F16   halves  [0, 2n)       a "block" is one binary16 weight
//   BF16  values  [0, 2n)       a "block" is one bfloat16 weight: an f32's top half
// F32, F16 and BF16 group gi is values 32gi .. 32gi + 31 (f32.wgsl, f16.wgsl,
// bf16.wgsl); each decodes to its exact f32 with no arithmetic to round.
// Groups are counted flat over the piece — group gi is row gi / G's group
// gi % G — so a Q6_K row need not be whole super-blocks (q6_k.wgsl:13-42).
//
// Every weight decodes exactly: (q - 8) d and (d sc)(q - 32) are products of
// at most 24 significant bits, so fma(q, d, -8d) and fma(q, d sc, -32 d sc)
// return them exactly, one instruction a weight after the code's conversion.
// Q8_0's q d is exact likewise. Q4_1's q d + m rounds once, at the add: q d
// (4 + 11 significant bits) is exact, so fma(q, d, m) is both of the
// reference's admissible answers, the multiply-add rounded twice and fused
// (q4_1_reference.h), which are always the same bits.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace chm {

enum Format : uint32_t { kF32 = 0, kF16 = 1, kQ4_0 = 2, kQ4_1 = 3, kQ8_0 = 8, kQ6_K = 14, kBF16 = 30 };

// Bytes a stored block, and weights a block (src/core/gguf/types.h:65-101).
constexpr uint32_t block_bytes(uint32_t f) {
    return f == kF32 ? 4u
           : f == kF16 || f == kBF16 ? 2u
           : f == kQ4_0 ? 18u
           : f == kQ4_1 ? 20u
           : f == kQ8_0 ? 34u
           : f == kQ6_K ? 210u
                        : 0u;
}
constexpr uint32_t block_weights(uint32_t f) {
    return f == kF32 || f == kF16 || f == kBF16 ? 1u : f == kQ4_0 || f == kQ4_1 || f == kQ8_0 ? 32u : f == kQ6_K ? 256u : 0u;
}
// The unquantized formats: a group is its 32 values as stored, 128 or 64 bytes.
constexpr bool plain_values(uint32_t f) { return f == kF32 || f == kF16 || f == kBF16; }

// binary16 bits -> binary32, exact for every finite input, subnormals
// included (the f16 denormal mode is left at its IEEE default).
__device__ __forceinline__ float half_to_float(uint32_t bits) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits)));
}

// bfloat16 -> binary32: the value's 16 bits are the top of the f32 (the low
// half of a dword shifted up, the high half masked), exact.
__device__ __forceinline__ float bf16_low(uint32_t word) { return __uint_as_float(word << 16); }
__device__ __forceinline__ float bf16_high(uint32_t word) { return __uint_as_float(word & 0xFFFF0000u); }

// The 16 code bytes and scale of Q4_0 group gi, and the group's data of Q6_K.
struct Q4_0Group {
    uint32_t w[4];
    float d, minus_8d;
};

struct Q6_KGroup {
    uint32_t lo[4];
    uint32_t hi[2];
    float first, minus_32_first, second, minus_32_second;
};

// A group's bytes as loaded, before any arithmetic on them (fetch_*), and
// the group they make (group_of): a kernel may load a group well before it
// uses it without waiting on the loads at once.
struct Q4_0Bytes {
    uint4 c;
    uint32_t d;
};

__device__ __forceinline__ Q4_0Bytes fetch_q4_0(const uint8_t* piece, uint64_t n, uint64_t gi) {
    return {*reinterpret_cast<const uint4*>(piece + 16 * gi), *reinterpret_cast<const uint16_t*>(piece + 16 * n + 2 * gi)};
}

__device__ __forceinline__ Q4_0Group group_of(const Q4_0Bytes& b) {
    Q4_0Group g;
    g.w[0] = b.c.x;
    g.w[1] = b.c.y;
    g.w[2] = b.c.z;
    g.w[3] = b.c.w;
    g.d = half_to_float(b.d);
    g.minus_8d = -8.0f * g.d;
    return g;
}

__device__ __forceinline__ Q4_0Group load_q4_0(const uint8_t* piece, uint64_t n, uint64_t gi) {
    return group_of(fetch_q4_0(piece, n, gi));
}

struct Q6_KBytes {
    uint4 lo;
    uint2 hi;
    uint32_t sc, d;
};

__device__ __forceinline__ Q6_KBytes fetch_q6_k(const uint8_t* piece, uint64_t n, uint64_t gi) {
    return {*reinterpret_cast<const uint4*>(piece + 16 * gi), *reinterpret_cast<const uint2*>(piece + 128 * n + 8 * gi),
            *reinterpret_cast<const uint16_t*>(piece + 192 * n + 2 * gi),
            *reinterpret_cast<const uint16_t*>(piece + 208 * n + 2 * (gi / 8))};
}

__device__ __forceinline__ Q6_KGroup group_of(const Q6_KBytes& b) {
    Q6_KGroup g;
    const float d = half_to_float(b.d);
    g.lo[0] = b.lo.x;
    g.lo[1] = b.lo.y;
    g.lo[2] = b.lo.z;
    g.lo[3] = b.lo.w;
    g.hi[0] = b.hi.x;
    g.hi[1] = b.hi.y;
    g.first = d * static_cast<float>(static_cast<int8_t>(b.sc & 0xFFu));
    g.second = d * static_cast<float>(static_cast<int8_t>(b.sc >> 8));
    g.minus_32_first = -32.0f * g.first;
    g.minus_32_second = -32.0f * g.second;
    return g;
}

__device__ __forceinline__ Q6_KGroup load_q6_k(const uint8_t* piece, uint64_t n, uint64_t gi) {
    return group_of(fetch_q6_k(piece, n, gi));
}

struct Q4_1Group {
    uint32_t w[4];
    float d, m;
};

struct Q8_0Group {
    uint32_t w[8];
    float d;
};

struct Q4_1Bytes {
    uint4 c;
    uint32_t dm;
};

__device__ __forceinline__ Q4_1Bytes fetch_q4_1(const uint8_t* piece, uint64_t n, uint64_t gi) {
    return {*reinterpret_cast<const uint4*>(piece + 16 * gi), *reinterpret_cast<const uint32_t*>(piece + 16 * n + 4 * gi)};
}

__device__ __forceinline__ Q4_1Group group_of(const Q4_1Bytes& b) {
    Q4_1Group g;
    g.w[0] = b.c.x;
    g.w[1] = b.c.y;
    g.w[2] = b.c.z;
    g.w[3] = b.c.w;
    g.d = half_to_float(b.dm & 0xFFFFu);
    g.m = half_to_float(b.dm >> 16);
    return g;
}

__device__ __forceinline__ Q4_1Group load_q4_1(const uint8_t* piece, uint64_t n, uint64_t gi) {
    return group_of(fetch_q4_1(piece, n, gi));
}

struct Q8_0Bytes {
    uint4 a, b;
    uint32_t d;
};

__device__ __forceinline__ Q8_0Bytes fetch_q8_0(const uint8_t* piece, uint64_t n, uint64_t gi) {
    const uint4* c = reinterpret_cast<const uint4*>(piece + 32 * gi);
    return {c[0], c[1], *reinterpret_cast<const uint16_t*>(piece + 32 * n + 2 * gi)};
}

__device__ __forceinline__ Q8_0Group group_of(const Q8_0Bytes& b) {
    Q8_0Group g;
    g.w[0] = b.a.x;
    g.w[1] = b.a.y;
    g.w[2] = b.a.z;
    g.w[3] = b.a.w;
    g.w[4] = b.b.x;
    g.w[5] = b.b.y;
    g.w[6] = b.b.z;
    g.w[7] = b.b.w;
    g.d = half_to_float(b.d);
    return g;
}

__device__ __forceinline__ Q8_0Group load_q8_0(const uint8_t* piece, uint64_t n, uint64_t gi) {
    return group_of(fetch_q8_0(piece, n, gi));
}

// Half h of an unquantized group — values 16h .. 16h + 15 — as the prefill
// tile stages it: F32 four float4s, F16 and BF16 two dwords' worth of uint4.
template <uint32_t F>
struct ValuesHalf {
    uint4 v[F == kF32 ? 4 : 2];
};

template <uint32_t F>
__device__ __forceinline__ ValuesHalf<F> fetch_values_half(const uint8_t* piece, uint64_t gi, uint32_t h) {
    constexpr uint32_t group_bytes = F == kF32 ? 128u : 64u;
    const uint4* at = reinterpret_cast<const uint4*>(piece + group_bytes * gi + group_bytes / 2 * h);
    ValuesHalf<F> out;
#pragma unroll
    for (int i = 0; i < (F == kF32 ? 4 : 2); ++i) out.v[i] = at[i];
    return out;
}

// Value j (0..15) of a fetched half, exact.
template <uint32_t F>
__device__ __forceinline__ float value(const ValuesHalf<F>& h, int j) {
    const uint4 q = h.v[F == kF32 ? j >> 2 : j >> 3];
    const int word = F == kF32 ? j & 3 : (j >> 1) & 3;
    const uint32_t w = word == 0 ? q.x : word == 1 ? q.y : word == 2 ? q.z : q.w;
    if constexpr (F == kF32) return __uint_as_float(w);
    else if constexpr (F == kF16) return half_to_float((j & 1) ? w >> 16 : w & 0xFFFFu);
    else return (j & 1) ? bf16_high(w) : bf16_low(w);
}

// Weight l (0..31) of a group, exact.
__device__ __forceinline__ float weight(const Q4_0Group& g, int l) {
    const uint32_t q = (g.w[(l & 15) >> 2] >> (8 * (l & 3) + 4 * (l >> 4))) & 0xFu;
    return __builtin_fmaf(static_cast<float>(q), g.d, g.minus_8d);
}

__device__ __forceinline__ float weight(const Q6_KGroup& g, int l) {
    const uint32_t low = (g.lo[(l & 15) >> 2] >> (8 * (l & 3) + 4 * (l >> 4))) & 0xFu;
    const uint32_t pair = (g.hi[(l & 7) >> 2] >> (8 * (l & 3) + 2 * (l >> 3))) & 3u;
    const float q = static_cast<float>(low | (pair << 4));
    return l < 16 ? __builtin_fmaf(q, g.first, g.minus_32_first) : __builtin_fmaf(q, g.second, g.minus_32_second);
}

// s continued over the group's 32 weights in k order, each an fma:
// s = fma(w_l, x_l, s) for l = 0..31 (matmul.wgsl:121-126, 224-230).
template <typename G>
__device__ __forceinline__ float chain(const G& g, const float* x, float s) {
#pragma unroll
    for (int l = 0; l < 32; ++l) s = __builtin_fmaf(weight(g, l), x[l], s);
    return s;
}

__device__ __forceinline__ float weight(const Q4_1Group& g, int l) {
    const uint32_t q = (g.w[(l & 15) >> 2] >> (8 * (l & 3) + 4 * (l >> 4))) & 0xFu;
    return __builtin_fmaf(static_cast<float>(q), g.d, g.m);
}

__device__ __forceinline__ float weight(const Q8_0Group& g, int l) {
    const int32_t q = static_cast<int8_t>((g.w[l >> 2] >> (8 * (l & 3))) & 0xFFu);
    return static_cast<float>(q) * g.d;
}

template <uint32_t F>
__device__ __forceinline__ float chain_group(const uint8_t* piece, uint64_t n, uint64_t gi, const float* x, float s) {
    if constexpr (F == kQ4_0) {
        return chain(load_q4_0(piece, n, gi), x, s);
    } else if constexpr (F == kQ4_1) {
        return chain(load_q4_1(piece, n, gi), x, s);
    } else if constexpr (F == kQ8_0) {
        return chain(load_q8_0(piece, n, gi), x, s);
    } else {
        return chain(load_q6_k(piece, n, gi), x, s);
    }
}

// The 32 weights of group gi, exact (the unpack of format.h:36-77).
template <uint32_t F>
__device__ __forceinline__ void unpack(const uint8_t* piece, uint64_t n, uint64_t gi, float* out) {
    if constexpr (F == kQ4_0) {
        const Q4_0Group g = load_q4_0(piece, n, gi);
#pragma unroll
        for (int l = 0; l < 32; ++l) out[l] = weight(g, l);
    } else if constexpr (F == kQ4_1) {
        const Q4_1Group g = load_q4_1(piece, n, gi);
#pragma unroll
        for (int l = 0; l < 32; ++l) out[l] = weight(g, l);
    } else if constexpr (F == kQ8_0) {
        const Q8_0Group g = load_q8_0(piece, n, gi);
#pragma unroll
        for (int l = 0; l < 32; ++l) out[l] = weight(g, l);
    } else if constexpr (F == kF32) {
        const float4* f = reinterpret_cast<const float4*>(piece + 128 * gi);
#pragma unroll
        for (int v = 0; v < 8; ++v) {
            const float4 q = f[v];
            out[4 * v] = q.x;
            out[4 * v + 1] = q.y;
            out[4 * v + 2] = q.z;
            out[4 * v + 3] = q.w;
        }
    } else if constexpr (F == kF16 || F == kBF16) {
        const uint4* h = reinterpret_cast<const uint4*>(piece + 64 * gi);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const uint4 q = h[v];
            const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                out[8 * v + 2 * i] = F == kF16 ? half_to_float(w[i] & 0xFFFFu) : bf16_low(w[i]);
                out[8 * v + 2 * i + 1] = F == kF16 ? half_to_float(w[i] >> 16) : bf16_high(w[i]);
            }
        }
    } else {
        const Q6_KGroup g = load_q6_k(piece, n, gi);
#pragma unroll
        for (int l = 0; l < 32; ++l) out[l] = weight(g, l);
    }
}

// Range r of a row's G groups: groups [range_lo(r, G), range_lo(r + 1, G))
// (matmul.wgsl:134-137).
__host__ __device__ __forceinline__ uint32_t range_lo(uint32_t r, uint32_t groups) {
    return static_cast<uint32_t>((static_cast<uint64_t>(r) * groups) / 32u);
}

}  // namespace chm
