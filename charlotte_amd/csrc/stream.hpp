// What the LDS-streamed decodes share: the DMA copy of a stream's 16-byte
// chunks into a wave's LDS stage, the wait for it, and a row's ordered total
// from its range sums in LDS.
#pragma once

#include "limbs.hpp"

namespace chm {

typedef __attribute__((address_space(3))) void* lds_void;

// vmcnt(0) alone, in s_waitcnt's gfx9 encoding (the other counters at
// their no-wait values).
constexpr int kVmcnt0 = (0x7 << 4) | (0xF << 8);

// The cache policy of the streamed decodes' weight copies: non-temporal
// (the instruction's nt bit). A decode reads each weight byte once, and the
// part reads a stream so marked markedly faster: C2's 248.8 MB by the LDS
// copy in 9 KB wave steps 40.4 -> 36.6 us, in 4 KB steps 39.1 -> 35.1 us
// (7.07 TB/s); the canonical C2 decode 48.4-50.5 -> 46.8-47.2 us, its
// INT8_LIMBS form 46.9 -> 42.5 us (two rounds A/B on one box).
constexpr int kStreamPolicy = 2;

// Copies `kChunks` 16-byte chunks from `from` to LDS `to`, 64 a wave
// instruction (lanes past the last chunk copy nothing): whole 1 KB runs,
// nothing landing in registers.
template <uint32_t kChunks>
__device__ __forceinline__ void copy_stream(const uint8_t* from, u32x4s_t* to, uint32_t lane) {
#pragma unroll
    for (uint32_t i = 0; i < (kChunks + 63) / 64; ++i) {
        if (64 * i + 64 <= kChunks || 64 * i + lane < kChunks)
            __builtin_amdgcn_global_load_lds(from + 16 * (64 * i + lane), (lds_void)(to + 64 * i), 16, 0,
                                             kStreamPolicy);
    }
}

// A row's 32 range sums added in order from zero — ((0 + s0) + s1) + ...,
// the order of matmul.h:34-50 — read from LDS in eight 16-byte reads issued
// together: one LDS round trip, where reads of a pair at a time between the
// adds took four (Q4_0 3,072 x 1,024: 3.55 -> 3.42 us). `row` is 16-byte
// aligned; the reads claim memory, so the row's stores stay above them.
__device__ __forceinline__ float ordered_total(const float* row) {
    const uint32_t at = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(row));
    u32x4s_t v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k)
        __asm__ __volatile__("ds_read_b128 %0, %1 offset:%2" : "=v"(v[k]) : "v"(at), "i"(16 * k) : "memory");
    __asm__ __volatile__("s_waitcnt lgkmcnt(0)"
                         : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]), "+v"(v[7]));
    float total = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k)
#pragma unroll
        for (int e = 0; e < 4; ++e) total = total + __uint_as_float(v[k][e]);
    return total;
}

}  // namespace chm
