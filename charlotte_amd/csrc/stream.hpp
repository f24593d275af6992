// What the LDS-streamed decodes (gemv_stream.hip, gemv_stream8.hip) share:
// the DMA copy of a stream's 16-byte chunks into a wave's LDS stage, and the
// wait for it.
#pragma once

#include "limbs.hpp"

namespace chm {

typedef __attribute__((address_space(3))) void* lds_void;

// vmcnt(0) alone, in s_waitcnt's gfx9 encoding (the other counters at
// their no-wait values).
constexpr int kVmcnt0 = (0x7 << 4) | (0xF << 8);

// Copies `kChunks` 16-byte chunks from `from` to LDS `to`, 64 a wave
// instruction (lanes past the last chunk copy nothing): whole 1 KB runs,
// nothing landing in registers.
template <uint32_t kChunks>
__device__ __forceinline__ void copy_stream(const uint8_t* from, u32x4s_t* to, uint32_t lane) {
#pragma unroll
    for (uint32_t i = 0; i < (kChunks + 63) / 64; ++i) {
        if (64 * i + 64 <= kChunks || 64 * i + lane < kChunks)
            __builtin_amdgcn_global_load_lds(from + 16 * (64 * i + lane), (lds_void)(to + 64 * i), 16, 0, 0);
    }
}

}  // namespace chm
