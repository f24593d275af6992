// Host-side device layout (layout.cpp), as the C ABI (capi.cpp) calls it.
#pragma once

#include <stdint.h>

namespace chm {

// GGUF types 0 F32, 1 F16, 2 Q4_0, 3 Q4_1, 8 Q8_0, 14 Q6_K, 30 BF16
// (src/core/gguf/types.h:65-101).
constexpr uint32_t block_bytes_host(uint32_t f) {
    return f == 0 ? 4u : f == 1 || f == 30 ? 2u : f == 2 ? 18u : f == 3 ? 20u : f == 8 ? 34u : f == 14 ? 210u : 0u;
}
constexpr uint32_t block_weights_host(uint32_t f) {
    return f == 0 || f == 1 || f == 30 ? 1u : f == 2 || f == 3 || f == 8 ? 32u : f == 14 ? 256u : 0u;
}

uint64_t layout_bytes(uint32_t format, uint64_t blocks);
bool lay_out(uint32_t format, const uint8_t* stored, uint64_t blocks, uint8_t* device);
void repack_q6_k(const uint8_t* stored, uint64_t blocks, uint8_t* lo, uint8_t* hi, uint8_t* scales, uint8_t* d);

}  // namespace chm
