// Host-side device layout (layout.cpp) and the kernels' launchers, as the
// C ABI (capi.cpp) calls them.
#pragma once

#include <stdint.h>

#include <hip/hip_runtime_api.h>

namespace chm {

struct Product;

// GGUF types 0 F32, 2 Q4_0, 3 Q4_1, 8 Q8_0, 14 Q6_K (src/core/gguf/types.h:65-101).
constexpr uint32_t block_bytes_host(uint32_t f) {
    return f == 0 ? 4u : f == 2 ? 18u : f == 3 ? 20u : f == 8 ? 34u : f == 14 ? 210u : 0u;
}
constexpr uint32_t block_weights_host(uint32_t f) {
    return f == 0 ? 1u : f == 2 || f == 3 || f == 8 ? 32u : f == 14 ? 256u : 0u;
}

uint64_t layout_bytes(uint32_t format, uint64_t blocks);
bool lay_out(uint32_t format, const uint8_t* stored, uint64_t blocks, uint8_t* device);
void repack_q6_k(const uint8_t* stored, uint64_t blocks, uint8_t* lo, uint8_t* hi, uint8_t* scales, uint8_t* d);

bool gemv_supports(uint32_t groups);
bool gemv_limbs_takes(const Product& a, uint32_t format);
hipError_t launch_gemv(const Product& a, uint32_t format, uint32_t compute_units, bool limbs, hipStream_t stream);
hipError_t launch_gemm_canonical(const Product& a, uint32_t format, uint32_t compute_units, float* range_sums,
                                 hipStream_t stream);
uint64_t mfma_workspace_bytes(uint32_t tokens, uint32_t groups);
hipError_t launch_gemm_mfma(const Product& a, uint32_t format, uint32_t compute_units, void* workspace,
                            hipStream_t stream);

}  // namespace chm
