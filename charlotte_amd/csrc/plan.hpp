// How a product runs — which kernel, its tile, its grid — chosen on the host
// from the product's shape and the device's compute units alone, so a caller
// can ask without a device (charlotte_hip_matmul_plan_launch) and a launch
// runs exactly what its plan says. The role of the reference's pure launcher,
// kernels::matmul_launches (src/core/kernels/matmul/matmul.h:661-673,
// src/core/kernels/interface.h:29-34).
#pragma once

#include <stdint.h>

#include <hip/hip_runtime_api.h>

namespace chm {

struct Product;

// Values are the C ABI's charlotte_hip_matmul_kernel.
enum Kernel : uint32_t {
    kNoKernel = 0,
    kGemvRanges = 1,    // decode, 32 lanes a row, lane r range r (the reference's mapping)
    kGemvQuarters = 2,  // decode, 4 lanes a row, 9 groups each (K = 1,152)
    kGemvStream = 3,    // decode, LDS-streamed Q6_K, K = 1,152
    kGemvStream8 = 4,   // decode, LDS-streamed Q6_K, K = 1,024 and 2,048
    kGemvChunked = 5,   // decode past K = 8,192: x staged a chunk of groups at a time
    kGemvStream4 = 6,   // decode, LDS-streamed Q4_0, K = 1,024 .. 8,192 (powers of two)
    kGemvWide = 7,      // decode, LDS-streamed Q4_0, K = 9,216 .. 16,384 (whole 1,024s), a lane a range
    kGemmTiled = 16,    // prefill, the VALU tile
    kGemmSplit = 17,    // prefill split along K, then the ordered combine
    kGemmMfma = 18,     // prefill on the matrix cores, x split into two f16 parts
    kGemmShort = 19,    // prefill of a short step: 16 or 8 rows x 32 tokens, K split among the waves
    kGemmExact = 20,    // prefill on the matrix cores' K = 1 f32 instruction, the canonical order
    kGemmExactSplit = 21,  // the same split along K, then the ordered combine
    kGemmExactShort = 22,  // a short step on the matrix cores: 32 x 32, K split among 8 waves
};

struct Plan {
    uint32_t kernel = kNoKernel;
    uint32_t launches = 0;     // kernel launches the product issues
    bool canonical = true;     // the reference's order of addition: bit-exact, batch-invariant
    bool limbs = false;        // decode: the INT8_LIMBS form
    bool xreg = false;         // decode (L = 32): x's slice held in registers
    uint32_t lanes = 0;        // decode: lanes a row
    uint32_t span = 0;         // decode: the most groups a lane holds
    uint32_t steps = 0;        // decode: steps a wave
    uint32_t waves = 4;        // decode (L = 32): waves a workgroup, 4 or 1
    uint32_t tile_tokens = 0;  // prefill: tokens a workgroup's tile (decode: 1)
    uint32_t tile_rows = 0;    // product rows a workgroup's tile
    uint32_t token_tiles = 0, row_tiles = 0;
    uint32_t chunks = 1;       // the split along K: workgroups a tile
    uint32_t wave_rows = 0, wave_tokens = 0;  // matrix cores: 16-row and 16-token blocks a wave
    uint64_t tiles = 0;        // the main kernel's tiles; persistent decode grids loop over them
    uint64_t workgroups = 0;   // the main kernel's grid (persistent decode grids: at most this)
};

// Decode. False when the shape has no decode kernel.
bool plan_gemv(const Product& a, uint32_t format, uint32_t compute_units, bool limbs, Plan* plan);
hipError_t launch_gemv(const Product& a, uint32_t format, const Plan& plan, uint32_t compute_units,
                       hipStream_t stream);
bool gemv_stream_takes(const Product& a, uint32_t format);
bool gemv_stream8_takes(const Product& a, uint32_t format);
bool gemv_stream4_takes(const Product& a, uint32_t format);
hipError_t launch_gemv_stream(const Product& a, uint32_t compute_units, bool limbs, hipStream_t stream);
hipError_t launch_gemv_stream8(const Product& a, uint32_t compute_units, bool limbs, hipStream_t stream);
hipError_t launch_gemv_stream4(const Product& a, uint32_t compute_units, bool limbs, hipStream_t stream);
uint64_t gemv_stream4_workgroups(uint32_t groups, uint32_t compute_units, uint64_t steps);
bool gemv_wide_takes(const Product& a, uint32_t format);
hipError_t launch_gemv_wide(const Product& a, uint32_t compute_units, hipStream_t stream);
uint64_t gemv_wide_workgroups(uint32_t compute_units, uint64_t steps);

// Prefill on the VALU tile; `split` for the split along K.
void plan_gemm_canonical(const Product& a, uint32_t compute_units, bool split, Plan* plan);
hipError_t launch_gemm_canonical(const Product& a, uint32_t format, const Plan& plan, float* range_sums,
                                 hipStream_t stream);
// The split form's ordered combine of range sums (gemm.hip).
hipError_t launch_combine_ranges(const Product& a, const float* range_sums, hipStream_t stream);

// Prefill of a short step (gemm_short.hip): a step that does not split and
// whose 128-row tiles would leave compute units idle.
void plan_gemm_short(const Product& a, uint32_t compute_units, Plan* plan);
hipError_t launch_gemm_short(const Product& a, uint32_t format, const Plan& plan, hipStream_t stream);

// Prefill on the matrix cores in the canonical order (gemm_exact.hip):
// every format, every epilogue, the VALU tile's bits.
void plan_gemm_exact(const Product& a, uint32_t format, uint32_t compute_units, bool split, Plan* plan);
void plan_gemm_exact_short(const Product& a, uint32_t compute_units, Plan* plan);
hipError_t launch_gemm_exact_short(const Product& a, uint32_t format, const Plan& plan, hipStream_t stream);
hipError_t launch_gemm_exact(const Product& a, uint32_t format, const Plan& plan, float* range_sums,
                             hipStream_t stream);

// Prefill on the matrix cores, x split into two f16 parts.
bool mfma_reads(uint32_t format);
uint64_t mfma_workspace_bytes(uint32_t tokens, uint32_t groups);
void plan_gemm_mfma(const Product& a, uint32_t format, uint32_t compute_units, Plan* plan);
hipError_t launch_gemm_mfma(const Product& a, uint32_t format, const Plan& plan, void* workspace,
                            hipStream_t stream);

}  // namespace chm
