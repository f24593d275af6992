// Decode: the matrix-vector product, one token, bound by reading each weight
// once from HBM. Every output in the canonical order (formats.hpp's chain,
// range sums added in order from zero), so its bits are the prefill tile's
// and the CPU restatement's.
//
// gemv_ranges — the reference's lane mapping (matmul.wgsl:207-296) on wave64:
// a wave is two half-waves, each taking one row at a time; lane r of a half
// owns range r, so the half's 32 lanes read 32 adjacent groups of the row —
// adjacent 16-byte code blocks, coalesced — and lane r's slice of x never
// changes, so it is loaded into registers once per wave and reused for every
// row the wave takes. Each half takes `rows_per_half` consecutive rows (1 to
// 32, chosen so the launch still fills the GPU); the range sums meet in LDS
// and lane i then adds row i's 32 sums in order, all lanes at once.
#include "product.hpp"

namespace chm {

constexpr int kWaves = 4;        // waves a workgroup
constexpr int kPad = 33;         // a row's 32 range sums, padded so lane-per-row reads spread over banks

__device__ __forceinline__ void write_output(const Product& a, uint32_t p, float total) {
    uint32_t row;
    const int m = locate(a, p, &row);
    const Member& mem = a.m[m];
    const uint32_t at = (a.epilogue == kQKV ? 0u : mem.out_row) + (p - mem.first);
    mem.out[at] = total;
}

// MAXG > 0: every range holds at most MAXG groups and x's slice lives in
// registers. MAXG == 0: any width; x is read per group (from cache).
template <uint32_t F, int MAXG>
__global__ __launch_bounds__(256) void gemv_ranges(Product a, uint32_t rows_per_half) {
    __shared__ float partials[kWaves][64 * kPad];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t half = lane >> 5, r = lane & 31u;
    const uint32_t G = a.groups;
    const uint32_t g0 = range_lo(r, G), g1 = range_lo(r + 1, G);
    const uint32_t token = a.last_token ? a.tokens - 1 : 0;
    const float* x = a.x + static_cast<uint64_t>(token) * G * 32;
    const uint32_t first_row = ((blockIdx.x * kWaves + wave) * 2 + half) * rows_per_half;

    float xr[MAXG > 0 ? MAXG * 32 : 1];
    if constexpr (MAXG > 0) {
#pragma unroll
        for (int i = 0; i < MAXG; ++i) {
            if (g0 + i < g1) {
                const float4* src = reinterpret_cast<const float4*>(x + (g0 + i) * 32);
#pragma unroll
                for (int v = 0; v < 8; ++v) {
                    const float4 q = src[v];
                    xr[i * 32 + 4 * v + 0] = q.x;
                    xr[i * 32 + 4 * v + 1] = q.y;
                    xr[i * 32 + 4 * v + 2] = q.z;
                    xr[i * 32 + 4 * v + 3] = q.w;
                }
            }
        }
    }

    float* mine = partials[wave];
    for (uint32_t i = 0; i < rows_per_half; ++i) {
        const uint32_t p = first_row + i;
        float s = 0.0f;
        if (p < a.rows) {
            uint32_t row;
            const Member& mem = a.m[locate(a, p, &row)];
            const uint64_t base = static_cast<uint64_t>(row) * G;
            if constexpr (MAXG > 0) {
#pragma unroll
                for (int j = 0; j < MAXG; ++j) {
                    if (g0 + j < g1) s = chain_group<F>(mem.piece, mem.blocks, base + g0 + j, xr + 32 * j, s);
                }
            } else {
                for (uint32_t g = g0; g < g1; ++g) {
                    float xg[32];
                    const float4* src = reinterpret_cast<const float4*>(x + g * 32);
#pragma unroll
                    for (int v = 0; v < 8; ++v) {
                        const float4 q = src[v];
                        xg[4 * v + 0] = q.x;
                        xg[4 * v + 1] = q.y;
                        xg[4 * v + 2] = q.z;
                        xg[4 * v + 3] = q.w;
                    }
                    s = chain_group<F>(mem.piece, mem.blocks, base + g, xg, s);
                }
            }
        }
        mine[(half * rows_per_half + i) * kPad + r] = s;
    }
    __syncthreads();
    if (lane < 2 * rows_per_half) {
        const uint32_t p = ((blockIdx.x * kWaves + wave) * 2 + lane / rows_per_half) * rows_per_half +
                           lane % rows_per_half;
        if (p < a.rows) {
            const float* sums = mine + lane * kPad;
            float total = 0.0f;
#pragma unroll
            for (int q = 0; q < 32; ++q) total = total + sums[q];
            write_output(a, p, total);
        }
    }
}

template <uint32_t F>
static hipError_t launch_format(const Product& a, uint32_t rows_per_half, hipStream_t stream) {
    const uint32_t rows_a_block = kWaves * 2 * rows_per_half;
    const dim3 grid((a.rows + rows_a_block - 1) / rows_a_block);
    const uint32_t span = (a.groups + 31) / 32;  // the most groups a range holds
    switch (span) {
        case 1: hipLaunchKernelGGL((gemv_ranges<F, 1>), grid, dim3(256), 0, stream, a, rows_per_half); break;
        case 2: hipLaunchKernelGGL((gemv_ranges<F, 2>), grid, dim3(256), 0, stream, a, rows_per_half); break;
        case 3: hipLaunchKernelGGL((gemv_ranges<F, 3>), grid, dim3(256), 0, stream, a, rows_per_half); break;
        default: hipLaunchKernelGGL((gemv_ranges<F, 0>), grid, dim3(256), 0, stream, a, rows_per_half); break;
    }
    return hipGetLastError();
}

// Rows a half-wave takes: the most, up to 32, that still gives every CU
// about 8 waves, so x's registers are reused as far as the GPU's fill allows.
uint32_t gemv_rows_per_half(uint32_t rows, uint32_t compute_units) {
    const uint32_t waves = compute_units * 8;
    uint32_t rph = rows / (2 * waves);
    if (rph < 1) rph = 1;
    if (rph > 32) rph = 32;
    return rph;
}

hipError_t launch_gemv(const Product& a, uint32_t format, uint32_t compute_units, hipStream_t stream) {
    const uint32_t rph = gemv_rows_per_half(a.rows, compute_units);
    if (format == kQ4_0) return launch_format<kQ4_0>(a, rph, stream);
    return launch_format<kQ6_K>(a, rph, stream);
}

}  // namespace chm
