// Prefill: the tiled matrix product over a step's tokens.
//
// gemm_canonical — VALU, the canonical order, bit-exact with decode and the
// CPU restatement (matmul.wgsl:395-533 restated for CDNA4). A workgroup of
// 256 lanes takes a tile of BM tokens x 128 rows and walks K one 32-weight
// group at a time: the group's 128 rows are decoded once into LDS (exact
// f32), the tokens' 32 inputs staged beside them, then each lane runs its
// micro-tile of TM tokens x 8 rows, 32 multiply-adds in k order per output,
// each output keeping its range sum and its total: at a range's last group
// the total adds the range sum and the range sum restarts from zero. So every
// output's order of addition is decode's, whatever BM. Workgroups are
// numbered token tile first, so the tiles that read one weight tile run
// together and find it in L2 (matmul.wgsl:480-482).
#include "product.hpp"

namespace chm {

constexpr int kRowsATile = 128;

__device__ __forceinline__ void store_output(const Product& a, uint32_t token, uint32_t p, float v) {
    *output_of(a, p, token) = v;
}

template <uint32_t F, int BM>
__global__ __launch_bounds__(256) void gemm_canonical(Product a, uint32_t token_tiles) {
    constexpr int TM = BM / 16;  // a lane's tokens
    __shared__ float4 Ws[32][kRowsATile / 4];
    __shared__ float4 Xs[32][BM / 4];
    const uint32_t t = threadIdx.x, tx = t & 15u, ty = t >> 4;
    const uint32_t tile_t = blockIdx.x % token_tiles, tile_r = blockIdx.x / token_tiles;
    const uint32_t m0 = tile_t * BM, n0 = tile_r * kRowsATile;
    const uint32_t G = a.groups, K = G * 32;

    // Staging roles: weights — row t % 128, weights 16 (t / 128) .. + 15 of
    // its group; inputs — BM tokens x 32 floats, BM / 8 floats a lane.
    const uint32_t srow = t & 127u, shalf = t >> 7;
    const uint32_t sp = n0 + srow;
    const bool slive = sp < a.rows;
    const Piece spiece = piece_of(a, slive ? sp : 0);
    constexpr int XPer = BM / 8;                 // floats a lane stages: 16 or 8
    const uint32_t xtok = t % BM, xpart = t / BM;
    const bool xlive = m0 + xtok < a.tokens;
    const float* xsrc = a.x + static_cast<uint64_t>(m0 + xtok) * K + xpart * XPer;
    float* wflat = reinterpret_cast<float*>(Ws);
    float* xflat = reinterpret_cast<float*>(Xs);

    float s[TM][8], tot[TM][8];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) s[i][j] = tot[i][j] = 0.0f;

    uint32_t next_r = 1;  // the next range boundary, range_lo(next_r)
    while (next_r < 32 && range_lo(next_r, G) == 0) ++next_r;

    for (uint32_t g = 0; g < G; ++g) {
        __syncthreads();  // the last group's tiles are read
        {
            float w[16];
            if (slive) {
                const uint64_t gi = static_cast<uint64_t>(spiece.row) * G + g;
                if constexpr (F == kQ4_0) {
                    const Q4_0Group q = load_q4_0(spiece.piece, spiece.blocks, gi);
#pragma unroll
                    for (int j = 0; j < 16; ++j) w[j] = weight(q, 16 * shalf + j);
                } else {
                    const Q6_KGroup q = load_q6_k(spiece.piece, spiece.blocks, gi);
#pragma unroll
                    for (int j = 0; j < 16; ++j) w[j] = weight(q, 16 * shalf + j);
                }
            } else {
#pragma unroll
                for (int j = 0; j < 16; ++j) w[j] = 0.0f;
            }
#pragma unroll
            for (int j = 0; j < 16; ++j) wflat[(16 * shalf + j) * kRowsATile + srow] = w[j];
        }
        {
            float xv[XPer];
            if (xlive) {
                const float4* src = reinterpret_cast<const float4*>(xsrc + g * 32);
#pragma unroll
                for (int v = 0; v < XPer / 4; ++v) {
                    const float4 q = src[v];
                    xv[4 * v] = q.x;
                    xv[4 * v + 1] = q.y;
                    xv[4 * v + 2] = q.z;
                    xv[4 * v + 3] = q.w;
                }
            } else {
#pragma unroll
                for (int v = 0; v < XPer; ++v) xv[v] = 0.0f;
            }
#pragma unroll
            for (int v = 0; v < XPer; ++v) xflat[(xpart * XPer + v) * BM + xtok] = xv[v];
        }
        __syncthreads();
#pragma unroll 4
        for (int k = 0; k < 32; ++k) {
            const float4 wa = Ws[k][tx], wb = Ws[k][16 + tx];
            const float w[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
            float x[TM];
            const float4 xa = Xs[k][ty];
            x[0] = xa.x;
            x[1] = xa.y;
            x[2] = xa.z;
            x[3] = xa.w;
            if constexpr (TM == 8) {
                const float4 xb = Xs[k][16 + ty];
                x[4] = xb.x;
                x[5] = xb.y;
                x[6] = xb.z;
                x[7] = xb.w;
            }
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < 8; ++j) s[i][j] = __builtin_fmaf(w[j], x[i], s[i][j]);
        }
        if (g + 1 == range_lo(next_r, G)) {
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    tot[i][j] = tot[i][j] + s[i][j];
                    s[i][j] = 0.0f;
                }
            while (next_r < 32 && range_lo(next_r, G) <= g + 1) ++next_r;
        }
    }

#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const uint32_t token = m0 + 4 * ty + (i & 3) + 64 * (i >> 2);
        if (token >= a.tokens) continue;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t p = n0 + 4 * tx + (j & 3) + 64 * (j >> 2);
            if (p < a.rows) store_output(a, token, p, tot[i][j]);
        }
    }
}

hipError_t launch_gemm_canonical(const Product& a, uint32_t format, uint32_t compute_units, hipStream_t stream) {
    const uint32_t row_tiles = (a.rows + kRowsATile - 1) / kRowsATile;
    const bool wide = ((a.tokens + 127) / 128) * row_tiles >= 2 * compute_units;
    if (wide) {
        const uint32_t token_tiles = (a.tokens + 127) / 128;
        const dim3 grid(token_tiles * row_tiles);
        if (format == kQ4_0)
            hipLaunchKernelGGL((gemm_canonical<kQ4_0, 128>), grid, dim3(256), 0, stream, a, token_tiles);
        else
            hipLaunchKernelGGL((gemm_canonical<kQ6_K, 128>), grid, dim3(256), 0, stream, a, token_tiles);
    } else {
        const uint32_t token_tiles = (a.tokens + 63) / 64;
        const dim3 grid(token_tiles * row_tiles);
        if (format == kQ4_0)
            hipLaunchKernelGGL((gemm_canonical<kQ4_0, 64>), grid, dim3(256), 0, stream, a, token_tiles);
        else
            hipLaunchKernelGGL((gemm_canonical<kQ6_K, 64>), grid, dim3(256), 0, stream, a, token_tiles);
    }
    return hipGetLastError();
}

}  // namespace chm
