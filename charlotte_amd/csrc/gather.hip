// The embedding gather (src/core/kernels/gather/gather.h, gather.wgsl:21-58):
// row i of `hidden` becomes the table row of the step's token i, each weight
// decoded exactly through the table's format — the same decode the products
// use — then multiplied by the scale. And its position form
// (gather.wgsl:65-84): a vision patch row's column row plus its row row of
// an F32 table.
//
// Every weight is the file-order decode's bits, the sign of a zero included.
//
// Mapping: eight lanes a 32-weight group, lane v decoding weights 4v .. 4v + 3
// and storing them as one float4, so a wave's store writes 1 KiB of `hidden`
// contiguously (8 groups of a row, or the end of one row and the start of the
// next). Each lane reads one dword of codes (Q8_0, Q4_0, Q4_1; two for Q6_K)
// and its group's scales. Bound by the writes: 4 bytes a weight out against
// at most 1.1 bytes a weight read.
//
// A lane whose token lies outside the piece, or is the media placeholder of
// a step that carries a medium, writes nothing: the piece holding it, or the
// media encoder, writes that row (gather.h).
#include "gather.hpp"

namespace chm {

// Weights 4v .. 4v + 3 of group gi of a piece, exact.
template <uint32_t F>
__device__ __forceinline__ float4 unpack4(const uint8_t* piece, uint64_t n, uint64_t gi, uint32_t v) {
    if constexpr (F == kF32) {
        return *reinterpret_cast<const float4*>(piece + 128 * gi + 16 * v);
    } else if constexpr (F == kF16 || F == kBF16) {
        const uint2 h = *reinterpret_cast<const uint2*>(piece + 64 * gi + 8 * v);
        if constexpr (F == kF16)
            return {half_to_float(h.x & 0xFFFFu), half_to_float(h.x >> 16), half_to_float(h.y & 0xFFFFu),
                    half_to_float(h.y >> 16)};
        else
            return {bf16_low(h.x), bf16_high(h.x), bf16_low(h.y), bf16_high(h.y)};
    } else if constexpr (F == kQ8_0) {
        const uint32_t c = *reinterpret_cast<const uint32_t*>(piece + 32 * gi + 4 * v);
        const float d = half_to_float(*reinterpret_cast<const uint16_t*>(piece + 32 * n + 2 * gi));
        auto w = [&](int b) { return static_cast<float>(static_cast<int32_t>(static_cast<int8_t>(c >> (8 * b)))) * d; };
        return {w(0), w(1), w(2), w(3)};
    } else if constexpr (F == kQ4_0 || F == kQ4_1) {
        // weights 4v .. 4v + 3: dword v % 4 of the codes, nibble v / 4
        const uint32_t c = *reinterpret_cast<const uint32_t*>(piece + 16 * gi + 4 * (v & 3u)) >> (4 * (v >> 2));
        if constexpr (F == kQ4_0) {
            // (q - 8) d, the product exact — and a zero weight's sign d's, as
            // the file-order decode gives it (an fma would give +0)
            const float d = half_to_float(*reinterpret_cast<const uint16_t*>(piece + 16 * n + 2 * gi));
            auto w = [&](int b) { return static_cast<float>(static_cast<int32_t>((c >> (8 * b)) & 0xFu) - 8) * d; };
            return {w(0), w(1), w(2), w(3)};
        } else {
            // fma(q, d, m): q d exact, one rounding, the zero signs of q d + m
            const uint32_t dm = *reinterpret_cast<const uint32_t*>(piece + 16 * n + 4 * gi);
            const float d = half_to_float(dm & 0xFFFFu), m = half_to_float(dm >> 16);
            auto w = [&](int b) { return __builtin_fmaf(static_cast<float>((c >> (8 * b)) & 0xFu), d, m); };
            return {w(0), w(1), w(2), w(3)};
        }
    } else {
        // Q6_K: low nibbles in lo dword v % 4, nibble v / 4; high pairs in hi
        // dword v % 2, bits 2 (v / 2) of each byte; scale v < 4 ? first : second.
        const uint32_t lo = *reinterpret_cast<const uint32_t*>(piece + 16 * gi + 4 * (v & 3u)) >> (4 * (v >> 2));
        const uint32_t hi = *reinterpret_cast<const uint32_t*>(piece + 128 * n + 8 * gi + 4 * (v & 1u)) >> (2 * (v >> 1));
        const int8_t sc = static_cast<int8_t>(*(piece + 192 * n + 2 * gi + (v >> 2)));
        const float d = half_to_float(*reinterpret_cast<const uint16_t*>(piece + 208 * n + 2 * (gi / 8)));
        const float scale = d * static_cast<float>(sc);
        auto w = [&](int b) {  // (d sc)(q - 32), exact, its zeros signed as the file-order decode's
            const int32_t q = static_cast<int32_t>(((lo >> (8 * b)) & 0xFu) | (((hi >> (8 * b)) & 3u) << 4));
            return scale * static_cast<float>(q - 32);
        };
        return {w(0), w(1), w(2), w(3)};
    }
}

template <uint32_t F>
__global__ __launch_bounds__(256) void gather_rows(Gather g) {
    const uint64_t id = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
    const uint64_t group_of_step = id >> 3;
    const uint32_t v = static_cast<uint32_t>(id & 7u);
    const uint64_t row = group_of_step / g.groups;
    if (row >= g.tokens) return;
    const uint32_t group = static_cast<uint32_t>(group_of_step % g.groups);
    uint32_t token;
    if (g.fed) {
        token = g.fed[0];
    } else {
        token = g.ids[row];
        if (g.media && token == g.media_token) return;
    }
    if (token < g.first_row || token - g.first_row >= g.row_count) return;
    const uint64_t gi = static_cast<uint64_t>(token - g.first_row) * g.groups + group;
    float4 w = unpack4<F>(g.piece, g.blocks, gi, v);
    w.x *= g.scale;
    w.y *= g.scale;
    w.z *= g.scale;
    w.w *= g.scale;
    reinterpret_cast<float4*>(g.hidden)[group_of_step * 8 + v] = w;
}

__global__ __launch_bounds__(256) void gather_positions(Gather g) {
    const uint64_t id = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
    const uint64_t group_of_step = id >> 3;
    const uint32_t v = static_cast<uint32_t>(id & 7u);
    const uint64_t row = group_of_step / g.groups;
    if (row >= g.tokens) return;
    const uint32_t group = static_cast<uint32_t>(group_of_step % g.groups);
    const uint64_t x = row % g.grid_columns, y = row / g.grid_columns;
    const float4 across = unpack4<kF32>(g.piece, g.blocks, x * g.groups + group, v);
    const float4 down = unpack4<kF32>(g.piece, g.blocks, (g.positions + y) * g.groups + group, v);
    reinterpret_cast<float4*>(g.hidden)[group_of_step * 8 + v] =
        make_float4(across.x + down.x, across.y + down.y, across.z + down.z, across.w + down.w);
}

static dim3 grid_of(const Gather& g) {
    const uint64_t lanes = static_cast<uint64_t>(g.tokens) * g.groups * 8;
    return dim3(static_cast<uint32_t>((lanes + 255) / 256));
}

hipError_t launch_gather(const Gather& g, uint32_t format, hipStream_t stream) {
    const dim3 grid = grid_of(g);
    switch (format) {
        case kF32: hipLaunchKernelGGL(gather_rows<kF32>, grid, dim3(256), 0, stream, g); break;
        case kF16: hipLaunchKernelGGL(gather_rows<kF16>, grid, dim3(256), 0, stream, g); break;
        case kBF16: hipLaunchKernelGGL(gather_rows<kBF16>, grid, dim3(256), 0, stream, g); break;
        case kQ4_0: hipLaunchKernelGGL(gather_rows<kQ4_0>, grid, dim3(256), 0, stream, g); break;
        case kQ4_1: hipLaunchKernelGGL(gather_rows<kQ4_1>, grid, dim3(256), 0, stream, g); break;
        case kQ8_0: hipLaunchKernelGGL(gather_rows<kQ8_0>, grid, dim3(256), 0, stream, g); break;
        case kQ6_K: hipLaunchKernelGGL(gather_rows<kQ6_K>, grid, dim3(256), 0, stream, g); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_gather_positions(const Gather& g, hipStream_t stream) {
    hipLaunchKernelGGL(gather_positions, grid_of(g), dim3(256), 0, stream, g);
    return hipGetLastError();
}

}  // namespace chm
