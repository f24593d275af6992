// A product as its kernels receive it: up to three members, each a piece
// and a run of its rows, and where each member's outputs go. Built on the
// host from a charlotte_hip_matmul_desc (capi.cpp), passed by value.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "formats.hpp"

namespace chm {

enum Epilogue : uint32_t { kWrite = 0, kQKV = 1, kGated = 2, kGatedByInput = 3 };

struct Member {
    const uint8_t* piece;  // the piece's first stream byte
    uint64_t blocks;       // blocks in the piece (Q4_0) or super-blocks (Q6_K)
    uint32_t row_offset;   // first row read within the piece
    uint32_t rows;         // product rows this member supplies
    uint32_t first;        // its first product row
    uint32_t out_row;      // output index of its first row (WRITE, GATED_BY_INPUT)
    uint32_t out_width;    // floats a token's output row (GATED: member 0's)
    uint32_t pad;
    float* out;            // its output buffer
};

struct Product {
    Member m[3];
    const float* x;        // tokens rows of K floats
    uint32_t members;
    uint32_t rows;         // product rows: the members' together (GATED: interleaved)
    uint32_t groups;       // G = K / 32
    uint32_t epilogue;
    uint32_t activation;
    uint32_t last_token;   // nonzero: one output row, from the step's last token
    uint32_t tokens;       // rows of x in the step
    uint32_t gate_stride;  // GATED_BY_INPUT
    uint32_t gate_column;
    uint32_t activated;
    const float* gate_input;
    // device: the four bounds in_min, in_max, out_min, out_max, each its own
    // word wherever the caller keeps it, or all four null
    const float* clip[4];
    const float* bias;     // device, or null
};

__host__ __device__ __forceinline__ bool clipped(const Product& a) { return a.clip[0] != nullptr; }

// Where product row p's weights lie: its member's piece and p's row within
// it. Members are compared with constant indices only, so their fields stay
// in scalar registers (an index into the kernel argument would reload them
// from memory on every use). A gated product's rows interleave its members:
// row 2r is the gate's row r, row 2r + 1 the up's, so one lane or one
// micro-tile holds both totals an output needs.
struct Piece {
    const uint8_t* piece;
    uint64_t blocks;
    uint32_t row;
};

__device__ __forceinline__ Piece piece_of(const Product& a, uint32_t p) {
    if (a.epilogue == kGated) {
        const bool up = p & 1u;
        return {up ? a.m[1].piece : a.m[0].piece, up ? a.m[1].blocks : a.m[0].blocks,
                (up ? a.m[1].row_offset : a.m[0].row_offset) + (p >> 1)};
    }
    Piece w{a.m[0].piece, a.m[0].blocks, a.m[0].row_offset + (p - a.m[0].first)};
    if (a.members > 1 && p >= a.m[1].first) w = {a.m[1].piece, a.m[1].blocks, a.m[1].row_offset + (p - a.m[1].first)};
    if (a.members > 2 && p >= a.m[2].first) w = {a.m[2].piece, a.m[2].blocks, a.m[2].row_offset + (p - a.m[2].first)};
    return w;
}

// Where product row p's output of `token` goes, and its index o in the
// token's output row: QKV writes each member's own buffer, `rows` wide; Write
// and GatedByInput write out_row + the member's row, out_width wide.
struct Place {
    float* at;
    uint32_t o;
};

__device__ __forceinline__ Place place_of(const Product& a, uint32_t p, uint32_t token) {
    float* out = a.m[0].out;
    uint32_t first = a.m[0].first, at = a.m[0].out_row, width = a.m[0].out_width, rows = a.m[0].rows;
    if (a.members > 1 && p >= a.m[1].first) {
        out = a.m[1].out, first = a.m[1].first, at = a.m[1].out_row, width = a.m[1].out_width, rows = a.m[1].rows;
    }
    if (a.members > 2 && p >= a.m[2].first) {
        out = a.m[2].out, first = a.m[2].first, at = a.m[2].out_row, width = a.m[2].out_width, rows = a.m[2].rows;
    }
    if (a.epilogue == kQKV) return {out + static_cast<uint64_t>(token) * rows + (p - first), p - first};
    const uint32_t o = at + (p - first);
    return {out + static_cast<uint64_t>(token) * width + o, o};
}

// e^x for x <= 0 as explicit arithmetic (matmul.wgsl:163-182): x = k ln 2 + r
// with ln 2 in two parts (Cody and Waite), e^r by its Taylor series to r^6 in
// Horner's form, 2^k by ldexp. Every multiply-add an fma, so the value is the
// same on every path that evaluates it.
__device__ __forceinline__ float exp_nonpositive(float x) {
    const float xc = fmaxf(x, -100.0f);
    const float k = floorf(__builtin_fmaf(xc, 1.4426950408889634f, 0.5f));
    float r = __builtin_fmaf(k, -0.693145751953125f, xc);
    r = __builtin_fmaf(k, -1.4286068203094172e-06f, r);
    float q = 1.0f / 720.0f;
    q = __builtin_fmaf(q, r, 1.0f / 120.0f);
    q = __builtin_fmaf(q, r, 1.0f / 24.0f);
    q = __builtin_fmaf(q, r, 1.0f / 6.0f);
    q = __builtin_fmaf(q, r, 0.5f);
    q = __builtin_fmaf(q, r, 1.0f);
    q = __builtin_fmaf(q, r, 1.0f);
    return ldexpf(q, static_cast<int>(k));
}

// matmul.wgsl:184-205: 0 SiLU, 1 GELU in its tanh form, 2 the sigmoid, each
// from e^x of a non-positive x; each quotient a correctly rounded division.
__device__ __forceinline__ float activate(uint32_t activation, float g) {
    if (activation != 1u) {
        const float e = exp_nonpositive(-fabsf(g));
        const float r = 1.0f / (1.0f + e);
        const float s = g >= 0.0f ? r : e * r;
        return activation == 0u ? g * s : s;
    }
    const float z = 0.7978845608028654f * __builtin_fmaf(0.044715f * g * g, g, g);
    const float e = exp_nonpositive(-2.0f * fabsf(z));
    const float sign = z > 0.0f ? 1.0f : (z < 0.0f ? -1.0f : 0.0f);
    const float t = sign * ((1.0f - e) * (1.0f / (1.0f + e)));
    const float half_g = 0.5f * g;
    return __builtin_fmaf(half_g, t, half_g);
}

// Whether a product's epilogue is a plain store (no FULL kernel needed).
inline bool plain_epilogue(const Product& a) {
    return a.epilogue == kQKV || (a.epilogue == kWrite && !clipped(a) && !a.bias && !a.activated);
}

// WGSL's clamp(e, low, high): min(max(e, low), high). Exact.
__device__ __forceinline__ float clamp_to(float v, float lo, float hi) { return fminf(fmaxf(v, lo), hi); }

// The input as a product reads it: clamped to its bounds where clipped
// (matmul.wgsl:117-124). Applied as x is staged.
__device__ __forceinline__ float4 clamp_input(const Product& a, float4 v) {
    if (!clipped(a)) return v;
    const float lo = *a.clip[0], hi = *a.clip[1];
    return {clamp_to(v.x, lo, hi), clamp_to(v.y, lo, hi), clamp_to(v.z, lo, hi), clamp_to(v.w, lo, hi)};
}

// Product row p's output of output row `token` from its total, as the
// epilogue asks (matmul.wgsl:272-351): Write clamps, adds its bias, then
// activates, as its options ask; QKV writes the total; GatedByInput writes
// activate(total) u[in_token stride + column + o]; a gated product's even row
// writes activate(clamp(gate)) clamp(up), `partner` the up total (row p + 1).
// `in_token` is the input row the output came from (the head's last token).
// Kernels are built twice: FULL for any epilogue, and without it for the
// plain ones — QKV, and a Write with no options — which store the total
// and keep the registers the rest would hold.
//
// THROUGH stores at system scope (a relaxed atomic store: global_store_dword
// sc0 sc1, which the compiler sees and counts), written through the L2: a
// small decode's few outputs then leave nothing dirty for the end of the
// kernel to write back (Qwen3 0.6B's decode step 486 -> 479 us); large
// outputs (the prefill tiles) store the ordinary way, at less than half the
// rate through.
template <bool THROUGH>
__device__ __forceinline__ void put(float v, float* at) {
    if constexpr (THROUGH)
        __hip_atomic_store(at, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    else
        *at = v;
}

template <bool FULL, bool THROUGH = false>
__device__ __forceinline__ void emit(const Product& a, uint32_t p, uint32_t token, uint32_t in_token, float total,
                                     float partner) {
    if constexpr (!FULL) {
        put<THROUGH>(total, place_of(a, p, token).at);
        return;
    }
    if (a.epilogue == kGated) {
        if (p & 1u) return;
        float g = total, u = partner;
        if (clipped(a)) {
            const float lo = *a.clip[2], hi = *a.clip[3];
            g = clamp_to(g, lo, hi), u = clamp_to(u, lo, hi);
        }
        put<THROUGH>(activate(a.activation, g) * u, &a.m[0].out[static_cast<uint64_t>(token) * a.m[0].out_width + (p >> 1)]);
        return;
    }
    const Place w = place_of(a, p, token);
    float y = total;
    if (a.epilogue == kGatedByInput) {
        y = activate(a.activation, y) *
            a.gate_input[static_cast<uint64_t>(in_token) * a.gate_stride + a.gate_column + w.o];
    } else if (a.epilogue == kWrite) {
        if (clipped(a)) y = clamp_to(y, *a.clip[2], *a.clip[3]);
        if (a.bias) y = y + a.bias[w.o];
        if (a.activated) y = activate(a.activation, y);
    }
    put<THROUGH>(y, w.at);
}

}  // namespace chm
