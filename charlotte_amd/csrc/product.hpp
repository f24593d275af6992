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
    uint32_t out_width;    // floats a token's output row
    uint32_t pad;
    float* out;            // its output buffer
};

struct Product {
    Member m[3];
    const float* x;        // tokens rows of K floats
    uint32_t members;
    uint32_t rows;         // product rows: the members' together
    uint32_t groups;       // G = K / 32
    uint32_t epilogue;
    uint32_t activation;
    uint32_t last_token;   // nonzero: one output row, from the step's last token
    uint32_t tokens;       // rows of x in the step
    uint32_t gate_stride;  // GATED_BY_INPUT
    uint32_t gate_column;
    uint32_t activated;
    const float* gate_input;
    const float* clip;     // device: in_min, in_max, out_min, out_max, or null
    const float* bias;     // device, or null
};

// Where product row p's weights lie: its member's piece and p's row within
// it. Members are compared with constant indices only, so their fields stay
// in scalar registers (an index into the kernel argument would reload them
// from memory on every use).
struct Piece {
    const uint8_t* piece;
    uint64_t blocks;
    uint32_t row;
};

__device__ __forceinline__ Piece piece_of(const Product& a, uint32_t p) {
    Piece w{a.m[0].piece, a.m[0].blocks, a.m[0].row_offset + (p - a.m[0].first)};
    if (a.members > 1 && p >= a.m[1].first) w = {a.m[1].piece, a.m[1].blocks, a.m[1].row_offset + (p - a.m[1].first)};
    if (a.members > 2 && p >= a.m[2].first) w = {a.m[2].piece, a.m[2].blocks, a.m[2].row_offset + (p - a.m[2].first)};
    return w;
}

// Where product row p's output of `token` goes: QKV writes each member's own
// buffer, `rows` wide; the others write out_row + their row, out_width wide.
__device__ __forceinline__ float* output_of(const Product& a, uint32_t p, uint32_t token) {
    float* out = a.m[0].out;
    uint32_t first = a.m[0].first, at = a.m[0].out_row, width = a.m[0].out_width, rows = a.m[0].rows;
    if (a.members > 1 && p >= a.m[1].first) {
        out = a.m[1].out, first = a.m[1].first, at = a.m[1].out_row, width = a.m[1].out_width, rows = a.m[1].rows;
    }
    if (a.members > 2 && p >= a.m[2].first) {
        out = a.m[2].out, first = a.m[2].first, at = a.m[2].out_row, width = a.m[2].out_width, rows = a.m[2].rows;
    }
    if (a.epilogue == kQKV) return out + static_cast<uint64_t>(token) * rows + (p - first);
    return out + static_cast<uint64_t>(token) * width + at + (p - first);
}

}  // namespace chm
