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

// The member holding product row p, and p's row within its piece.
__device__ __forceinline__ int locate(const Product& a, uint32_t p, uint32_t* row) {
    int m = 0;
    if (a.members > 1 && p >= a.m[0].first + a.m[0].rows) m = (a.members > 2 && p >= a.m[1].first + a.m[1].rows) ? 2 : 1;
    *row = a.m[m].row_offset + (p - a.m[m].first);
    return m;
}

}  // namespace chm
