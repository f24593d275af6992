// The embedding gather as its kernels receive it (gather.hip), built on the
// host from a charlotte_hip_matmul_gather_desc (capi.cpp).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "formats.hpp"

namespace chm {

// gather.wgsl's Gather constants (gather.wgsl:6-13) and its bindings.
struct Gather {
    const uint8_t* piece;    // the table's piece
    uint64_t blocks;         // blocks in the piece
    const uint32_t* ids;     // the step's identifiers
    const uint32_t* fed;     // a fed step's draw record, or null
    float* hidden;           // tokens rows of groups * 32 floats
    uint32_t tokens;
    uint32_t groups;         // 32-weight groups a row
    uint32_t first_row;      // the piece's first vocabulary row
    uint32_t row_count;      // rows in the piece
    uint32_t media;          // nonzero: rows whose identifier is media_token are skipped
    uint32_t media_token;
    float scale;
    uint32_t positions;      // the position form: rows of each axis table
    uint32_t grid_columns;   // the position form: the patch grid's columns
};

hipError_t launch_gather(const Gather& g, uint32_t format, hipStream_t stream);
hipError_t launch_gather_positions(const Gather& g, hipStream_t stream);

}  // namespace chm
