// GGUF v3 index reading (gguf.cpp), for the C ABI's charlotte_hip_matmul_gguf_*.
#pragma once

#include <stdint.h>

#include <string>
#include <vector>

namespace chm {

// The reference's gguf::ReadError (src/core/gguf/types.h:112-141), numbered
// alike.
enum class GgufError : uint32_t {
    kOk = 0,
    kNeedMoreBytes,
    kShortRead,
    kBadMagic,
    kUnsupportedVersion,
    kCountTooLarge,
    kStringTooLong,
    kArrayTooLong,
    kUnknownValueType,
    kUnknownTensorType,
    kRowNotWholeBlocks,
    kTooManyDimensions,
    kNegativeDimension,
    kElementCountOverflow,
    kOffsetOverflow,
    kTensorDataOutOfBounds,
    kDuplicateTensorName,
    kTensorNameTooLong,
    kMisalignedTensorData,
    kOverlappingTensorData,
    kBadAlignment,
    kEmptyKey,
    kDuplicateMetadataKey,
    kNestedArray,
    kWrongElementType,
};

const char* gguf_error_string(GgufError e);

struct GgufTensor {
    std::string name;
    uint32_t type = 0;
    uint32_t dimension_count = 0;
    uint64_t dimensions[4] = {1, 1, 1, 1};
    uint64_t elements = 0;
    uint64_t offset = 0;  // absolute, once read
    uint64_t bytes = 0;
};

// A file's tensor index over bytes the caller keeps alive.
struct GgufIndex {
    std::vector<GgufTensor> tensors;
    uint64_t alignment = 32;
    const uint8_t* bytes = nullptr;
    uint64_t size = 0;
    // Reads the index of `size` bytes; leaves `tensors` empty unless Ok.
    GgufError read(const uint8_t* bytes, uint64_t size);
    int64_t find(const char* name) const;
};

// A file mapped read-only and its index.
struct GgufFile {
    GgufIndex index;
    uint64_t mapped = 0;
    GgufError open(const char* path, int* os_error);
    ~GgufFile();
};

}  // namespace chm
