// GGUF v3 index reading for loading weights from real model files: the
// header, the metadata (walked and validated, with general.alignment
// honoured), and every tensor's name, format, shape and absolute byte range,
// validated against the file. The role of the reference's gguf::read_index
// (src/core/gguf/reader.cpp); the error vocabulary is its ReadError
// (src/core/gguf/types.h:112-141), numbered alike, so a caller maps one onto
// the other. Never reads outside the bytes it is given; every offset,
// length and shape product is checked before use.
#include "gguf.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstring>
#include <limits>
#include <string_view>

namespace chm {
namespace {

// GGUF's format table (src/core/gguf/types.h:69-101, ggml's GGML_QUANT_SIZES):
// a format stores `elements` consecutive values of a row in `bytes` bytes.
struct Layout {
    uint32_t type, elements, bytes;
};
constexpr Layout kLayouts[] = {
    {0, 1, 4},      {1, 1, 2},      {2, 32, 18},    {3, 32, 20},    {6, 32, 22},    {7, 32, 24},
    {8, 32, 34},    {9, 32, 36},    {10, 256, 84},  {11, 256, 110}, {12, 256, 144}, {13, 256, 176},
    {14, 256, 210}, {15, 256, 292}, {16, 256, 66},  {17, 256, 74},  {18, 256, 98},  {19, 256, 50},
    {20, 32, 18},   {21, 256, 110}, {22, 256, 82},  {23, 256, 136}, {24, 1, 1},     {25, 1, 2},
    {26, 1, 4},     {27, 1, 8},     {28, 1, 8},     {29, 256, 56},  {30, 1, 2},     {34, 256, 54},
    {35, 256, 66},  {39, 32, 17},   {40, 64, 36},   {41, 128, 18},  {42, 64, 18},
};

const Layout* layout_of(uint32_t type) {
    for (const Layout& l : kLayouts)
        if (l.type == type) return &l;
    return nullptr;
}

// The reader's own bounds against allocation by a hostile file
// (src/core/gguf/types.h:16-25): not format limits.
constexpr uint64_t kMaxTensors = 1u << 20, kMaxKeys = 1u << 20, kMaxString = 1u << 20, kMaxArray = 1u << 24;
constexpr uint64_t kMaxName = 64;
constexpr uint32_t kMaxDims = 4;
constexpr uint64_t kDefaultAlignment = 32;

enum ValueType : uint32_t { kU8, kI8, kU16, kI16, kU32, kI32, kF32, kBool, kString, kArray, kU64, kI64, kF64 };

uint64_t scalar_bytes(uint32_t t) {
    switch (t) {
        case kU8: case kI8: case kBool: return 1;
        case kU16: case kI16: return 2;
        case kU32: case kI32: case kF32: return 4;
        case kU64: case kI64: case kF64: return 8;
        default: return 0;
    }
}

bool add_ok(uint64_t a, uint64_t b, uint64_t& out) {
    if (a > std::numeric_limits<uint64_t>::max() - b) return false;
    out = a + b;
    return true;
}
bool mul_ok(uint64_t a, uint64_t b, uint64_t& out) {
    if (a != 0 && b > std::numeric_limits<uint64_t>::max() / a) return false;
    out = a * b;
    return true;
}
// [at, at + n) inside [0, size), the addition itself never taken.
bool inside(uint64_t at, uint64_t n, uint64_t size) { return at <= size && n <= size - at; }

// A cursor over the file's bytes; each take advances only on success.
class Cursor {
public:
    Cursor(const uint8_t* bytes, uint64_t size) : p_(bytes), size_(size) {}
    uint64_t at() const { return at_; }
    GgufError uint(int n, uint64_t& out) {
        if (!inside(at_, static_cast<uint64_t>(n), size_)) return GgufError::kShortRead;
        out = 0;
        for (int i = n - 1; i >= 0; --i) out = (out << 8) | p_[at_ + i];  // little-endian
        at_ += n;
        return GgufError::kOk;
    }
    GgufError skip(uint64_t n) {
        if (!inside(at_, n, size_)) return GgufError::kShortRead;
        at_ += n;
        return GgufError::kOk;
    }
    GgufError string(std::string& out) {
        uint64_t n = 0;
        if (GgufError e = uint(8, n); e != GgufError::kOk) return e;
        if (n > kMaxString) return GgufError::kStringTooLong;
        if (!inside(at_, n, size_)) return GgufError::kShortRead;
        out.assign(reinterpret_cast<const char*>(p_ + at_), n);
        at_ += n;
        return GgufError::kOk;
    }
    GgufError skip_string() {
        uint64_t n = 0;
        if (GgufError e = uint(8, n); e != GgufError::kOk) return e;
        if (n > kMaxString) return GgufError::kStringTooLong;
        return skip(n);
    }

private:
    const uint8_t* p_;
    uint64_t size_;
    uint64_t at_ = 0;
};

bool sorted_has_duplicate(std::vector<std::string_view> names) {
    std::sort(names.begin(), names.end());
    return std::adjacent_find(names.begin(), names.end()) != names.end();
}

// One metadata value: scalars read (general.alignment is kept), strings and
// arrays walked; arrays of arrays refused.
GgufError value(Cursor& c, uint32_t type, uint64_t& scalar) {
    if (type > kF64) return GgufError::kUnknownValueType;
    if (type == kString) return c.skip_string();
    if (type == kArray) {
        uint64_t element = 0, count = 0;
        if (GgufError e = c.uint(4, element); e != GgufError::kOk) return e;
        if (element > kF64) return GgufError::kUnknownValueType;
        if (element == kArray) return GgufError::kNestedArray;
        if (GgufError e = c.uint(8, count); e != GgufError::kOk) return e;
        if (count > kMaxArray) return GgufError::kArrayTooLong;
        if (element == kString) {
            for (uint64_t i = 0; i < count; ++i)
                if (GgufError e = c.skip_string(); e != GgufError::kOk) return e;
            return GgufError::kOk;
        }
        uint64_t n = 0;
        if (!mul_ok(count, scalar_bytes(element), n)) return GgufError::kOffsetOverflow;
        return c.skip(n);
    }
    return c.uint(static_cast<int>(scalar_bytes(type)), scalar);
}

}  // namespace

const char* gguf_error_string(GgufError e) {
    switch (e) {
        case GgufError::kOk: return "ok";
        case GgufError::kNeedMoreBytes: return "more of the file is needed to read its index";
        case GgufError::kShortRead: return "the file ends before this field";
        case GgufError::kBadMagic: return "not a GGUF file: magic mismatch";
        case GgufError::kUnsupportedVersion: return "unsupported GGUF version (3 is read)";
        case GgufError::kCountTooLarge: return "a declared count exceeds the reader's bound";
        case GgufError::kStringTooLong: return "a string's length exceeds the reader's bound";
        case GgufError::kArrayTooLong: return "an array's length exceeds the reader's bound";
        case GgufError::kUnknownValueType: return "unknown metadata value type";
        case GgufError::kUnknownTensorType: return "a tensor format GGUF does not define";
        case GgufError::kRowNotWholeBlocks: return "a tensor row is not a whole number of its format's blocks";
        case GgufError::kTooManyDimensions: return "a tensor declares more than 4 dimensions";
        case GgufError::kNegativeDimension: return "a tensor declares a negative dimension";
        case GgufError::kElementCountOverflow: return "a tensor's element count overflows";
        case GgufError::kOffsetOverflow: return "an offset plus a length overflows";
        case GgufError::kTensorDataOutOfBounds: return "tensor data lies outside the file";
        case GgufError::kDuplicateTensorName: return "two tensors share a name";
        case GgufError::kTensorNameTooLong: return "a tensor name is longer than 64 bytes";
        case GgufError::kMisalignedTensorData: return "tensor data is not aligned as the file declares";
        case GgufError::kOverlappingTensorData: return "two tensors claim the same bytes";
        case GgufError::kBadAlignment: return "general.alignment is not a power-of-two uint32";
        case GgufError::kEmptyKey: return "a metadata key is empty";
        case GgufError::kDuplicateMetadataKey: return "two metadata entries share a key";
        case GgufError::kNestedArray: return "arrays of arrays are not read";
        case GgufError::kWrongElementType: return "an array holds another element type";
    }
    return "unrecognised error";
}

GgufError GgufIndex::read(const uint8_t* bytes, uint64_t size) {
    tensors.clear();
    Cursor c(bytes, size);
    uint64_t magic = 0, version = 0, tensor_count = 0, key_count = 0;
    if (GgufError e = c.uint(4, magic); e != GgufError::kOk) return e;
    if (magic != 0x46554747u) return GgufError::kBadMagic;  // "GGUF"
    if (GgufError e = c.uint(4, version); e != GgufError::kOk) return e;
    if (version != 3) return GgufError::kUnsupportedVersion;
    if (GgufError e = c.uint(8, tensor_count); e != GgufError::kOk) return e;
    if (GgufError e = c.uint(8, key_count); e != GgufError::kOk) return e;
    if (tensor_count > kMaxTensors || key_count > kMaxKeys) return GgufError::kCountTooLarge;

    // Metadata: keys non-empty and distinct; general.alignment, when
    // declared, a power-of-two uint32.
    std::vector<std::string> keys;
    keys.reserve(key_count);
    alignment = kDefaultAlignment;
    for (uint64_t i = 0; i < key_count; ++i) {
        std::string key;
        if (GgufError e = c.string(key); e != GgufError::kOk) return e;
        if (key.empty()) return GgufError::kEmptyKey;
        uint64_t type = 0, scalar = 0;
        if (GgufError e = c.uint(4, type); e != GgufError::kOk) return e;
        if (GgufError e = value(c, static_cast<uint32_t>(type), scalar); e != GgufError::kOk) return e;
        if (key == "general.alignment") {
            if (type != kU32 || scalar == 0 || (scalar & (scalar - 1)) != 0) return GgufError::kBadAlignment;
            alignment = scalar;
        }
        keys.push_back(std::move(key));
    }
    {
        std::vector<std::string_view> views(keys.begin(), keys.end());
        if (sorted_has_duplicate(std::move(views))) return GgufError::kDuplicateMetadataKey;
    }

    // Tensors: a name of at most 64 bytes, at most 4 non-negative dimensions
    // whose product fits, a defined format whose blocks tile a row, and an
    // offset relative to the data region.
    std::vector<GgufTensor> found;
    found.reserve(tensor_count);
    for (uint64_t i = 0; i < tensor_count; ++i) {
        GgufTensor t{};
        if (GgufError e = c.string(t.name); e != GgufError::kOk) return e;
        if (t.name.size() > kMaxName) return GgufError::kTensorNameTooLong;
        uint64_t dims = 0;
        if (GgufError e = c.uint(4, dims); e != GgufError::kOk) return e;
        if (dims > kMaxDims) return GgufError::kTooManyDimensions;
        t.dimension_count = static_cast<uint32_t>(dims);
        t.elements = 1;
        for (uint32_t d = 0; d < kMaxDims; ++d) t.dimensions[d] = 1;
        for (uint32_t d = 0; d < t.dimension_count; ++d) {
            uint64_t extent = 0;
            if (GgufError e = c.uint(8, extent); e != GgufError::kOk) return e;
            if (extent >> 63) return GgufError::kNegativeDimension;  // an int64 on disk
            t.dimensions[d] = extent;
            if (!mul_ok(t.elements, extent, t.elements)) return GgufError::kElementCountOverflow;
        }
        uint64_t type = 0;
        if (GgufError e = c.uint(4, type); e != GgufError::kOk) return e;
        const Layout* layout = layout_of(static_cast<uint32_t>(type));
        if (!layout) return GgufError::kUnknownTensorType;
        t.type = static_cast<uint32_t>(type);
        if (t.dimensions[0] % layout->elements != 0) return GgufError::kRowNotWholeBlocks;
        if (GgufError e = c.uint(8, t.offset); e != GgufError::kOk) return e;
        if (!mul_ok(t.elements / layout->elements, layout->bytes, t.bytes)) return GgufError::kOffsetOverflow;
        found.push_back(std::move(t));
    }
    {
        std::vector<std::string_view> views;
        views.reserve(found.size());
        for (const GgufTensor& t : found) views.push_back(t.name);
        if (sorted_has_duplicate(std::move(views))) return GgufError::kDuplicateTensorName;
    }

    // The data region starts at the next alignment boundary after the index;
    // each offset is a multiple of the alignment, made absolute, inside the
    // file, and no two ranges meet.
    uint64_t data = 0;
    if (!add_ok(c.at(), (alignment - c.at() % alignment) % alignment, data)) return GgufError::kOffsetOverflow;
    if (data > size) return GgufError::kTensorDataOutOfBounds;
    for (GgufTensor& t : found) {
        if (t.offset % alignment != 0) return GgufError::kMisalignedTensorData;
        uint64_t absolute = 0;
        if (!add_ok(data, t.offset, absolute)) return GgufError::kOffsetOverflow;
        if (!inside(absolute, t.bytes, size)) return GgufError::kTensorDataOutOfBounds;
        t.offset = absolute;
    }
    {
        std::vector<std::pair<uint64_t, uint64_t>> ranges;
        ranges.reserve(found.size());
        for (const GgufTensor& t : found) ranges.emplace_back(t.offset, t.bytes);
        std::sort(ranges.begin(), ranges.end());
        for (size_t i = 1; i < ranges.size(); ++i)
            if (ranges[i].first < ranges[i - 1].first + ranges[i - 1].second) return GgufError::kOverlappingTensorData;
    }
    tensors = std::move(found);
    this->bytes = bytes;
    this->size = size;
    return GgufError::kOk;
}

int64_t GgufIndex::find(const char* name) const {
    for (size_t i = 0; i < tensors.size(); ++i)
        if (tensors[i].name == name) return static_cast<int64_t>(i);
    return -1;
}

GgufFile::~GgufFile() {
    if (mapped) munmap(const_cast<uint8_t*>(index.bytes), mapped);
}

GgufError GgufFile::open(const char* path, int* os_error) {
    *os_error = 0;
    const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) {
        *os_error = errno;
        return GgufError::kShortRead;
    }
    struct stat st {};
    if (fstat(fd, &st) != 0) {
        *os_error = errno;
        ::close(fd);
        return GgufError::kShortRead;
    }
    const uint64_t size = static_cast<uint64_t>(st.st_size);
    const uint8_t* p = nullptr;
    if (size > 0) {
        void* m = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
        if (m == MAP_FAILED) {
            *os_error = errno;
            ::close(fd);
            return GgufError::kShortRead;
        }
        p = static_cast<const uint8_t*>(m);
        mapped = size;
    }
    ::close(fd);
    static const uint8_t kEmpty = 0;
    const GgufError e = index.read(p ? p : &kEmpty, size);
    if (e != GgufError::kOk && mapped) {
        munmap(const_cast<uint8_t*>(p), mapped);
        mapped = 0;
    }
    if (e != GgufError::kOk) return e;
    index.bytes = p ? p : &kEmpty;
    return e;
}

}  // namespace chm
