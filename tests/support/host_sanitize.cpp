// Host-side code of the library (the GGUF index reader, gguf.cpp, and the
// device layout, layout.cpp) driven under AddressSanitizer and UBSan by
// tests/test_host_sanitized.py: every fixture file read whole, every prefix
// of the small ones, seeded byte mutations of each one's first 4 KB, then the
// layout and Q6_K repack of blocks of every format. Test infrastructure only.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <iterator>
#include <string>
#include <vector>

#include "gguf.hpp"
#include "layout.hpp"

static std::vector<uint8_t> slurp(const char* path) {
    std::ifstream f(path, std::ios::binary);
    return std::vector<uint8_t>(std::istreambuf_iterator<char>(f), std::istreambuf_iterator<char>());
}

int main(int argc, char** argv) {
    uint64_t reads = 0, accepted = 0;
    uint32_t state = 0x2545F491u;
    auto next = [&]() { return state = state * 1664525u + 1013904223u; };
    for (int i = 1; i < argc; ++i) {
        const std::vector<uint8_t> whole = slurp(argv[i]);
        chm::GgufFile file;
        int os_error = 0;
        if (file.open(argv[i], &os_error) == chm::GgufError::kOk) {
            ++accepted;
            for (const auto& t : file.index.tensors) (void)file.index.find(t.name.c_str());
        }
        // every prefix of a small file; of a large one, the first 4 KB
        const uint64_t cut_to = whole.size() <= 65536 ? whole.size() : 4096;
        for (uint64_t cut = 0; cut <= cut_to; ++cut) {
            std::vector<uint8_t> part(whole.begin(), whole.begin() + static_cast<long>(cut));
            chm::GgufIndex index;
            if (index.read(part.data(), part.size()) == chm::GgufError::kOk) ++accepted;
            ++reads;
        }
        // mutations: one to four bytes of the first 4 KB changed, then put back
        std::vector<uint8_t> bytes = whole;
        for (int m = 0; m < 20000 && !bytes.empty(); ++m) {
            const uint64_t span = bytes.size() < 4096 ? bytes.size() : 4096;
            const int count = 1 + static_cast<int>(next() % 4);
            uint64_t at[4];
            for (int k = 0; k < count; ++k) {
                at[k] = next() % span;
                bytes[at[k]] = static_cast<uint8_t>(next() >> 24);
            }
            chm::GgufIndex index;
            if (index.read(bytes.data(), bytes.size()) == chm::GgufError::kOk) {
                ++accepted;
                for (const auto& t : index.tensors) (void)index.find(t.name.c_str());
            }
            ++reads;
            for (int k = 0; k < count; ++k) bytes[at[k]] = whole[at[k]];
        }
    }
    // layout of every format from pseudo-random blocks (odd counts, one block, many)
    for (uint32_t format : {0u, 2u, 3u, 8u, 14u}) {
        for (uint64_t blocks : {1ull, 3ull, 257ull, 4099ull}) {
            std::vector<uint8_t> stored(blocks * chm::block_bytes_host(format));
            for (auto& b : stored) b = static_cast<uint8_t>(next() >> 24);
            std::vector<uint8_t> device(chm::layout_bytes(format, blocks));
            if (!chm::lay_out(format, stored.data(), blocks, device.data())) return 3;
            if (format == 14u) {
                std::vector<uint8_t> lo(128 * blocks), hi(64 * blocks), sc(16 * blocks), d(2 * blocks);
                chm::repack_q6_k(stored.data(), blocks, lo.data(), hi.data(), sc.data(), d.data());
            }
        }
    }
    std::printf("host ok: %llu index reads, %llu accepted\n", static_cast<unsigned long long>(reads),
                static_cast<unsigned long long>(accepted));
    return 0;
}
