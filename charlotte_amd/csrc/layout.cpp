// The device layout, written on the host from file-order blocks
// (src/core/formats/device_layout.h:95-136; residency/piece_writer.cpp:51-73,
// 194-205; formats/q6_k/q6_k_repack.cpp:52-87).
//
// Q4_0: a piece is every block's 16 code bytes, then every block's fp16
// scale; Q4_1 its 16 code bytes, then its d and m, a dword a block; Q8_0 its
// 32 code bytes, then its fp16 scale; F32, F16 and BF16 the values as
// stored (device_layout.h:118-120). Q6_K: each super-block repacked so a 32-weight group's bits lie
// together — its low nibbles in 16 bytes (byte j: weight j's nibble, then
// weight j + 16's), its high pairs in 8 (byte m: weights m, m + 8, m + 16,
// m + 24 at bits 0, 2, 4, 6) — the piece being every block's lo, then hi, then
// the scales and the d's as stored. The stored block keeps weight l of group
// k = 4h + r at nibble r / 2 of ql[64h + 32(r % 2) + l] and bits 2r of
// qh[32h + l].
//
// The repack here works a group at a time on whole byte rows, so the
// compiler vectorizes each row: lo's 16 bytes are two 16-byte runs of ql
// shifted and masked, hi's 8 bytes four 8-byte runs of qh. Large tensors are
// split over threads by blocks.
#include "layout.hpp"

#include <algorithm>
#include <cstring>
#include <thread>
#include <vector>

namespace chm {

uint64_t layout_bytes(uint32_t format, uint64_t blocks) {
    const uint32_t b = block_bytes_host(format);
    return b == 0 ? 0 : (blocks * b + 3) / 4 * 4;
}

static void repack_q6_k_range(const uint8_t* stored, uint64_t begin, uint64_t end, uint8_t* lo, uint8_t* hi,
                              uint8_t* scales, uint8_t* d) {
    for (uint64_t b = begin; b < end; ++b) {
        const uint8_t* block = stored + 210 * b;
        uint8_t* blo = lo + 128 * b;
        uint8_t* bhi = hi + 64 * b;
        for (int k = 0; k < 8; ++k) {
            const int h = k >> 2, r = k & 3;
            const uint8_t* ql = block + 64 * h + 32 * (r & 1);
            const int nibble = 4 * (r >> 1);
            uint8_t* out = blo + 16 * k;
            for (int j = 0; j < 16; ++j) {
                out[j] = static_cast<uint8_t>(((ql[j] >> nibble) & 0x0F) | (((ql[j + 16] >> nibble) & 0x0F) << 4));
            }
            const uint8_t* qh = block + 128 + 32 * h;
            uint8_t* pairs = bhi + 8 * k;
            for (int m = 0; m < 8; ++m) {
                pairs[m] = static_cast<uint8_t>(((qh[m] >> (2 * r)) & 3) | (((qh[m + 8] >> (2 * r)) & 3) << 2) |
                                                (((qh[m + 16] >> (2 * r)) & 3) << 4) |
                                                (((qh[m + 24] >> (2 * r)) & 3) << 6));
            }
        }
        std::memcpy(scales + 16 * b, block + 192, 16);
        std::memcpy(d + 2 * b, block + 208, 2);
    }
}

static void gather_q4_0_range(const uint8_t* stored, uint64_t begin, uint64_t end, uint64_t n, uint8_t* device) {
    for (uint64_t b = begin; b < end; ++b) {
        std::memcpy(device + 16 * b, stored + 18 * b + 2, 16);
        std::memcpy(device + 16 * n + 2 * b, stored + 18 * b, 2);
    }
}

// Codes, then the block's leading `head` bytes (its scales), for the formats
// whose streams are the stored block's fields (device_layout.h:121-123).
static void split_range(const uint8_t* stored, uint64_t begin, uint64_t end, uint64_t n, uint32_t head,
                        uint32_t codes, uint8_t* device) {
    const uint32_t block = head + codes;
    for (uint64_t b = begin; b < end; ++b) {
        std::memcpy(device + codes * b, stored + block * b + head, codes);
        std::memcpy(device + codes * n + head * b, stored + block * b, head);
    }
}

// Blocks a thread takes at least, so small tensors stay on one thread.
constexpr uint64_t kBlocksAThread = 1u << 14;

template <typename Fn>
static void over_threads(uint64_t blocks, Fn fn) {
    const uint64_t hw = std::max(1u, std::thread::hardware_concurrency());
    const uint64_t threads = std::min<uint64_t>(std::min<uint64_t>(hw, 32), std::max<uint64_t>(1, blocks / kBlocksAThread));
    if (threads <= 1) {
        fn(0, blocks);
        return;
    }
    std::vector<std::thread> pool;
    for (uint64_t i = 0; i < threads; ++i) {
        pool.emplace_back(fn, blocks * i / threads, blocks * (i + 1) / threads);
    }
    for (auto& t : pool) t.join();
}

void repack_q6_k(const uint8_t* stored, uint64_t blocks, uint8_t* lo, uint8_t* hi, uint8_t* scales, uint8_t* d) {
    over_threads(blocks, [&](uint64_t b0, uint64_t b1) { repack_q6_k_range(stored, b0, b1, lo, hi, scales, d); });
}

bool lay_out(uint32_t format, const uint8_t* stored, uint64_t blocks, uint8_t* device) {
    const uint64_t total = layout_bytes(format, blocks);
    if (total == 0 && blocks != 0) return false;
    const uint64_t stored_bytes = blocks * block_bytes_host(format);
    std::memset(device + stored_bytes, 0, total - stored_bytes);
    if (format == 2) {
        over_threads(blocks, [&](uint64_t b0, uint64_t b1) { gather_q4_0_range(stored, b0, b1, blocks, device); });
        return true;
    }
    if (format == 3 || format == 8) {
        const uint32_t head = format == 3 ? 4 : 2, codes = format == 3 ? 16 : 32;
        over_threads(blocks, [&](uint64_t b0, uint64_t b1) { split_range(stored, b0, b1, blocks, head, codes, device); });
        return true;
    }
    if (format == 0 || format == 1 || format == 30) {
        std::memcpy(device, stored, stored_bytes);
        return true;
    }
    if (format == 14) {
        repack_q6_k(stored, blocks, device, device + 128 * blocks, device + 192 * blocks, device + 208 * blocks);
        return true;
    }
    return false;
}

}  // namespace chm
