// oracle/_ref: the reference's own hot-path C++ compiled from its sources
// where they lie under /root/reference, behind a C interface for the tests.
// TEST INFRASTRUCTURE ONLY (see oracle.h). This file is this repository's;
// it includes, and does not copy, the reference's:
//   src/core/quant/q4_0.h            fp16_to_fp32 (lines 66-95)
//   tests/support/q4_0_reference.h   dequantize_q4_0 (lines 25-53)
//   tests/support/q6_k_reference.h   dequantize_q6_k (lines 17-47)
//   tests/support/q4_1_reference.h   dequantize_q4_1 (lines 27-54)
//   tests/support/q8_0_reference.h   dequantize_q8_0 (lines 14-27)
//   src/core/formats/device_layout.h kQ6_KLayout.repack (lines 124-134),
//                                    defined in q6_k/q6_k_repack.cpp:52-87
#include <array>
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <span>

#include "core/formats/device_layout.h"
#include "core/quant/q4_0.h"
#include "support/q4_0_reference.h"
#include "support/q4_1_reference.h"
#include "support/q6_k_reference.h"
#include "support/q8_0_reference.h"

extern "C" {

float ref_fp16_to_fp32(std::uint16_t h) { return bllm::quant::fp16_to_fp32(h); }

void ref_dequantize_q4_0(const std::uint8_t* blocks, std::uint64_t n, float* out) {
    const auto v = bllm::test::dequantize_q4_0(std::span<const std::uint8_t>(blocks, n * 18));
    std::memcpy(out, v.data(), v.size() * sizeof(float));
}

void ref_dequantize_q6_k(const std::uint8_t* blocks, std::uint64_t n, float* out) {
    const auto v = bllm::test::dequantize_q6_k(std::span<const std::uint8_t>(blocks, n * 210));
    std::memcpy(out, v.data(), v.size() * sizeof(float));
}

void ref_dequantize_q4_1(const std::uint8_t* blocks, std::uint64_t n, float* rounded, float* fused) {
    const auto v = bllm::test::dequantize_q4_1(std::span<const std::uint8_t>(blocks, n * 20));
    std::memcpy(rounded, v.rounded.data(), v.rounded.size() * sizeof(float));
    std::memcpy(fused, v.fused.data(), v.fused.size() * sizeof(float));
}

void ref_dequantize_q8_0(const std::uint8_t* blocks, std::uint64_t n, float* out) {
    const auto v = bllm::test::dequantize_q8_0(std::span<const std::uint8_t>(blocks, n * 34));
    std::memcpy(out, v.data(), v.size() * sizeof(float));
}

void ref_repack_q6_k(const std::uint8_t* blocks, std::uint64_t n, std::uint8_t* lo, std::uint8_t* hi,
                     std::uint8_t* scales, std::uint8_t* d) {
    const auto* bytes = reinterpret_cast<const std::byte*>(blocks);
    bllm::formats::kQ6_KLayout.repack(std::span<const std::byte>(bytes, n * 210),
                                      {reinterpret_cast<std::byte*>(lo), reinterpret_cast<std::byte*>(hi),
                                       reinterpret_cast<std::byte*>(scales), reinterpret_cast<std::byte*>(d)});
}

}  // extern "C"
