/*
 * CPU oracle for the quantized GGUF matrix product — TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker. The product (charlotte_amd/)
 * never links, loads or calls it.
 *
 * Each function restates one piece of plainsight-systems/charlotte's
 * algorithm for this path, citing the reference file:line it follows.
 * Pinning, per function (the checks live in tests/test_oracle.py):
 *   orc_fp16_to_fp32        known answers of tests/quant_q4_0_test.cpp:41-65;
 *                           all 65,536 inputs against numpy's float16 and
 *                           against oracle/_ref (the reference's own code).
 *   orc_bf16_to_fp32        every one of the 65,536 inputs against numpy's
 *                           uint32 shift and against the edge list of
 *                           tests/gpu/unpack_bf16_test.cpp:29-40.
 *   orc_dequantize_range    F16 and BF16 over the edge-and-LCG values of
 *   (F16, BF16)             tests/gpu/unpack_f16_test.cpp:24-35 and
 *                           unpack_bf16_test.cpp:29-40 against numpy's
 *                           float16 conversion and uint32 shift; F16 also
 *                           against oracle/_ref's fp16_to_fp32.
 *   orc_dequantize_q4_0     known answers of tests/quant_q4_0_test.cpp:87-145;
 *                           closed form; oracle/_ref on the edge-scale blocks
 *                           of tests/gpu/unpack_q4_0_test.cpp:24-37.
 *   orc_dequantize_q4_1     oracle/_ref (tests/support/q4_1_reference.h) on the
 *                           edge-scale blocks of tests/gpu/unpack_q4_1_test.cpp:
 *                           24-46, both answers; numpy's float32 (unfused)
 *                           evaluation; rounded == fused over every finite d.
 *   orc_dequantize_q8_0     oracle/_ref (q8_0_reference.h); closed form in numpy;
 *                           the reference fixture embedding_q8_0.gguf's
 *                           expected rows (tests/gpu/gather_test.cpp:149).
 *   orc_dequantize_q6_k     closed form (6-bit code, int8 scale, fp16 d) built
 *                           from the stored fields independently in the test;
 *                           oracle/_ref on tests/gpu/unpack_q6_k_test.cpp:24-41.
 *   orc_repack_q6_k /
 *   orc_lay_out             the placement invariant of
 *                           tests/formats_q6_k_repack_test.cpp:24-69; byte
 *                           equality with oracle/_ref's repack_q6_k.
 *   orc_unpack_group        equality with the file-order dequant over every
 *                           group (the device layout is lossless), each format.
 *   orc_gather,
 *   orc_gather_positions    rows against the file-order dequant of the fixture
 *                           tables tests/fixtures/gguf/embedding_*.gguf, with
 *                           the skip rules of gather.wgsl:34-52 checked on
 *                           hand-built steps (untouched rows keep a sentinel).
 *   orc_matmul_f32          order of addition pinned by hand-built cases whose
 *                           bits differ between orders (test_oracle.py), plus
 *                           within gamma(2K) of orc_matmul_f64.
 *   orc_matmul_f64          brute force against numpy float64 dot products.
 *   orc_matmul_f64_threads  the same rows split over threads: equal to the
 *                           one-thread result element for element (test).
 *   orc_fill_unit           the hash of tests/gpu/support/fill.h:24-29, pinned
 *                           by its range and by recomputation in numpy.
 *   orc_activate            against math.exp/tanh within its stated bound.
 *   orc_clamp, orc_finish,
 *   orc_gated,
 *   orc_gated_by_input      known answers whose values differ under any other
 *                           order of clamp, bias and activation, or with the
 *                           gate and up swapped; SiLU/GELU/sigmoid against
 *                           math.exp and math.tanh.
 * Nothing here is "parity unpinned".
 */
#ifndef CHARLOTTE_ORACLE_H
#define CHARLOTTE_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF tensor types (src/core/gguf/types.h:41-43). */
enum { ORC_F32 = 0, ORC_F16 = 1, ORC_Q4_0 = 2, ORC_Q4_1 = 3, ORC_Q8_0 = 8, ORC_Q6_K = 14, ORC_BF16 = 30 };

float orc_fp16_to_fp32(uint16_t h);
float orc_bf16_to_fp32(uint16_t h);

/* File-order blocks -> f32 weights, flat. */
void orc_dequantize_q4_0(const uint8_t* blocks, uint64_t nblocks, float* out);
void orc_dequantize_q6_k(const uint8_t* blocks, uint64_t nblocks, float* out);
/* Q4_1's two admissible answers: multiply and add each rounded, and one fma
 * (`fused` may be NULL). */
void orc_dequantize_q4_1(const uint8_t* blocks, uint64_t nblocks, float* rounded, float* fused);
void orc_dequantize_q8_0(const uint8_t* blocks, uint64_t nblocks, float* out);
/* Weights [first, first + count) of a tensor stored as `type` blocks. */
int orc_dequantize_range(uint32_t type, const uint8_t* blocks, uint64_t first, uint64_t count, float* out);

/* Device layout: bytes of a piece of `nblocks` blocks, rounded up to 4. */
uint64_t orc_layout_bytes(uint32_t type, uint64_t nblocks);
/* File-order blocks -> the piece's streams (SoA; Q6_K repacked). */
int orc_lay_out(uint32_t type, const uint8_t* blocks, uint64_t nblocks, uint8_t* device);
void orc_repack_q6_k(const uint8_t* blocks, uint64_t nblocks, uint8_t* lo, uint8_t* hi, uint8_t* scales,
                     uint8_t* d);
/* The 32 weights of `group` read from a piece's streams. */
int orc_unpack_group(uint32_t type, const uint8_t* device, uint64_t blocks_in_piece, uint64_t group, float* out);

/* The canonical range of a row of G groups: groups [lo(r), lo(r + 1)). */
uint64_t orc_range_lo(uint64_t r, uint64_t groups);

/* y[t * rows + o] over file-order blocks, in the reference's order of
 * addition (32 ranges, each an fma chain from zero, added in order). */
int orc_matmul_f32(uint32_t type, const uint8_t* blocks, uint64_t rows, uint64_t columns, const float* x,
                   uint32_t tokens, float* y, uint32_t threads);
/* The same in f64, and each output's bound gamma(2K) * sum |w x|. */
int orc_matmul_f64(uint32_t type, const uint8_t* blocks, uint64_t rows, uint64_t columns, const float* x,
                   uint32_t tokens, double* y, double* bound);
int orc_matmul_f64_threads(uint32_t type, const uint8_t* blocks, uint64_t rows, uint64_t columns, const float* x,
                           uint32_t tokens, double* y, double* bound, uint32_t threads);

/* tests/gpu/support/fill.h:24-29: a value in [-1, 1) for index i. */
float orc_fill_unit(uint32_t i);
void orc_fill(uint32_t seed, uint64_t count, float amplitude, float* out);

/* matmul.wgsl:169-205: 0 SiLU, 1 GELU (tanh form), 2 sigmoid. */
float orc_exp_nonpositive(float x);
float orc_activate(uint32_t activation, float g);

/* Epilogues (matmul.wgsl:117-132, 272-351): clamp_input/clamp_output; a
 * Write's finish (clamp, bias, activation, in order); the gated product
 * activate(clamp(gate)) * clamp(up); GatedByInput's activate(total) * u.
 * clip = {in_min, in_max, out_min, out_max} or NULL. */
void orc_clamp(const float* x, uint64_t count, float lo, float hi, float* out);
void orc_finish(const float* totals, uint64_t tokens, uint64_t rows, const float* clip, const float* bias,
                int activated, uint32_t activation, float* out);
void orc_gated(const float* gate, const float* up, uint64_t count, const float* clip, uint32_t activation,
               float* out);
void orc_gated_by_input(const float* totals, const float* u, uint64_t count, uint32_t activation, float* out);

/* The embedding gather (gather.wgsl:21-58): rows of `hidden` [tokens][columns]
 * from a piece of `row_count` stored rows holding vocabulary rows first_row ..;
 * rows whose token lies elsewhere, or is the media placeholder, untouched. */
int orc_gather(uint32_t type, const uint8_t* stored_rows, uint64_t row_count, uint64_t columns, uint64_t first_row,
               const uint32_t* ids, uint32_t tokens, const uint32_t* fed, int media, uint32_t media_token,
               float scale, float* hidden);
/* Its position form (gather.wgsl:65-84) over an F32 table of 2 x positions rows. */
int orc_gather_positions(const float* table, uint64_t columns, uint32_t positions, uint32_t grid_columns,
                         uint32_t tokens, float* out);

/* Monotonic seconds, for the CPU baseline timing. */
double orc_now(void);

#ifdef __cplusplus
}
#endif
#endif
