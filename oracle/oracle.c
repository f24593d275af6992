/*
 * CPU oracle for the quantized GGUF matrix product — TEST INFRASTRUCTURE ONLY.
 * See oracle.h for what may load it and how each function is pinned.
 *
 * Built with -ffp-contract=off so every expression rounds as written; every
 * multiply-add that the reference writes as an fma is an explicit fmaf here
 * (tests/gpu/CMakeLists.txt:44-46 builds the reference's oracles the same way).
 */
#define _GNU_SOURCE
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

/* ---- fp16 ---------------------------------------------------------------- */

/* IEEE binary16 -> binary32, exact for every input
 * (src/core/quant/q4_0.h:66-95). A subnormal half is its 10-bit mantissa
 * times 2^-24, which binary32 holds exactly. */
float orc_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exponent = (h >> 10) & 0x1Fu;
    const uint32_t mantissa = h & 0x3FFu;
    uint32_t bits;
    if (exponent == 0) {
        const float magnitude = ldexpf((float)mantissa, -24);
        memcpy(&bits, &magnitude, 4);
        bits |= sign;
    } else if (exponent == 0x1Fu) {
        bits = sign | 0x7F800000u | (mantissa << 13);
    } else {
        bits = sign | ((exponent + 112u) << 23) | (mantissa << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static uint16_t le16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* bfloat16 -> binary32: the 16 bits are the top half of an f32, so the value
 * is exact, sign of zero and subnormals as stored (ggml_bf16_to_fp32, as
 * src/core/formats/bf16/bf16.h:16-25 and tests/gpu/unpack_bf16_test.cpp:21
 * state it). */
float orc_bf16_to_fp32(uint16_t h) {
    const uint32_t bits = (uint32_t)h << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* ---- dequantization (file order) ---------------------------------------- */

/* ggml's dequantize_row_q4_0 as tests/support/q4_0_reference.h:25-53 mirrors
 * it: an 18-byte block is the fp16 scale d, then 16 code bytes; byte j holds
 * weight j in its low nibble and weight j + 16 in its high nibble
 * (src/core/quant/q4_0.h:41-58); weight = (code - 8) * d. */
void orc_dequantize_q4_0(const uint8_t* blocks, uint64_t nblocks, float* out) {
    for (uint64_t b = 0; b < nblocks; ++b) {
        const uint8_t* block = blocks + b * 18;
        const float d = orc_fp16_to_fp32(le16(block));
        for (int j = 0; j < 16; ++j) {
            const int low = (block[2 + j] & 0x0F) - 8;
            const int high = (block[2 + j] >> 4) - 8;
            out[b * 32 + j] = (float)low * d;
            out[b * 32 + j + 16] = (float)high * d;
        }
    }
}

/* ggml's dequantize_row_q6_K as tests/support/q6_k_reference.h:17-47 mirrors
 * it: a 210-byte super-block of 256 weights is ql[128], qh[64], int8
 * scales[16], fp16 d. Weight l of group k (h = k / 4, r = k % 4) takes its low
 * nibble from nibble r / 2 of ql[64h + 32(r % 2) + l] and its high pair from
 * bits 2r of qh[32h + l]; its scale is scales[2k + l / 16]; the weight is
 * (d * scale) * (q - 32), evaluated left to right. */
void orc_dequantize_q6_k(const uint8_t* blocks, uint64_t nblocks, float* out) {
    for (uint64_t b = 0; b < nblocks; ++b) {
        const uint8_t* block = blocks + b * 210;
        const float d = orc_fp16_to_fp32(le16(block + 208));
        for (int k = 0; k < 8; ++k) {
            const int h = k / 4, r = k % 4;
            for (int l = 0; l < 32; ++l) {
                const int low = (block[64 * h + 32 * (r % 2) + l] >> (4 * (r / 2))) & 0xF;
                const int pair = (block[128 + 32 * h + l] >> (2 * r)) & 3;
                const int q = (low | (pair << 4)) - 32;
                const float scale = (float)(int8_t)block[192 + 2 * k + l / 16];
                out[b * 256 + 32 * k + l] = d * scale * (float)q;
            }
        }
    }
}

/* ggml's dequantize_row_q4_1 as tests/support/q4_1_reference.h:27-54 mirrors
 * it: a 20-byte block is fp16 d, fp16 m, then 16 code bytes; weight j is
 * (qs[j] & 0xF) * d + m and weight j + 16 is (qs[j] >> 4) * d + m. The
 * reference keeps two answers, the multiply and the add each rounded
 * (`rounded`) and one fma (`fused`); `fused` may be NULL. Either is written
 * out explicitly here. (The 4-bit code times the 11-bit d is exact in f32, so
 * the two agree on every block; the tests check that rather than assume it.) */
void orc_dequantize_q4_1(const uint8_t* blocks, uint64_t nblocks, float* rounded, float* fused) {
    for (uint64_t b = 0; b < nblocks; ++b) {
        const uint8_t* block = blocks + b * 20;
        const float d = orc_fp16_to_fp32(le16(block));
        const float m = orc_fp16_to_fp32(le16(block + 2));
        for (int j = 0; j < 16; ++j) {
            const float lo = (float)(block[4 + j] & 0x0F);
            const float hi = (float)(block[4 + j] >> 4);
            const float lo_d = lo * d;
            const float hi_d = hi * d;
            rounded[b * 32 + j] = lo_d + m;
            rounded[b * 32 + j + 16] = hi_d + m;
            if (fused) {
                fused[b * 32 + j] = fmaf(lo, d, m);
                fused[b * 32 + j + 16] = fmaf(hi, d, m);
            }
        }
    }
}

/* ggml's dequantize_row_q8_0 as tests/support/q8_0_reference.h:14-27 mirrors
 * it: a 34-byte block is fp16 d, then 32 signed 8-bit codes; weight j is
 * qs[j] * d. */
void orc_dequantize_q8_0(const uint8_t* blocks, uint64_t nblocks, float* out) {
    for (uint64_t b = 0; b < nblocks; ++b) {
        const uint8_t* block = blocks + b * 34;
        const float d = orc_fp16_to_fp32(le16(block));
        for (int j = 0; j < 32; ++j) out[b * 32 + j] = (float)(int8_t)block[2 + j] * d;
    }
}

/* src/core/gguf/types.h:65-101: weights a block and bytes a block. F32's
 * "block" is one float. */
static int block_shape(uint32_t type, uint64_t* elements, uint64_t* bytes) {
    switch (type) {
        case ORC_F32: *elements = 1; *bytes = 4; return 0;
        case ORC_F16: *elements = 1; *bytes = 2; return 0;
        case ORC_BF16: *elements = 1; *bytes = 2; return 0;
        case ORC_Q4_0: *elements = 32; *bytes = 18; return 0;
        case ORC_Q4_1: *elements = 32; *bytes = 20; return 0;
        case ORC_Q8_0: *elements = 32; *bytes = 34; return 0;
        case ORC_Q6_K: *elements = 256; *bytes = 210; return 0;
        default: return -1;
    }
}

int orc_dequantize_range(uint32_t type, const uint8_t* blocks, uint64_t first, uint64_t count, float* out) {
    uint64_t per_block, block_bytes;
    if (block_shape(type, &per_block, &block_bytes) != 0) return -1;
    if (count == 0) return 0;
    const uint64_t b0 = first / per_block, b1 = (first + count - 1) / per_block;
    float* tmp = malloc((size_t)((b1 - b0 + 1) * per_block * sizeof(float)));
    if (!tmp) return -2;
    const uint8_t* at = blocks + b0 * block_bytes;
    const uint64_t n = b1 - b0 + 1;
    switch (type) {
        case ORC_F32: memcpy(tmp, at, (size_t)(n * 4)); break;
        /* F16: quant::fp16_to_fp32 of each half (tests/gpu/unpack_f16_test.cpp:39);
         * BF16: its top-half shift (unpack_bf16_test.cpp:21). */
        case ORC_F16:
            for (uint64_t i = 0; i < n; ++i) tmp[i] = orc_fp16_to_fp32(le16(at + 2 * i));
            break;
        case ORC_BF16:
            for (uint64_t i = 0; i < n; ++i) tmp[i] = orc_bf16_to_fp32(le16(at + 2 * i));
            break;
        case ORC_Q4_0: orc_dequantize_q4_0(at, n, tmp); break;
        /* tests/gpu/matmul_test.cpp:153 decodes Q4_1 by its rounded answer */
        case ORC_Q4_1: orc_dequantize_q4_1(at, n, tmp, NULL); break;
        case ORC_Q8_0: orc_dequantize_q8_0(at, n, tmp); break;
        default: orc_dequantize_q6_k(at, n, tmp); break;
    }
    memcpy(out, tmp + (first - b0 * per_block), (size_t)count * sizeof(float));
    free(tmp);
    return 0;
}

/* ---- device layout -------------------------------------------------------- */

/* src/core/formats/device_layout.h:111-136: a piece of n blocks is its
 * streams one after another, every block's field of one stream before the
 * next stream's; the piece is the stored bytes rounded up to 4. */
uint64_t orc_layout_bytes(uint32_t type, uint64_t nblocks) {
    uint64_t per_block, block_bytes;
    if (block_shape(type, &per_block, &block_bytes) != 0) return 0;
    return (nblocks * block_bytes + 3) / 4 * 4;
}

/* The repack of src/core/formats/q6_k/q6_k.h:11-21 restated weight by weight
 * (the reference moves 8 bytes at a time, src/core/formats/q6_k/
 * q6_k_repack.cpp:52-87; the layout is the contract): group k's low nibbles at
 * lo byte 16k + l % 16 (low half for l < 16), its high pairs at hi byte
 * 8k + l % 8, bits 2(l / 8); scales and d copied as stored. */
void orc_repack_q6_k(const uint8_t* blocks, uint64_t nblocks, uint8_t* lo, uint8_t* hi, uint8_t* scales,
                     uint8_t* d) {
    for (uint64_t b = 0; b < nblocks; ++b) {
        const uint8_t* block = blocks + b * 210;
        uint8_t* blo = lo + b * 128;
        uint8_t* bhi = hi + b * 64;
        memset(blo, 0, 128);
        memset(bhi, 0, 64);
        for (int k = 0; k < 8; ++k) {
            const int h = k / 4, r = k % 4;
            for (int l = 0; l < 32; ++l) {
                const int low = (block[64 * h + 32 * (r % 2) + l] >> (4 * (r / 2))) & 0xF;
                const int pair = (block[128 + 32 * h + l] >> (2 * r)) & 3;
                blo[16 * k + l % 16] |= (uint8_t)(low << (4 * (l / 16)));
                bhi[8 * k + l % 8] |= (uint8_t)(pair << (2 * (l / 8)));
            }
        }
        memcpy(scales + b * 16, block + 192, 16);
        memcpy(d + b * 2, block + 208, 2);
    }
}

int orc_lay_out(uint32_t type, const uint8_t* blocks, uint64_t nblocks, uint8_t* device) {
    const uint64_t total = orc_layout_bytes(type, nblocks);
    if (total == 0 && nblocks != 0) return -1;
    memset(device, 0, (size_t)total);
    if (type == ORC_Q4_0) {
        /* kQ4_0 = {{2, 16}, {0, 2}}: the codes, then the scales
         * (device_layout.h:121; residency/piece_writer.cpp:51-73). */
        for (uint64_t b = 0; b < nblocks; ++b) {
            memcpy(device + 16 * b, blocks + 18 * b + 2, 16);
            memcpy(device + 16 * nblocks + 2 * b, blocks + 18 * b, 2);
        }
        return 0;
    }
    if (type == ORC_Q6_K) {
        /* kQ6_K = {{0,128},{128,64},{192,16},{208,2}} of the repacked block
         * (device_layout.h:124-127). */
        orc_repack_q6_k(blocks, nblocks, device, device + 128 * nblocks, device + 192 * nblocks,
                        device + 208 * nblocks);
        return 0;
    }
    if (type == ORC_Q4_1) {
        /* kQ4_1 = {{4, 16}, {0, 4}}: the codes, then d and m together, one
         * word a block (device_layout.h:122). */
        for (uint64_t b = 0; b < nblocks; ++b) {
            memcpy(device + 16 * b, blocks + 20 * b + 4, 16);
            memcpy(device + 16 * nblocks + 4 * b, blocks + 20 * b, 4);
        }
        return 0;
    }
    if (type == ORC_Q8_0) {
        /* kQ8_0 = {{2, 32}, {0, 2}}: the codes, then the scales
         * (device_layout.h:123). */
        for (uint64_t b = 0; b < nblocks; ++b) {
            memcpy(device + 32 * b, blocks + 34 * b + 2, 32);
            memcpy(device + 32 * nblocks + 2 * b, blocks + 34 * b, 2);
        }
        return 0;
    }
    if (type == ORC_F32) {
        /* kF32 = {{0, 4}}: the floats as stored (device_layout.h:118). */
        memcpy(device, blocks, (size_t)(4 * nblocks));
        return 0;
    }
    if (type == ORC_F16 || type == ORC_BF16) {
        /* kF16 = kBF16 = {{0, 2}}: the values as stored (device_layout.h:119-120). */
        memcpy(device, blocks, (size_t)(2 * nblocks));
        return 0;
    }
    return -1;
}

/* The 32 weights of `group` as the format's unpack reads them from a piece
 * (src/core/formats/q4_0/q4_0.wgsl:6-18, src/core/formats/q6_k/q6_k.wgsl:13-42):
 * Q4_0 group g is block g; Q6_K group g is group g % 8 of super-block g / 8,
 * counted flat over the piece, so a row need not be whole super-blocks. */
int orc_unpack_group(uint32_t type, const uint8_t* device, uint64_t n, uint64_t group, float* out) {
    if (type == ORC_Q4_0) {
        const uint8_t* codes = device + 16 * group;
        const float d = orc_fp16_to_fp32(le16(device + 16 * n + 2 * group));
        for (int j = 0; j < 16; ++j) {
            out[j] = (float)((codes[j] & 0xF) - 8) * d;
            out[j + 16] = (float)((codes[j] >> 4) - 8) * d;
        }
        return 0;
    }
    if (type == ORC_Q6_K) {
        const uint64_t b = group / 8, k = group % 8;
        const uint8_t* lo = device + 128 * b + 16 * k;
        const uint8_t* hi = device + 128 * n + 64 * b + 8 * k;
        const uint8_t* sc = device + 192 * n + 16 * b + 2 * k;
        const float d = orc_fp16_to_fp32(le16(device + 208 * n + 2 * b));
        const float first = d * (float)(int8_t)sc[0];
        const float second = d * (float)(int8_t)sc[1];
        for (int l = 0; l < 32; ++l) {
            const int low = (lo[l % 16] >> (4 * (l / 16))) & 0xF;
            const int pair = (hi[l % 8] >> (2 * (l / 8))) & 3;
            out[l] = (l < 16 ? first : second) * (float)((low | (pair << 4)) - 32);
        }
        return 0;
    }
    if (type == ORC_Q4_1) {
        /* src/core/formats/q4_1/q4_1.wgsl:6-17; the rounded answer. */
        const uint8_t* codes = device + 16 * group;
        const float d = orc_fp16_to_fp32(le16(device + 16 * n + 4 * group));
        const float m = orc_fp16_to_fp32(le16(device + 16 * n + 4 * group + 2));
        for (int j = 0; j < 16; ++j) {
            const float lo_d = (float)(codes[j] & 0xF) * d;
            const float hi_d = (float)(codes[j] >> 4) * d;
            out[j] = lo_d + m;
            out[j + 16] = hi_d + m;
        }
        return 0;
    }
    if (type == ORC_Q8_0) {
        /* src/core/formats/q8_0/q8_0.wgsl:6-17. */
        const uint8_t* codes = device + 32 * group;
        const float d = orc_fp16_to_fp32(le16(device + 32 * n + 2 * group));
        for (int j = 0; j < 32; ++j) out[j] = (float)(int8_t)codes[j] * d;
        return 0;
    }
    if (type == ORC_F32) {
        /* src/core/formats/f32/f32.wgsl:5-13: floats 32g .. 32g + 31. */
        memcpy(out, device + 128 * group, 128);
        return 0;
    }
    if (type == ORC_F16 || type == ORC_BF16) {
        /* src/core/formats/f16/f16.wgsl:6-13, bf16/bf16.wgsl:8-18: values
         * 32g .. 32g + 31, two a word, the lower half first. */
        const uint8_t* at = device + 64 * group;
        for (int j = 0; j < 32; ++j)
            out[j] = type == ORC_F16 ? orc_fp16_to_fp32(le16(at + 2 * j)) : orc_bf16_to_fp32(le16(at + 2 * j));
        return 0;
    }
    return -1;
}

/* ---- the products ---------------------------------------------------------- */

/* src/core/kernels/matmul/matmul.h:34-40, matmul.wgsl:134-137: range r of a
 * row's G groups is groups floor(rG / 32) .. floor((r + 1)G / 32). */
uint64_t orc_range_lo(uint64_t r, uint64_t groups) { return r * groups / 32; }

struct f32_job {
    uint32_t type;
    const uint8_t* blocks;
    uint64_t rows, columns, row_begin, row_end;
    const float* x;
    uint32_t tokens;
    float* y;
    int status;
};

enum { kRowBlock = 8 };

/* Rows [row_begin, row_end) for every token. Each output is
 *   y = ((0 + s_0) + s_1) + ... + s_31,  s_r = fma chain from 0 over range r
 * (src/core/kernels/matmul/matmul.h:34-50): the 32 range sums added in order
 * to a total from zero, each range its weights in k order. kRowBlock rows go
 * together so the compiler may run their independent chains side by side;
 * each chain is still its own, in order. */
static void* f32_rows(void* arg) {
    struct f32_job* job = arg;
    const uint64_t K = job->columns, G = K / 32;
    float* w = malloc((size_t)(kRowBlock * K * sizeof(float)));
    if (!w) {
        job->status = -2;
        return NULL;
    }
    for (uint64_t o0 = job->row_begin; o0 < job->row_end; o0 += kRowBlock) {
        const uint64_t n = job->row_end - o0 < kRowBlock ? job->row_end - o0 : kRowBlock;
        if (orc_dequantize_range(job->type, job->blocks, o0 * K, n * K, w) != 0) {
            job->status = -1;
            break;
        }
        for (uint32_t t = 0; t < job->tokens; ++t) {
            const float* x = job->x + (uint64_t)t * K;
            float total[kRowBlock] = {0};
            for (uint64_t r = 0; r < 32; ++r) {
                float s[kRowBlock] = {0};
                const uint64_t k0 = orc_range_lo(r, G) * 32, k1 = orc_range_lo(r + 1, G) * 32;
                for (uint64_t k = k0; k < k1; ++k) {
                    for (uint64_t i = 0; i < kRowBlock; ++i) s[i] = fmaf(w[(i < n ? i : 0) * K + k], x[k], s[i]);
                }
                for (uint64_t i = 0; i < kRowBlock; ++i) total[i] = total[i] + s[i];
            }
            for (uint64_t i = 0; i < n; ++i) job->y[(uint64_t)t * job->rows + o0 + i] = total[i];
        }
    }
    free(w);
    return NULL;
}

int orc_matmul_f32(uint32_t type, const uint8_t* blocks, uint64_t rows, uint64_t columns, const float* x,
                   uint32_t tokens, float* y, uint32_t threads) {
    uint64_t per_block, block_bytes;
    if (columns % 32 != 0 || block_shape(type, &per_block, &block_bytes) != 0) return -1;
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    struct f32_job jobs[256];
    pthread_t ids[256];
    /* Whole kRowBlock groups of rows a thread, so every thread's blocks
     * start on the same boundaries whatever the count. */
    const uint64_t units = (rows + kRowBlock - 1) / kRowBlock;
    for (uint32_t i = 0; i < threads; ++i) {
        const uint64_t u0 = units * i / threads, u1 = units * (i + 1) / threads;
        const uint64_t r0 = u0 * kRowBlock, r1 = u1 * kRowBlock < rows ? u1 * kRowBlock : rows;
        jobs[i] = (struct f32_job){type, blocks, rows, columns, r0, r1 > r0 ? r1 : r0, x, tokens, y, 0};
    }
    if (threads == 1) {
        f32_rows(&jobs[0]);
        return jobs[0].status;
    }
    for (uint32_t i = 0; i < threads; ++i) pthread_create(&ids[i], NULL, f32_rows, &jobs[i]);
    int status = 0;
    for (uint32_t i = 0; i < threads; ++i) {
        pthread_join(ids[i], NULL);
        if (jobs[i].status != 0) status = jobs[i].status;
    }
    return status;
}

/* tests/gpu/matmul_test.cpp:190-211: each output in f64 over the decoded
 * weights, and its bound gamma(2K) * sum_k |w x|, gamma(n) = nu / (1 - nu),
 * u = 2^-24. Rows [r0, r1) of the product, one job of orc_matmul_f64_threads. */
struct f64_job {
    uint32_t type;
    const uint8_t* blocks;
    uint64_t rows, columns, r0, r1;
    const float* x;
    uint32_t tokens;
    double *y, *bound;
    int status;
};

static void* f64_rows(void* arg) {
    struct f64_job* j = arg;
    const uint64_t K = j->columns;
    const double nu = (double)(2 * K) * ldexp(1.0, -24);
    const double gamma = nu / (1 - nu);
    float* w = malloc((size_t)(K * sizeof(float)));
    if (!w) {
        j->status = -2;
        return NULL;
    }
    for (uint64_t o = j->r0; o < j->r1; ++o) {
        if (orc_dequantize_range(j->type, j->blocks, o * K, K, w) != 0) {
            j->status = -1;
            break;
        }
        for (uint32_t t = 0; t < j->tokens; ++t) {
            double sum = 0, absolute = 0;
            for (uint64_t k = 0; k < K; ++k) {
                const double p = (double)w[k] * (double)j->x[(uint64_t)t * K + k];
                sum += p;
                absolute += fabs(p);
            }
            j->y[(uint64_t)t * j->rows + o] = sum;
            if (j->bound) j->bound[(uint64_t)t * j->rows + o] = gamma * absolute;
        }
    }
    free(w);
    return NULL;
}

/* The same on `threads` host threads, rows split evenly (each output is one
 * thread's whole sum, so the values do not depend on the count). */
int orc_matmul_f64_threads(uint32_t type, const uint8_t* blocks, uint64_t rows, uint64_t columns, const float* x,
                           uint32_t tokens, double* y, double* bound, uint32_t threads) {
    if (columns % 32 != 0) return -1;
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    struct f64_job jobs[256];
    pthread_t ids[256];
    for (uint32_t i = 0; i < threads; ++i)
        jobs[i] = (struct f64_job){type, blocks, rows, columns, rows * i / threads, rows * (i + 1) / threads,
                                   x, tokens, y, bound, 0};
    if (threads == 1) {
        f64_rows(&jobs[0]);
        return jobs[0].status;
    }
    for (uint32_t i = 0; i < threads; ++i) pthread_create(&ids[i], NULL, f64_rows, &jobs[i]);
    int status = 0;
    for (uint32_t i = 0; i < threads; ++i) {
        pthread_join(ids[i], NULL);
        if (jobs[i].status != 0) status = jobs[i].status;
    }
    return status;
}

int orc_matmul_f64(uint32_t type, const uint8_t* blocks, uint64_t rows, uint64_t columns, const float* x,
                   uint32_t tokens, double* y, double* bound) {
    return orc_matmul_f64_threads(type, blocks, rows, columns, x, tokens, y, bound, 1);
}

/* ---- the reference tests' input fill -------------------------------------- */

/* tests/gpu/support/fill.h:24-29: a 32-bit integer hash, its top 24 bits
 * scaled to [0, 2) and shifted to [-1, 1). */
float orc_fill_unit(uint32_t i) {
    uint32_t v = i * 747796405u + 2891336453u;
    v = ((v >> ((v >> 28) + 4u)) ^ v) * 277803737u;
    v = (v >> 22) ^ v;
    return (float)(v >> 8) / 8388608.0f - 1.0f;
}

void orc_fill(uint32_t seed, uint64_t count, float amplitude, float* out) {
    for (uint64_t i = 0; i < count; ++i) out[i] = orc_fill_unit(seed + (uint32_t)i) * amplitude;
}

/* ---- activations (epilogues) ---------------------------------------------- */

/* matmul.wgsl:169-185: e^x for x <= 0 by Cody-Waite reduction with ln 2 in two
 * parts, a degree-6 Taylor polynomial in Horner form, then 2^k; every
 * multiply-add an fma. */
float orc_exp_nonpositive(float x) {
    const float xc = fmaxf(x, -100.0f);
    const float k = floorf(fmaf(xc, 1.4426950408889634f, 0.5f));
    float r = fmaf(k, -0.693145751953125f, xc);
    r = fmaf(k, -1.4286068203094172e-06f, r);
    float p = 1.0f / 720.0f;
    p = fmaf(p, r, 1.0f / 120.0f);
    p = fmaf(p, r, 1.0f / 24.0f);
    p = fmaf(p, r, 1.0f / 6.0f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return ldexpf(p, (int)k);
}

/* matmul.wgsl:187-205. */
float orc_activate(uint32_t activation, float g) {
    if (activation == 0 || activation == 2) {
        const float e = orc_exp_nonpositive(-fabsf(g));
        const float r = 1.0f / (1.0f + e);
        const float s = g >= 0.0f ? r : e * r;
        return activation == 0 ? g * s : s;
    }
    const float z = 0.7978845608028654f * fmaf(0.044715f * g * g, g, g);
    const float e = orc_exp_nonpositive(-2.0f * fabsf(z));
    const float sign = z > 0.0f ? 1.0f : (z < 0.0f ? -1.0f : 0.0f);
    const float t = sign * ((1.0f - e) * (1.0f / (1.0f + e)));
    const float half_g = 0.5f * g;
    return fmaf(half_g, t, half_g);
}

/* matmul.wgsl:117-132: WGSL's clamp(e, low, high) = min(max(e, low), high),
 * the input's bounds as it is staged, the output's on each total. */
static float clampf(float v, float lo, float hi) { return fminf(fmaxf(v, lo), hi); }

void orc_clamp(const float* x, uint64_t count, float lo, float hi, float* out) {
    for (uint64_t i = 0; i < count; ++i) out[i] = clampf(x[i], lo, hi);
}

/* matmul.wgsl:272-284 (finish): a Write's output from its total, clamped to
 * the output bounds, then the bias of its output row added, then the
 * activation, in that order. `clip` is in_min, in_max, out_min, out_max or
 * NULL; `bias` one float an output row or NULL. totals/out [tokens][rows]. */
void orc_finish(const float* totals, uint64_t tokens, uint64_t rows, const float* clip, const float* bias,
                int activated, uint32_t activation, float* out) {
    for (uint64_t t = 0; t < tokens; ++t)
        for (uint64_t o = 0; o < rows; ++o) {
            float y = totals[t * rows + o];
            if (clip) y = clampf(y, clip[2], clip[3]);
            if (bias) y = y + bias[o];
            if (activated) y = orc_activate(activation, y);
            out[t * rows + o] = y;
        }
}

/* matmul.wgsl:318-345, 556-573 (decode_gated, prefill_gated): activation of
 * the clamped gate total times the clamped up total. */
void orc_gated(const float* gate, const float* up, uint64_t count, const float* clip, uint32_t activation,
               float* out) {
    for (uint64_t i = 0; i < count; ++i) {
        const float g = clip ? clampf(gate[i], clip[2], clip[3]) : gate[i];
        const float u = clip ? clampf(up[i], clip[2], clip[3]) : up[i];
        out[i] = orc_activate(activation, g) * u;
    }
}

/* matmul.wgsl:347-351 (gated_by_input): the activation of the total times u. */
void orc_gated_by_input(const float* totals, const float* u, uint64_t count, uint32_t activation, float* out) {
    for (uint64_t i = 0; i < count; ++i) out[i] = orc_activate(activation, totals[i]) * u[i];
}

/* ---- the embedding gather ------------------------------------------------ */

/* src/core/kernels/gather/gather.wgsl:21-58 over a piece of `row_count` table
 * rows of `columns` weights holding vocabulary rows first_row ..: row i of
 * `hidden` is its token's row, each weight decoded, then multiplied by
 * `scale` (tests/gpu/gather_test.cpp:130-152: the format's CPU reference times
 * the scale). A token is fed[0] when `fed` is not NULL, else ids[i]; with
 * `media`, a row whose id is media_token is left as it was; a token outside
 * the piece leaves its row as it was. */
int orc_gather(uint32_t type, const uint8_t* stored_rows, uint64_t row_count, uint64_t columns, uint64_t first_row,
               const uint32_t* ids, uint32_t tokens, const uint32_t* fed, int media, uint32_t media_token,
               float scale, float* hidden) {
    uint64_t per_block, block_bytes;
    if (block_shape(type, &per_block, &block_bytes) != 0 || columns % per_block != 0) return -1;
    const uint64_t row_bytes = columns / per_block * block_bytes;
    float* w = malloc((size_t)(columns * sizeof(float)));
    if (!w) return -2;
    for (uint32_t i = 0; i < tokens; ++i) {
        uint32_t token;
        if (fed) {
            token = fed[0];
        } else {
            token = ids[i];
            if (media && token == media_token) continue;
        }
        if (token < first_row || token - first_row >= row_count) continue;
        orc_dequantize_range(type, stored_rows + (token - first_row) * row_bytes, 0, columns, w);
        for (uint64_t c = 0; c < columns; ++c) hidden[(uint64_t)i * columns + c] = w[c] * scale;
    }
    free(w);
    return 0;
}

/* gather.wgsl:65-84 (the position form): patch row r, at x = r % grid_columns
 * and y = r / grid_columns, is table row x plus table row positions + y. */
int orc_gather_positions(const float* table, uint64_t columns, uint32_t positions, uint32_t grid_columns,
                         uint32_t tokens, float* out) {
    if (grid_columns == 0) return -1;
    for (uint32_t r = 0; r < tokens; ++r) {
        const uint64_t x = r % grid_columns, y = r / grid_columns;
        for (uint64_t c = 0; c < columns; ++c)
            out[(uint64_t)r * columns + c] = table[x * columns + c] + table[(positions + y) * columns + c];
    }
    return 0;
}

double orc_now(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}
