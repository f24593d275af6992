/*
 * charlotte_hip_matmul — the quantized GGUF matrix product of
 * plainsight-systems/charlotte on AMD Instinct MI355X (gfx950), behind a C ABI.
 *
 *   y[t][o] = sum_k W[o][k] * x[t][k]
 *
 * W stays in its GGUF format (Q4_0, Q4_1, Q8_0, Q6_K repacked, or F32, F16,
 * BF16 as stored) in device memory and is decoded in the kernels' load path;
 * x and y are f32. One token runs the decode form (a matrix-vector product
 * bound by HBM), more tokens the prefill form (a tiled matrix product). The
 * embedding gather decodes table rows through the same formats.
 *
 * What each part replaces in the reference (paths relative to its root):
 *   charlotte_hip_matmul_desc       kernels::MatmulLaunch  src/core/kernels/matmul/matmul.h:602-632
 *   charlotte_hip_matmul_member     a member weight's piece and rows, the Matmul
 *                                   constants' members     src/core/kernels/matmul/matmul.wgsl:22-38,
 *                                                          matmul.cpp:39-52
 *   charlotte_hip_matmul_split_gate kernels::SplitGate     matmul.h:634-646
 *   charlotte_hip_matmul_launch     kernels::matmul_launches + Program::run
 *                                                          matmul.h:661-673, src/core/kernels/program.h:271-318
 *   charlotte_hip_matmul_plan_launch kernels::matmul_launches alone: the launch's plan, pure, no
 *                                   device               matmul.h:661-673, src/core/kernels/interface.h:29-34
 *   charlotte_hip_matmul_desc.row_divisor  kernels::Launch::row_divisor  interface.h:270-279, 292
 *   charlotte_hip_matmul_split_tokens / _range_sum_floats  matmul.h:648-659, matmul.cpp:233-250
 *   charlotte_hip_matmul_weight_*   residency::WeightView/WeightPiece + PieceWriter
 *                                                          src/core/residency/weight_view.h:28-53,
 *                                                          src/core/residency/piece_writer.cpp:194-205
 *   charlotte_hip_matmul_lay_out    formats::DeviceLayout   src/core/formats/device_layout.h:95-136
 *   charlotte_hip_matmul_repack_q6_k formats::detail::repack_q6_k
 *                                                          src/core/formats/q6_k/q6_k_repack.cpp:52-87
 *   charlotte_hip_matmul_status     kernels::ProgramError  src/core/kernels/program.h:159-169
 *   charlotte_hip_matmul_gguf_*     gguf::read_index, gguf::TensorEntry, gguf::ReadError
 *                                                          src/core/gguf/reader.h:14-29, types.h:112-141, 191-243
 *   charlotte_hip_matmul_gather     kernels::gather_launches + Program::run
 *                                                          src/core/kernels/gather/gather.h:126-136, gather.wgsl:21-58
 *   charlotte_hip_matmul_gather_positions
 *                                   kernels::position_launch  gather.h:138-145, gather.wgsl:65-84
 *
 * Conventions: every function returns a status and never throws; a failure
 * names its subject in charlotte_hip_matmul_last_error(ctx). A context owns
 * one device; calls on one context come from one host thread. Launches are
 * asynchronous and ordered on the stream given (a hipStream_t passed as
 * void*, NULL for the null stream); the caller owns inputs and outputs, which
 * are borrowed until the stream reaches the launch. No launch allocates.
 *
 * Order of addition (determinism, batch invariance): every path but the
 * matrix-core prefill and the INT8_LIMBS decode (both opt-in, within
 * tolerance, never chosen by default; below) adds each output's products in the reference's one
 * order, fixed by K alone (matmul.h:34-50): a row's G = K / 32 groups cut into
 * 32 ranges, range r groups floor(rG/32) .. floor((r+1)G/32), each range an
 * fma chain from zero in k order, the 32 range sums added in order to a total
 * from zero. So a token's outputs are the same bits decoded alone or
 * prefilled in a step of any size, and the same bits as the CPU restatement
 * of that order.
 */
#ifndef CHARLOTTE_HIP_MATMUL_H
#define CHARLOTTE_HIP_MATMUL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* kernels::ProgramError (program.h:159-169) and the launcher's
 * preconditions (matmul.h:661-671), as codes. */
typedef enum {
    CHARLOTTE_HIP_MATMUL_OK = 0,
    CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT = 1,  /* a null, a size or a pointer the operation cannot take */
    CHARLOTTE_HIP_MATMUL_UNSUPPORTED_TYPE = 2,  /* a GGUF type this library has no kernels for */
    CHARLOTTE_HIP_MATMUL_SHAPE_NOT_GROUPS = 3,  /* K not whole 32-weight groups, or a tensor not whole blocks */
    CHARLOTTE_HIP_MATMUL_OUT_OF_MEMORY = 4,
    CHARLOTTE_HIP_MATMUL_HIP_ERROR = 5,         /* the HIP runtime refused a call; its message is in last_error */
    CHARLOTTE_HIP_MATMUL_NO_DEVICE = 6,
    CHARLOTTE_HIP_MATMUL_UNSUPPORTED = 7,       /* an epilogue, option or combination not built */
    CHARLOTTE_HIP_MATMUL_BAD_FILE = 8,          /* a GGUF file that fails validation: see read_error */
    CHARLOTTE_HIP_MATMUL_IO_ERROR = 9           /* a file that cannot be opened or mapped */
} charlotte_hip_matmul_status;

/* GGUF tensor types the kernels read (src/core/gguf/types.h:39-47): the
 * reference's format table, every row (src/core/capability/capability.cpp:57-65).
 * The products and the gather read all seven; the matrix-core prefill the
 * four quantized ones. */
enum {
    CHARLOTTE_HIP_MATMUL_F32 = 0,
    CHARLOTTE_HIP_MATMUL_F16 = 1,
    CHARLOTTE_HIP_MATMUL_Q4_0 = 2,
    CHARLOTTE_HIP_MATMUL_Q4_1 = 3,
    CHARLOTTE_HIP_MATMUL_Q8_0 = 8,
    CHARLOTTE_HIP_MATMUL_Q6_K = 14,
    CHARLOTTE_HIP_MATMUL_BF16 = 30
};

/* kernels::Epilogue (matmul.h:594-599). */
typedef enum {
    CHARLOTTE_HIP_MATMUL_WRITE = 0,
    CHARLOTTE_HIP_MATMUL_QKV = 1,
    CHARLOTTE_HIP_MATMUL_GATED_ACTIVATION = 2,
    CHARLOTTE_HIP_MATMUL_GATED_BY_INPUT = 3
} charlotte_hip_matmul_epilogue;

/* model::FeedForwardActivation, as the launcher passes it (matmul.cpp:62-69). */
typedef enum {
    CHARLOTTE_HIP_MATMUL_SILU = 0,
    CHARLOTTE_HIP_MATMUL_GELU_TANH = 1,
    CHARLOTTE_HIP_MATMUL_SIGMOID = 2
} charlotte_hip_matmul_activation;

/* kernels::Rows (src/core/kernels/interface.h:212-215). */
typedef enum {
    CHARLOTTE_HIP_MATMUL_EVERY_TOKEN = 0,
    CHARLOTTE_HIP_MATMUL_LAST_TOKEN = 1  /* the head: the step's last token alone, y written as one row */
} charlotte_hip_matmul_rows;

/* Which prefill kernel runs (no counterpart: the reference has one, on WebGPU's
 * shader cores). AUTO, the default, CANONICAL and EXACT_MFMA add in the
 * order above (split along K where the gate and the caller's range sums
 * allow), bit-exact and batch-invariant: a drop-in caller keeps the
 * reference's decode = prefill guarantee whatever workspace it sets. For a
 * step that does not split, AUTO takes the matrix cores' K = 1 f32
 * instruction (GEMM_EXACT: each range's chain one fused multiply-add a k, as
 * the VALU tile adds it, on 64-row waves) where the step gives it at least
 * three waves a compute unit; else the same chains split among a workgroup's
 * waves (GEMM_EXACT_SHORT: 32 rows by 32 tokens, or 16 by 16 where the larger
 * tiles would leave compute units idle, eight waves of four ranges, the range
 * sums combined in LDS). A step that splits runs its chunks of
 * ranges on the matrix-core chains under AUTO and EXACT_MFMA
 * (GEMM_EXACT_SPLIT), on the 128-row VALU tile under CANONICAL (GEMM_SPLIT);
 * the same range sums, the same combine. CANONICAL keeps to the VALU: the
 * 128-row tile, or the short-step tile (GEMM_SHORT: 16 or 8 rows by 32
 * tokens, K split among a workgroup's waves) where the 128-row tiles would
 * number fewer than the compute units. EXACT_MFMA always GEMM_EXACT. All
 * three give the same bits.
 * SPLIT_F16_MFMA, only when asked for, runs the products on the matrix cores
 * with x split into two f16 parts, within the tolerance max|err| / max|y| <=
 * 1e-5 but not bit-exact and not batch-invariant with decode; it needs a
 * workspace (below) and reads the quantized formats only. */
typedef enum {
    CHARLOTTE_HIP_MATMUL_GEMM_AUTO = 0,
    CHARLOTTE_HIP_MATMUL_GEMM_CANONICAL = 1,
    CHARLOTTE_HIP_MATMUL_GEMM_SPLIT_F16_MFMA = 2,
    CHARLOTTE_HIP_MATMUL_GEMM_EXACT_MFMA = 3
} charlotte_hip_matmul_gemm_path;

/* Which decode kernel runs (no counterpart: the reference decodes in its one
 * order). CANONICAL, the default, adds in the order above, bit-exact and
 * batch-invariant. INT8_LIMBS splits x, a 32-weight group at a time, into a
 * 22-bit fixed-point value (the group's max |x| sets the exponent) cut into
 * three int8 limbs, and sums code x limb products exactly in int32 on the dot
 * instructions, 16 weights at a time, before the scales and an f32 sum:
 * within max|err| / max|y| <= 1e-5 of the canonical order, not its bits, and
 * not batch-invariant with prefill; a non-finite input makes the outputs NaN.
 * It is built for the shapes of the streamed decodes: Q6_K at K = 1,024 or
 * 1,152 with each member's rows and first row multiples of 16, K = 2,048
 * with multiples of 8; Q4_0 at K = 1,024 or 2,048 in products of 2^20
 * groups or more, rows and first rows multiples of 16 or 8; any epilogue
 * but the gated one. Every other decode runs CANONICAL whatever the
 * setting. */
typedef enum {
    CHARLOTTE_HIP_MATMUL_GEMV_CANONICAL = 0,
    CHARLOTTE_HIP_MATMUL_GEMV_INT8_LIMBS = 1
} charlotte_hip_matmul_gemv_path;

typedef struct charlotte_hip_matmul_context charlotte_hip_matmul_context;
typedef struct charlotte_hip_matmul_weight charlotte_hip_matmul_weight;

/* ---- context ---------------------------------------------------------- */

charlotte_hip_matmul_status charlotte_hip_matmul_context_create(int device, charlotte_hip_matmul_context** out);
charlotte_hip_matmul_status charlotte_hip_matmul_context_destroy(charlotte_hip_matmul_context* ctx);
/* The last failure's message, naming its subject; "" after success. Owned by ctx. */
const char* charlotte_hip_matmul_last_error(const charlotte_hip_matmul_context* ctx);
charlotte_hip_matmul_status charlotte_hip_matmul_set_gemm_path(charlotte_hip_matmul_context* ctx,
                                                               charlotte_hip_matmul_gemm_path path);
charlotte_hip_matmul_status charlotte_hip_matmul_set_gemv_path(charlotte_hip_matmul_context* ctx,
                                                               charlotte_hip_matmul_gemv_path path);

/* The matrix-core prefill's working memory (no counterpart in the reference,
 * whose one prefill kernel needs none): the step's input split into two
 * binary16 parts, 4 bytes a weight column a token plus a scale a token,
 * tokens rounded up to 64. The caller allocates it and owns it; launches on
 * the context use it until it is set again (NULL, 0 unsets it), so steps that
 * use it must be ordered on one stream. Only SPLIT_F16_MFMA uses it; a step
 * it does not hold is refused with INVALID_ARGUMENT. */
charlotte_hip_matmul_status charlotte_hip_matmul_set_workspace(charlotte_hip_matmul_context* ctx, void* device,
                                                               uint64_t bytes);
/* Bytes the workspace needs for a step of `tokens` tokens of K = `columns`;
 * 0 when columns are not whole 32-weight groups. */
uint64_t charlotte_hip_matmul_workspace_bytes(uint32_t tokens, uint64_t columns);

/* ---- device layout (host only; no device needed) ---------------------------- */

/* Bytes of the device layout of `rows` x `columns` weights of `gguf_type`:
 * the stored bytes rounded up to 4 (device_layout.h:59-63). 0 when the type is
 * not one of the above or the shape is not whole blocks. */
uint64_t charlotte_hip_matmul_layout_bytes(uint32_t gguf_type, uint64_t rows, uint64_t columns);
/* File-order blocks -> the piece's streams, in host memory: Q4_0 and Q8_0 as
 * their codes then their scales, Q4_1 as its codes then its d and m words
 * (device_layout.h:121-123), Q6_K repacked, then its lo, hi, scales and d
 * streams (device_layout.h:124-127, q6_k.h:11-21), F32 as stored. `device`
 * holds layout_bytes(...) bytes. */
charlotte_hip_matmul_status charlotte_hip_matmul_lay_out(uint32_t gguf_type, const void* stored_blocks,
                                                         uint64_t blocks, void* device);
/* The Q6_K repack alone, block i's stream s at streams[s] + i * width(s),
 * widths 128, 64, 16, 2 (q6_k_repack.cpp:52-87). */
charlotte_hip_matmul_status charlotte_hip_matmul_repack_q6_k(const void* stored_blocks, uint64_t blocks,
                                                             void* const streams[4]);

/* ---- weights ------------------------------------------------------------ */

/* A weight of `rows` rows of `columns` (K) in the device layout, owned by the
 * library: the stored blocks (file order, `bytes` of them) laid out and copied
 * to the device. Rows need not be whole Q6_K super-blocks (Gemma 3's 1,152);
 * the tensor must be. Synchronous. */
charlotte_hip_matmul_status charlotte_hip_matmul_weight_upload(charlotte_hip_matmul_context* ctx,
                                                               uint32_t gguf_type, uint64_t rows,
                                                               uint64_t columns, const void* stored_blocks,
                                                               uint64_t bytes, charlotte_hip_matmul_weight** out);
/* A weight whose piece the caller already wrote in the device layout at
 * `device_piece` (16-byte aligned), as the reference's PieceWriter writes a
 * piece; borrowed, never freed by the library. */
charlotte_hip_matmul_status charlotte_hip_matmul_weight_wrap(charlotte_hip_matmul_context* ctx,
                                                             uint32_t gguf_type, uint64_t rows, uint64_t columns,
                                                             const void* device_piece, uint64_t bytes,
                                                             charlotte_hip_matmul_weight** out);
/* A weight of a shape and format with no device memory: a residency::WeightView
 * before upload (weight_view.h:28-53), for plans only. A launch refuses it. */
charlotte_hip_matmul_status charlotte_hip_matmul_weight_shape(uint32_t gguf_type, uint64_t rows, uint64_t columns,
                                                              charlotte_hip_matmul_weight** out);
charlotte_hip_matmul_status charlotte_hip_matmul_weight_free(charlotte_hip_matmul_weight* weight);
/* The weight's piece on the device (its first stream's first byte). */
const void* charlotte_hip_matmul_weight_device(const charlotte_hip_matmul_weight* weight);

/* ---- the product ------------------------------------------------------- */

/* One member of a product: rows row_offset .. row_offset + rows - 1 of
 * `weight`, the product's next `rows` outputs.
 *   WRITE, GATED_BY_INPUT: output index of the member's first row is
 *     output_row (a piece's first_row, matmul.cpp:283-291), in a row of
 *     desc.out_width outputs a token.
 *   QKV: members Q, K, V write outputs[0], [1], [2], each `rows` wide a token
 *     (matmul.wgsl:298-314); output_row is ignored.
 *   GATED_ACTIVATION: members gate then up, equal rows; row_offset is each
 *     member's first row within its weight — for a GLU over one weight's
 *     halves, gate {w, half, half} and up {w, 0, half} (matmul.cpp:270-279). */
typedef struct {
    const charlotte_hip_matmul_weight* weight;
    uint64_t row_offset;
    uint64_t rows;
    uint64_t output_row;
} charlotte_hip_matmul_member;

typedef struct {
    charlotte_hip_matmul_member members[3];
    uint32_t member_count;            /* 1, 2 or 3; members share K */
    uint32_t epilogue;                /* charlotte_hip_matmul_epilogue */
    uint32_t activation;              /* charlotte_hip_matmul_activation (gated epilogues, `activated`) */
    uint32_t rows;                    /* charlotte_hip_matmul_rows */
    const float* input;               /* device: tokens rows of K floats */
    float* outputs[3];                /* device: WRITE/GATED* use outputs[0]; QKV all three */
    uint64_t out_width;               /* floats a token's output row (WRITE/GATED_BY_INPUT; 0 = product rows) */
    /* GATED_BY_INPUT: output o of token t times u[t * stride + column + o]. */
    const float* gate_input;
    uint32_t gate_input_stride;
    uint32_t gate_input_column;
    /* Options (matmul.h:229-255). `clip`: the four bounds in_min, in_max,
     * out_min, out_max, each a device pointer to its own F32 word — the
     * reference keeps them as four scalars beside the weight and reads each
     * by its own word offset into the product's span (Constants.clip, a
     * vec4<u32> of first words, matmul.h:275-277, matmul.cpp:280-281), so
     * each pointer is that span's base plus 4 x its word; all four NULL for
     * an unclipped product (any other mix is refused). Each bound is read on
     * the device, never on the host. `bias` device floats, one an output
     * row, or NULL (WRITE); `activated` nonzero applies `activation` last
     * (WRITE). */
    const float* clip[4];
    const float* bias;
    uint32_t activated;
    /* kernels::Launch::row_divisor (interface.h:270-279): the launch's rows
     * are the step's tokens over this, rounded down (matmul.wgsl:87-91) — a
     * vision encoder's projection after pooling, its patches over k². 0 and
     * 1 both mean every token (a zero-initialised descriptor is undivided).
     * Not with LAST_TOKEN (program.cpp:382-387). A step of fewer tokens than
     * the divisor launches nothing. */
    uint32_t row_divisor;
} charlotte_hip_matmul_desc;

/* kernels::SplitGate: the tiled prefill splits along K when its workgroups W
 * satisfy W * denominator <= G * numerator and W <= max_workgroups. */
typedef struct {
    uint32_t numerator;
    uint32_t denominator;
    uint32_t max_workgroups;
} charlotte_hip_matmul_split_gate;

/* One product over a step of `tokens` tokens (1 decodes; more prefill), on
 * `stream`. `range_sums` is the split's working buffer (device, bytes), or
 * NULL/0: a step splits only while its range sums fit it (matmul.cpp:166-172). */
charlotte_hip_matmul_status charlotte_hip_matmul_launch(charlotte_hip_matmul_context* ctx,
                                                        const charlotte_hip_matmul_desc* desc,
                                                        charlotte_hip_matmul_split_gate gate, void* range_sums,
                                                        uint64_t range_sums_bytes, uint32_t tokens, void* stream);

/* ---- the launch's plan, without a device ------------------------------------ */

/* Which kernel a launch runs (plan.kernel). */
typedef enum {
    CHARLOTTE_HIP_MATMUL_KERNEL_NONE = 0,          /* nothing runs: a divided step of fewer tokens than the divisor */
    CHARLOTTE_HIP_MATMUL_KERNEL_GEMV_RANGES = 1,   /* decode, 32 lanes a row, lane r range r (matmul.wgsl:207-243) */
    CHARLOTTE_HIP_MATMUL_KERNEL_GEMV_QUARTERS = 2, /* decode, 4 lanes a row of 9 groups each (K = 1,152) */
    CHARLOTTE_HIP_MATMUL_KERNEL_GEMV_STREAM = 3,   /* decode, Q6_K at K = 1,152 streamed through LDS */
    CHARLOTTE_HIP_MATMUL_KERNEL_GEMV_STREAM8 = 4,  /* decode, Q6_K at K = 1,024 or 2,048 streamed through LDS */
    CHARLOTTE_HIP_MATMUL_KERNEL_GEMV_CHUNKED = 5,  /* decode past K = 8,192 (GEMV_WIDE aside): x staged a chunk at a time */
    CHARLOTTE_HIP_MATMUL_KERNEL_GEMV_STREAM4 = 6,  /* decode, Q4_0 at K = 1,024 .. 8,192 (powers of two) streamed through LDS */
    CHARLOTTE_HIP_MATMUL_KERNEL_GEMV_WIDE = 7,     /* decode, Q4_0 at K = 9,216 .. 16,384 (whole 1,024s) streamed through LDS */
    CHARLOTTE_HIP_MATMUL_KERNEL_GEMM_TILED = 16,   /* prefill, the VALU tile */
    CHARLOTTE_HIP_MATMUL_KERNEL_GEMM_SPLIT = 17,   /* prefill split along K, then the ordered combine */
    CHARLOTTE_HIP_MATMUL_KERNEL_GEMM_MFMA = 18,    /* prefill on the matrix cores (x split into two f16 parts) */
    CHARLOTTE_HIP_MATMUL_KERNEL_GEMM_SHORT = 19,   /* prefill of a short step: 16 or 8 rows x 32 tokens, K split in the workgroup */
    CHARLOTTE_HIP_MATMUL_KERNEL_GEMM_EXACT = 20,   /* prefill on the matrix cores' f32 fused multiply-add, the canonical order */
    CHARLOTTE_HIP_MATMUL_KERNEL_GEMM_EXACT_SPLIT = 21, /* the same split along K, then the ordered combine */
    CHARLOTTE_HIP_MATMUL_KERNEL_GEMM_EXACT_SHORT = 22  /* a short step on the matrix cores: 32 x 32 or 16 x 16 tiles, K split in the workgroup */
} charlotte_hip_matmul_kernel;

/* What a plan is made for: the device's compute units (256 on MI355X) and
 * the settings a context would hold. */
typedef struct {
    uint32_t compute_units;
    uint32_t gemm_path;         /* charlotte_hip_matmul_gemm_path */
    uint32_t gemv_path;         /* charlotte_hip_matmul_gemv_path */
    uint32_t reserved;          /* 0 */
    uint64_t workspace_bytes;   /* the matrix-core workspace set, 0 for none */
} charlotte_hip_matmul_target;

typedef struct {
    uint32_t kernel;            /* charlotte_hip_matmul_kernel */
    uint32_t launches;          /* kernel launches: 0, 1, or 2 (split + combine; matrix cores: x's split + product) */
    uint32_t canonical;         /* nonzero: the reference's order of addition — bit-exact, batch-invariant */
    uint32_t rows;              /* input and output rows of the launch: tokens / row_divisor, or 1 (LAST_TOKEN, decode) */
    uint32_t lanes_a_row;       /* decode: lanes a product row */
    uint32_t groups_a_lane;     /* decode: the most 32-weight groups a lane holds (the kernel's) */
    uint32_t steps_a_wave;      /* decode: row steps a wave takes a tile */
    uint32_t tile_tokens;       /* prefill: tokens a workgroup's tile (decode: 1) */
    uint32_t tile_rows;         /* product rows a workgroup's tile */
    uint32_t chunks;            /* the split along K: workgroups a tile (else 1) */
    uint64_t tiles;             /* tiles of the main kernel */
    uint64_t workgroups;        /* its grid; the persistent decode kernels run at most this, each looping over tiles */
} charlotte_hip_matmul_plan;

/* The plan charlotte_hip_matmul_launch would follow for `desc` over a step of
 * `tokens`, with `range_sums_bytes` of range sums, on `target` — and the
 * status it would return for the descriptor, before any device work: the
 * same checks, in the same order. Pure: no device, no allocation; the
 * members' weights may be shape-only (charlotte_hip_matmul_weight_shape) or
 * uploaded. A failure writes its message into `message` (up to
 * `message_bytes`, NUL-terminated) when given. */
charlotte_hip_matmul_status charlotte_hip_matmul_plan_launch(const charlotte_hip_matmul_desc* desc,
                                                             const charlotte_hip_matmul_target* target,
                                                             charlotte_hip_matmul_split_gate gate,
                                                             uint64_t range_sums_bytes, uint32_t tokens,
                                                             charlotte_hip_matmul_plan* out, char* message,
                                                             uint64_t message_bytes);

/* The allocation-free launch. No counterpart in the reference: for callers
 * that cannot allocate device memory — code under HIP graph capture, tight
 * serving loops, harnesses that forbid it. charlotte_hip_matmul_launch with
 * the split's range sums taken from the library's own static array, one a
 * device of CHARLOTTE_HIP_MATMUL_STATIC_SCRATCH_BYTES, held from the
 * library's load on the device until the process ends, in place of the
 * caller's buffer. It allocates nothing and frees nothing. It plans as the
 * ordinary launch plans with a range-sums buffer of the array's size: a step
 * the gate would split whose range sums (4 x 32 x tokens x rows bytes) pass
 * the array runs the tiled form, whose bits are the split's; every step runs
 * with the ordinary launch's bits. Every call on one GPU shares that
 * GPU's array and leaves its contents behind (nothing in it must start at
 * zero): calls that overlap on one GPU — on two streams, or from two
 * threads — race. */
#define CHARLOTTE_HIP_MATMUL_STATIC_SCRATCH_BYTES (16u * 1024u * 1024u)
charlotte_hip_matmul_status charlotte_hip_matmul_launch_static(charlotte_hip_matmul_context* ctx,
                                                               const charlotte_hip_matmul_desc* desc,
                                                               charlotte_hip_matmul_split_gate gate, uint32_t tokens,
                                                               void* stream);

/* matmul.h:648-659: the most tokens a step may hold for the product to split,
 * a whole number of 32-token tiles up to 512, or 1 when it never splits; and
 * the floats range_sums must hold for it. */
uint32_t charlotte_hip_matmul_split_tokens(uint32_t epilogue, uint64_t rows, uint64_t columns,
                                           charlotte_hip_matmul_split_gate gate);
uint64_t charlotte_hip_matmul_range_sum_floats(uint32_t epilogue, uint64_t rows, uint64_t columns,
                                               charlotte_hip_matmul_split_gate gate);

/* ---- the embedding gather (src/core/kernels/gather/gather.h) ------------------- */

/* Each token of a step becomes its row of the token embedding table, decoded
 * and multiplied by `scale`, in `hidden` (gather.wgsl:21-58). `table` is a
 * piece of the table holding vocabulary rows first_row .. first_row +
 * table rows - 1, in any format above; a table split into pieces takes one
 * call a piece, each writing the rows whose token it holds and leaving the
 * others as they are. With scale 1 every weight is the format's decode bit
 * for bit; with another, the decoded weight times the scale, rounded once
 * (llama.cpp's decode-then-scale). */
typedef struct {
    const charlotte_hip_matmul_weight* table;
    uint64_t first_row;
    const uint32_t* ids;   /* device: the step's `tokens` identifiers (unread when fed) */
    /* device or NULL: a fed step's draw record (sampler.h); its first word is
     * every row's token in place of ids, never compared with media_token */
    const uint32_t* fed;
    uint32_t media;        /* nonzero: a row whose identifier is media_token is left as it is */
    uint32_t media_token;
    float scale;
    float* hidden;         /* device, 16-byte aligned: tokens rows of the table's columns floats */
} charlotte_hip_matmul_gather_desc;

charlotte_hip_matmul_status charlotte_hip_matmul_gather(charlotte_hip_matmul_context* ctx,
                                                        const charlotte_hip_matmul_gather_desc* desc,
                                                        uint32_t tokens, void* stream);

/* The position form (gather.wgsl:65-84): patch row r of a vision step, at
 * column x = r % grid_columns and row y = r / grid_columns of its grid, is
 * the table's row x plus its row positions + y, written to `output`. `table`
 * is F32 of 2 x positions rows; grid_columns <= positions and tokens <=
 * grid_columns * positions. */
charlotte_hip_matmul_status charlotte_hip_matmul_gather_positions(charlotte_hip_matmul_context* ctx,
                                                                  const charlotte_hip_matmul_weight* table,
                                                                  uint32_t positions, uint32_t grid_columns,
                                                                  uint32_t tokens, float* output, void* stream);

/* ---- GGUF files (gguf::read_index, src/core/gguf/reader.cpp) -------------------- */

/* A GGUF v3 file's tensor index: every tensor's name, format, shape and
 * absolute byte range, validated against the file (a defined format whose
 * blocks tile a row, offsets aligned to general.alignment, ranges inside the
 * file and disjoint, names unique and at most 64 bytes, ...). A file that
 * fails returns BAD_FILE and sets *read_error to the reference's ReadError
 * number (src/core/gguf/types.h:112-141); charlotte_hip_matmul_gguf_error_string
 * names it. Host only. */
typedef struct charlotte_hip_matmul_gguf charlotte_hip_matmul_gguf;

typedef struct {
    const char* name;           /* owned by the file handle */
    uint32_t gguf_type;
    uint32_t dimension_count;
    uint64_t dimensions[4];     /* dimensions[0]: a row's length (K) */
    uint64_t element_count;
    uint64_t offset;            /* absolute, in the file */
    uint64_t bytes;
} charlotte_hip_matmul_gguf_tensor;

/* The file at `path`, mapped read-only until closed. */
charlotte_hip_matmul_status charlotte_hip_matmul_gguf_open(const char* path, charlotte_hip_matmul_gguf** out,
                                                           uint32_t* read_error);
/* The same over `size` bytes in memory, borrowed until closed. */
charlotte_hip_matmul_status charlotte_hip_matmul_gguf_read(const void* bytes, uint64_t size,
                                                           charlotte_hip_matmul_gguf** out, uint32_t* read_error);
const char* charlotte_hip_matmul_gguf_error_string(uint32_t read_error);
charlotte_hip_matmul_status charlotte_hip_matmul_gguf_close(charlotte_hip_matmul_gguf* file);
uint64_t charlotte_hip_matmul_gguf_tensor_count(const charlotte_hip_matmul_gguf* file);
charlotte_hip_matmul_status charlotte_hip_matmul_gguf_tensor_at(const charlotte_hip_matmul_gguf* file, uint64_t index,
                                                                charlotte_hip_matmul_gguf_tensor* out);
/* A tensor's index by name, or -1. */
int64_t charlotte_hip_matmul_gguf_find(const charlotte_hip_matmul_gguf* file, const char* name);
/* The file's first byte (tensor bytes are at their offsets from it). */
const void* charlotte_hip_matmul_gguf_bytes(const charlotte_hip_matmul_gguf* file);
/* Tensor `index` as a weight on ctx's device: its blocks laid out as
 * charlotte_hip_matmul_weight_upload lays them out, rows = element_count /
 * dimensions[0], columns = dimensions[0]. UNSUPPORTED_TYPE for a format the
 * kernels do not read. */
charlotte_hip_matmul_status charlotte_hip_matmul_gguf_upload(charlotte_hip_matmul_context* ctx,
                                                             const charlotte_hip_matmul_gguf* file, uint64_t index,
                                                             charlotte_hip_matmul_weight** out);

#ifdef __cplusplus
}
#endif
#endif
