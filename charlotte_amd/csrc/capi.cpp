// The C ABI (include/charlotte_hip_matmul.h): contexts, weights in the device
// layout, and each product's launches — the roles of the reference's
// kernels::matmul_launches (src/core/kernels/matmul/matmul.cpp:252-325) and
// Program::run (src/core/kernels/program.cpp:601-760), for HIP. Nothing here
// throws across the ABI; every failure is a status and a message.
#include "charlotte_hip_matmul.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "gather.hpp"
#include "gguf.hpp"
#include "layout.hpp"
#include "plan.hpp"
#include "product.hpp"

// The allocation-free launch's range sums (charlotte_hip_matmul_launch_static):
// one array a device, in the code object, held from the library's load on
// that device until the process ends. Host code never uses this name as an
// address: each device's copy is found with hipGetSymbolAddress (below) and
// kept per device.
static __device__ __align__(256) float scratch[CHARLOTTE_HIP_MATMUL_STATIC_SCRATCH_BYTES / sizeof(float)];

struct charlotte_hip_matmul_context {
    int device = 0;
    uint32_t compute_units = 0;
    float* scratch = nullptr;   // this device's copy of `scratch`
    charlotte_hip_matmul_gemm_path gemm_path = CHARLOTTE_HIP_MATMUL_GEMM_AUTO;
    charlotte_hip_matmul_gemv_path gemv_path = CHARLOTTE_HIP_MATMUL_GEMV_CANONICAL;
    void* workspace = nullptr;  // the matrix-core path's, the caller's memory
    uint64_t workspace_bytes = 0;
    std::string error;
};

struct charlotte_hip_matmul_gguf {
    chm::GgufFile file;
};

struct charlotte_hip_matmul_weight {
    charlotte_hip_matmul_context* ctx = nullptr;
    uint32_t type = 0;
    uint64_t rows = 0, columns = 0, blocks = 0, bytes = 0;
    uint8_t* piece = nullptr;
    bool owned = false;
};

namespace {

using Status = charlotte_hip_matmul_status;

Status fail(charlotte_hip_matmul_context* ctx, Status s, const std::string& message) {
    if (ctx) ctx->error = message;
    return s;
}

Status ok(charlotte_hip_matmul_context* ctx) {
    if (ctx) ctx->error.clear();
    return CHARLOTTE_HIP_MATMUL_OK;
}

Status hip_fail(charlotte_hip_matmul_context* ctx, hipError_t e, const char* what) {
    return fail(ctx, e == hipErrorOutOfMemory ? CHARLOTTE_HIP_MATMUL_OUT_OF_MEMORY : CHARLOTTE_HIP_MATMUL_HIP_ERROR,
                std::string(what) + ": " + hipGetErrorString(e));
}

// The formats a weight may hold: the reference's format table
// (capability.cpp:57-65). The products and the gather read them all.
bool known(uint32_t type) {
    return type == CHARLOTTE_HIP_MATMUL_F32 || type == CHARLOTTE_HIP_MATMUL_F16 || type == CHARLOTTE_HIP_MATMUL_BF16 ||
           type == CHARLOTTE_HIP_MATMUL_Q4_0 || type == CHARLOTTE_HIP_MATMUL_Q4_1 ||
           type == CHARLOTTE_HIP_MATMUL_Q8_0 || type == CHARLOTTE_HIP_MATMUL_Q6_K;
}

// The shape checks of a weight: rows of whole 32-weight groups
// (matmul.h:668-671, format.h:138-160) in a tensor of whole blocks.
Status check_shape(charlotte_hip_matmul_context* ctx, uint32_t type, uint64_t rows, uint64_t columns) {
    if (!known(type)) return fail(ctx, CHARLOTTE_HIP_MATMUL_UNSUPPORTED_TYPE, "weight: GGUF type " + std::to_string(type));
    if (rows == 0 || columns == 0) return fail(ctx, CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT, "weight: no rows or columns");
    if (columns % 32 != 0)
        return fail(ctx, CHARLOTTE_HIP_MATMUL_SHAPE_NOT_GROUPS,
                    "weight: " + std::to_string(columns) + " columns are not whole 32-weight groups");
    // Bounded first, so rows x columns (below 2^61) cannot wrap.
    if (rows > 0xFFFFFFFFull || columns / 32 > 0xFFFFFFull)
        return fail(ctx, CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT, "weight: too many rows or columns");
    if ((rows * columns) % chm::block_weights_host(type) != 0)
        return fail(ctx, CHARLOTTE_HIP_MATMUL_SHAPE_NOT_GROUPS, "weight: not a whole number of blocks");
    return CHARLOTTE_HIP_MATMUL_OK;
}

// kernels_matmul split geometry (matmul.cpp:26-37, 233-250; plan.h:113).
constexpr uint32_t kTileOutputs = 64, kTileTokens = 32, kPrefillBlock = 512;

uint32_t split_tokens_of(uint32_t epilogue, uint64_t rows, uint64_t columns, charlotte_hip_matmul_split_gate gate) {
    if (epilogue == CHARLOTTE_HIP_MATMUL_GATED_ACTIVATION || gate.denominator == 0 || rows == 0) return 1;
    const uint64_t groups = columns / 32;
    const uint64_t out_tiles = (rows + kTileOutputs - 1) / kTileOutputs;
    const uint64_t by_ratio = groups * gate.numerator / (uint64_t{gate.denominator} * out_tiles);
    const uint64_t by_cap = gate.max_workgroups / out_tiles;
    const uint64_t token_tiles = std::min(by_ratio, by_cap);
    if (token_tiles == 0) return 1;
    return static_cast<uint32_t>(std::min<uint64_t>(token_tiles * kTileTokens, kPrefillBlock));
}

// What a launch is planned for beyond its descriptor.
struct Target {
    uint32_t compute_units;
    uint32_t gemm_path, gemv_path;
    uint64_t workspace_bytes;
};

// A failed check: its status and its message.
struct Verdict {
    Status status = CHARLOTTE_HIP_MATMUL_OK;
    std::string message;
    bool ok() const { return status == CHARLOTTE_HIP_MATMUL_OK; }
};

Verdict refuse(Status s, std::string message) { return {s, std::move(message)}; }

// A launch's checks and the product its kernels receive, on the host alone:
// the reference's preconditions (matmul.h:661-671) and this library's. Every
// sum is taken in 64 bits and every value narrowed to a kernel's 32 is
// checked first, so no descriptor can wrap past a check into an access
// outside a weight or an output. `ctx` is the launching context, or null for
// a plan, which also takes shape-only weights.
Verdict describe(const charlotte_hip_matmul_desc* desc, uint32_t tokens, const charlotte_hip_matmul_context* ctx,
                 chm::Product* out, uint32_t* format) {
    const auto bad = [](std::string m) { return refuse(CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT, "launch: " + m); };
    if (!desc) return bad("no descriptor");
    if (tokens == 0) return bad("a step of no tokens");
    const charlotte_hip_matmul_desc& d = *desc;
    if (d.member_count < 1 || d.member_count > 3) return bad("member_count " + std::to_string(d.member_count));
    if (d.epilogue > CHARLOTTE_HIP_MATMUL_GATED_BY_INPUT) return bad("epilogue " + std::to_string(d.epilogue));
    if (d.rows > CHARLOTTE_HIP_MATMUL_LAST_TOKEN) return bad("rows " + std::to_string(d.rows));
    if (d.activation > CHARLOTTE_HIP_MATMUL_SIGMOID) return bad("activation " + std::to_string(d.activation));
    const uint32_t divisor = d.row_divisor ? d.row_divisor : 1;
    // program.cpp:382-387: a divided launch is never over the last token.
    if (divisor != 1 && d.rows == CHARLOTTE_HIP_MATMUL_LAST_TOKEN) return bad("a row divisor over the last token");
    const bool gated = d.epilogue == CHARLOTTE_HIP_MATMUL_GATED_ACTIVATION;
    const bool by_input = d.epilogue == CHARLOTTE_HIP_MATMUL_GATED_BY_INPUT;
    // The options are a Write's; a gated product may be clipped (matmul.h:229-255, 623-629).
    if ((d.bias || d.activated) && d.epilogue != CHARLOTTE_HIP_MATMUL_WRITE)
        return bad("bias and activated are a Write's options");
    // The four bounds come together (matmul.cpp:280-281 sets all four words
    // or none), each a 4-byte word of its own.
    const bool clip = d.clip[0] || d.clip[1] || d.clip[2] || d.clip[3];
    if (clip && !(d.clip[0] && d.clip[1] && d.clip[2] && d.clip[3]))
        return bad("clip takes its four bounds or none");
    for (const float* bound : d.clip)
        if (reinterpret_cast<uintptr_t>(bound) % 4 != 0) return bad("a clip bound not 4-byte aligned");
    if (clip && d.epilogue != CHARLOTTE_HIP_MATMUL_WRITE && !gated)
        return bad("clip is a Write's or a gated product's option");
    if (gated && d.member_count != 2) return bad("a gated product takes two members, gate and up");
    if (gated && d.members[0].rows != d.members[1].rows) return bad("gate and up rows differ");
    if (by_input && !d.gate_input) return bad("GatedByInput without its input");
    if (!d.input) return bad("no input");
    if (reinterpret_cast<uintptr_t>(d.input) % 16 != 0) return bad("input not 16-byte aligned");
    if (d.out_width > 0xFFFFFFFFull) return bad("out_width past 2^32");

    chm::Product a{};
    const charlotte_hip_matmul_weight* head = d.members[0].weight;
    if (!head) return bad("member 0 has no weight");
    if (!known(head->type))
        return refuse(CHARLOTTE_HIP_MATMUL_UNSUPPORTED_TYPE, "launch: GGUF type " + std::to_string(head->type));
    uint64_t rows = 0;
    for (uint32_t i = 0; i < d.member_count; ++i) {
        const charlotte_hip_matmul_member& m = d.members[i];
        const std::string who = "member " + std::to_string(i);
        if (!m.weight) return bad(who + " has no weight");
        if (ctx && !m.weight->piece) return bad(who + " is a shape-only weight");
        if (ctx && m.weight->ctx != ctx) return bad(who + " of another context");
        if (m.weight->type != head->type || m.weight->columns != head->columns)
            return bad("members differ in format or width");
        if (m.rows == 0 || m.row_offset > m.weight->rows || m.rows > m.weight->rows - m.row_offset)
            return bad(who + " rows past its weight");
        if (m.output_row > 0xFFFFFFFFull) return bad(who + " output_row past 2^32");
        float* o = d.epilogue == CHARLOTTE_HIP_MATMUL_QKV ? d.outputs[i] : d.outputs[0];
        if (!o) return bad(who + " has no output");
        // Weights hold at most 2^32 - 1 rows (check_shape), so each value
        // below fits 32 bits; `rows` is at most three of them.
        a.m[i] = chm::Member{m.weight->piece,
                             m.weight->blocks,
                             static_cast<uint32_t>(m.row_offset),
                             static_cast<uint32_t>(m.rows),
                             static_cast<uint32_t>(std::min<uint64_t>(rows, 0xFFFFFFFFull)),
                             static_cast<uint32_t>(m.output_row),
                             static_cast<uint32_t>(d.out_width),
                             0,
                             o};
        rows += m.rows;
    }
    if (rows > 0x7FFFFFFFull) return bad("too many rows");
    // A gated product writes its gate's rows a token; the rest, out_width
    // (0: the product's rows) with each member at its output_row.
    const uint64_t width = gated ? d.members[0].rows : rows;
    for (uint32_t i = 0; i < d.member_count; ++i) {
        if (a.m[i].out_width == 0) a.m[i].out_width = static_cast<uint32_t>(width);
        if (gated && a.m[i].out_width < width) return bad("out_width below the gate's rows");
        if ((d.epilogue == CHARLOTTE_HIP_MATMUL_WRITE || by_input) &&
            uint64_t{a.m[i].out_row} + a.m[i].rows > a.m[i].out_width)
            return bad("output rows past out_width");
    }
    a.x = d.input;
    a.members = d.member_count;
    a.rows = static_cast<uint32_t>(rows);
    a.groups = static_cast<uint32_t>(head->columns / 32);
    a.epilogue = d.epilogue;
    a.activation = d.activation;
    a.last_token = d.rows == CHARLOTTE_HIP_MATMUL_LAST_TOKEN;
    a.tokens = tokens / divisor;  // the launch's rows (matmul.wgsl:87-91)
    a.gate_stride = d.gate_input_stride;
    a.gate_column = d.gate_input_column;
    a.gate_input = d.gate_input;
    for (int i = 0; i < 4; ++i) a.clip[i] = d.clip[i];
    a.bias = d.bias;
    a.activated = d.activated ? 1u : 0u;
    *out = a;
    *format = head->type;
    return {};
}

// The kernel a described product runs on `t`, and its shape: decode for one
// token or the head's last; else the split along K when the gate allows the
// step and its range sums fit `range_sums_bytes` (a product with options, or
// gated, never splits: matmul.cpp:166-172, 233-241); else a tile in the
// canonical order (AUTO and EXACT_MFMA: the matrix cores' fused multiply-add,
// whole or split in the workgroup for a short step; CANONICAL: the 128-row
// VALU tile or the VALU short-step tile), or the split-f16 matrix cores when
// the target asks for them.
Verdict plan_product(const chm::Product& a, uint32_t format, const Target& t, charlotte_hip_matmul_split_gate gate,
                     uint64_t range_sums_bytes, chm::Plan* plan) {
    *plan = chm::Plan{};
    if (a.tokens == 0) return {};  // a divided step of fewer tokens than the divisor: nothing runs
    if (a.tokens == 1 || a.last_token) {
        if (!chm::plan_gemv(a, format, t.compute_units, t.gemv_path == CHARLOTTE_HIP_MATMUL_GEMV_INT8_LIMBS, plan))
            return refuse(CHARLOTTE_HIP_MATMUL_UNSUPPORTED, "launch: no decode kernel takes the product");
        return {};
    }
    if (t.gemm_path == CHARLOTTE_HIP_MATMUL_GEMM_SPLIT_F16_MFMA) {
        if (!chm::mfma_reads(format))
            return refuse(CHARLOTTE_HIP_MATMUL_UNSUPPORTED,
                          "launch: the matrix-core prefill reads Q4_0, Q4_1, Q8_0 and Q6_K, not GGUF type " +
                              std::to_string(format));
        const uint64_t need = chm::mfma_workspace_bytes(a.tokens, a.groups);
        if (t.workspace_bytes < need)
            return refuse(CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT,
                          "launch: the matrix-core path needs a workspace of " + std::to_string(need) + " bytes");
        chm::plan_gemm_mfma(a, format, t.compute_units, plan);
        return {};
    }
    bool split = false;
    const bool options = chm::clipped(a) || a.bias || a.activated;
    if (!options && a.epilogue != chm::kGated && range_sums_bytes && gate.denominator) {
        const uint64_t fits = range_sums_bytes / 4 / (uint64_t{a.rows} * 32);
        const uint64_t most = std::min<uint64_t>(split_tokens_of(a.epilogue, a.rows, uint64_t{a.groups} * 32, gate), fits);
        split = a.tokens <= most;
    }
    chm::plan_gemm_canonical(a, t.compute_units, split, plan);
    if (t.gemm_path == CHARLOTTE_HIP_MATMUL_GEMM_CANONICAL) {
        // the VALU tiles: the short-step tile where the 128-row tiles would
        // be fewer than the compute units
        if (!split && plan->tiles < t.compute_units) chm::plan_gemm_short(a, t.compute_units, plan);
        return {};
    }
    if (split) {
        // the split on the matrix cores' fused multiply-add: the same range
        // sums, the same combine
        chm::plan_gemm_exact(a, format, t.compute_units, true, plan);
        return {};
    }
    chm::Plan exact;
    chm::plan_gemm_exact(a, format, t.compute_units, false, &exact);
    // AUTO: the matrix cores' fused multiply-add tile where the step gives it
    // at least three waves a compute unit (at fewer each of its waves' walk
    // through K is the step's time: measured slower than the short-step tile
    // at 640 waves on 256 compute units, 91 against 79 us at 2,560 x 2,048 x
    // 512 tokens, faster at 768, 53 against 58 us at 3,072 x 1,024 x 512);
    // else the short-step form on the matrix cores, K split among a
    // workgroup's waves (measured faster than the VALU short-step tile at
    // every short step tried). The same bits whichever runs.
    const uint64_t exact_waves = uint64_t{(a.rows + 63) / 64} * exact.token_tiles;
    if (t.gemm_path == CHARLOTTE_HIP_MATMUL_GEMM_EXACT_MFMA || exact_waves >= 3ull * t.compute_units)
        *plan = exact;
    else
        chm::plan_gemm_exact_short(a, t.compute_units, plan);
    return {};
}

}  // namespace

extern "C" {

// Device `device`'s address of `scratch`, found once (with the device
// current) and kept; later contexts on the device reuse it.
static hipError_t scratch_of(int device, float** out) {
    constexpr int kDevices = 64;
    static std::mutex lock;
    static float* found[kDevices] = {};
    if (device < 0 || device >= kDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> hold(lock);
    if (!found[device]) {
        int previous = 0;
        if (hipError_t e = hipGetDevice(&previous); e != hipSuccess) return e;
        if (hipError_t e = hipSetDevice(device); e != hipSuccess) return e;
        void* at = nullptr;
        const hipError_t e = hipGetSymbolAddress(&at, HIP_SYMBOL(scratch));
        (void)hipSetDevice(previous);
        if (e != hipSuccess) return e;
        if (!at) return hipErrorInvalidSymbol;
        found[device] = static_cast<float*>(at);
    }
    *out = found[device];
    return hipSuccess;
}

charlotte_hip_matmul_status charlotte_hip_matmul_context_create(int device, charlotte_hip_matmul_context** out) {
    if (!out) return CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT;
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count == 0) return CHARLOTTE_HIP_MATMUL_NO_DEVICE;
    if (device < 0 || device >= count) return CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) return CHARLOTTE_HIP_MATMUL_HIP_ERROR;
    float* device_scratch = nullptr;
    if (scratch_of(device, &device_scratch) != hipSuccess) return CHARLOTTE_HIP_MATMUL_HIP_ERROR;
    auto* ctx = new (std::nothrow) charlotte_hip_matmul_context;
    if (!ctx) return CHARLOTTE_HIP_MATMUL_OUT_OF_MEMORY;
    ctx->device = device;
    ctx->compute_units = static_cast<uint32_t>(prop.multiProcessorCount);
    ctx->scratch = device_scratch;
    *out = ctx;
    return CHARLOTTE_HIP_MATMUL_OK;
}

charlotte_hip_matmul_status charlotte_hip_matmul_context_destroy(charlotte_hip_matmul_context* ctx) {
    delete ctx;
    return CHARLOTTE_HIP_MATMUL_OK;
}

const char* charlotte_hip_matmul_last_error(const charlotte_hip_matmul_context* ctx) {
    return ctx ? ctx->error.c_str() : "no context";
}

charlotte_hip_matmul_status charlotte_hip_matmul_set_gemm_path(charlotte_hip_matmul_context* ctx,
                                                               charlotte_hip_matmul_gemm_path path) {
    if (!ctx) return CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT;
    if (path != CHARLOTTE_HIP_MATMUL_GEMM_AUTO && path != CHARLOTTE_HIP_MATMUL_GEMM_CANONICAL &&
        path != CHARLOTTE_HIP_MATMUL_GEMM_SPLIT_F16_MFMA && path != CHARLOTTE_HIP_MATMUL_GEMM_EXACT_MFMA)
        return fail(ctx, CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT, "gemm path: " + std::to_string(path));
    ctx->gemm_path = path;
    return ok(ctx);
}

charlotte_hip_matmul_status charlotte_hip_matmul_set_gemv_path(charlotte_hip_matmul_context* ctx,
                                                               charlotte_hip_matmul_gemv_path path) {
    if (!ctx) return CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT;
    if (path != CHARLOTTE_HIP_MATMUL_GEMV_CANONICAL && path != CHARLOTTE_HIP_MATMUL_GEMV_INT8_LIMBS)
        return fail(ctx, CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT, "gemv path: " + std::to_string(path));
    ctx->gemv_path = path;
    return ok(ctx);
}

charlotte_hip_matmul_status charlotte_hip_matmul_set_workspace(charlotte_hip_matmul_context* ctx, void* device,
                                                               uint64_t bytes) {
    if (!ctx) return CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT;
    if (device && reinterpret_cast<uintptr_t>(device) % 16 != 0)
        return fail(ctx, CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT, "workspace: not 16-byte aligned");
    ctx->workspace = bytes ? device : nullptr;
    ctx->workspace_bytes = device ? bytes : 0;
    return ok(ctx);
}

uint64_t charlotte_hip_matmul_workspace_bytes(uint32_t tokens, uint64_t columns) {
    if (tokens == 0 || columns == 0 || columns % 32 != 0 || columns / 32 > 0xFFFFFFull) return 0;
    return chm::mfma_workspace_bytes(tokens, static_cast<uint32_t>(columns / 32));
}

uint64_t charlotte_hip_matmul_layout_bytes(uint32_t gguf_type, uint64_t rows, uint64_t columns) {
    if (check_shape(nullptr, gguf_type, rows, columns) != CHARLOTTE_HIP_MATMUL_OK) return 0;
    return chm::layout_bytes(gguf_type, rows * columns / chm::block_weights_host(gguf_type));
}

charlotte_hip_matmul_status charlotte_hip_matmul_lay_out(uint32_t gguf_type, const void* stored_blocks,
                                                         uint64_t blocks, void* device) {
    if (!known(gguf_type)) return CHARLOTTE_HIP_MATMUL_UNSUPPORTED_TYPE;
    if ((!stored_blocks || !device) && blocks != 0) return CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT;
    if (blocks == 0) return CHARLOTTE_HIP_MATMUL_OK;
    return chm::lay_out(gguf_type, static_cast<const uint8_t*>(stored_blocks), blocks, static_cast<uint8_t*>(device))
               ? CHARLOTTE_HIP_MATMUL_OK
               : CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT;
}

charlotte_hip_matmul_status charlotte_hip_matmul_repack_q6_k(const void* stored_blocks, uint64_t blocks,
                                                             void* const streams[4]) {
    if (blocks == 0) return CHARLOTTE_HIP_MATMUL_OK;
    if (!stored_blocks || !streams || !streams[0] || !streams[1] || !streams[2] || !streams[3])
        return CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT;
    chm::repack_q6_k(static_cast<const uint8_t*>(stored_blocks), blocks, static_cast<uint8_t*>(streams[0]),
                     static_cast<uint8_t*>(streams[1]), static_cast<uint8_t*>(streams[2]),
                     static_cast<uint8_t*>(streams[3]));
    return CHARLOTTE_HIP_MATMUL_OK;
}

charlotte_hip_matmul_status charlotte_hip_matmul_weight_upload(charlotte_hip_matmul_context* ctx,
                                                               uint32_t gguf_type, uint64_t rows,
                                                               uint64_t columns, const void* stored_blocks,
                                                               uint64_t bytes, charlotte_hip_matmul_weight** out) {
    if (!ctx || !out || !stored_blocks) return fail(ctx, CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT, "weight upload: null argument");
    *out = nullptr;
    if (Status s = check_shape(ctx, gguf_type, rows, columns); s != CHARLOTTE_HIP_MATMUL_OK) return s;
    const uint64_t blocks = rows * columns / chm::block_weights_host(gguf_type);
    if (bytes != blocks * chm::block_bytes_host(gguf_type))
        return fail(ctx, CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT,
                    "weight upload: " + std::to_string(bytes) + " bytes for " + std::to_string(blocks) + " blocks");
    const uint64_t device_bytes = chm::layout_bytes(gguf_type, blocks);
    std::vector<uint8_t> host;
    try {
        host.resize(device_bytes);
    } catch (const std::bad_alloc&) {
        return fail(ctx, CHARLOTTE_HIP_MATMUL_OUT_OF_MEMORY, "weight upload: host staging");
    }
    chm::lay_out(gguf_type, static_cast<const uint8_t*>(stored_blocks), blocks, host.data());
    if (hipError_t e = hipSetDevice(ctx->device); e != hipSuccess) return hip_fail(ctx, e, "weight upload: hipSetDevice");
    void* dev = nullptr;
    if (hipError_t e = hipMalloc(&dev, device_bytes); e != hipSuccess) return hip_fail(ctx, e, "weight upload: hipMalloc");
    if (hipError_t e = hipMemcpy(dev, host.data(), device_bytes, hipMemcpyHostToDevice); e != hipSuccess) {
        (void)hipFree(dev);
        return hip_fail(ctx, e, "weight upload: hipMemcpy");
    }
    auto* w = new (std::nothrow) charlotte_hip_matmul_weight;
    if (!w) {
        (void)hipFree(dev);
        return fail(ctx, CHARLOTTE_HIP_MATMUL_OUT_OF_MEMORY, "weight upload");
    }
    *w = {ctx, gguf_type, rows, columns, blocks, device_bytes, static_cast<uint8_t*>(dev), true};
    *out = w;
    return ok(ctx);
}

charlotte_hip_matmul_status charlotte_hip_matmul_weight_wrap(charlotte_hip_matmul_context* ctx, uint32_t gguf_type,
                                                             uint64_t rows, uint64_t columns, const void* device_piece,
                                                             uint64_t bytes, charlotte_hip_matmul_weight** out) {
    if (!ctx || !out || !device_piece) return fail(ctx, CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT, "weight wrap: null argument");
    *out = nullptr;
    if (Status s = check_shape(ctx, gguf_type, rows, columns); s != CHARLOTTE_HIP_MATMUL_OK) return s;
    const uint64_t blocks = rows * columns / chm::block_weights_host(gguf_type);
    if (bytes < chm::layout_bytes(gguf_type, blocks))
        return fail(ctx, CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT, "weight wrap: piece shorter than its layout");
    if (reinterpret_cast<uintptr_t>(device_piece) % 16 != 0)
        return fail(ctx, CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT, "weight wrap: piece not 16-byte aligned");
    auto* w = new (std::nothrow) charlotte_hip_matmul_weight;
    if (!w) return fail(ctx, CHARLOTTE_HIP_MATMUL_OUT_OF_MEMORY, "weight wrap");
    *w = {ctx, gguf_type, rows, columns, blocks, bytes,
          const_cast<uint8_t*>(static_cast<const uint8_t*>(device_piece)), false};
    *out = w;
    return ok(ctx);
}

charlotte_hip_matmul_status charlotte_hip_matmul_weight_shape(uint32_t gguf_type, uint64_t rows, uint64_t columns,
                                                              charlotte_hip_matmul_weight** out) {
    if (!out) return CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT;
    *out = nullptr;
    if (Status s = check_shape(nullptr, gguf_type, rows, columns); s != CHARLOTTE_HIP_MATMUL_OK) return s;
    auto* w = new (std::nothrow) charlotte_hip_matmul_weight;
    if (!w) return CHARLOTTE_HIP_MATMUL_OUT_OF_MEMORY;
    const uint64_t blocks = rows * columns / chm::block_weights_host(gguf_type);
    *w = {nullptr, gguf_type, rows, columns, blocks, chm::layout_bytes(gguf_type, blocks), nullptr, false};
    *out = w;
    return CHARLOTTE_HIP_MATMUL_OK;
}

charlotte_hip_matmul_status charlotte_hip_matmul_weight_free(charlotte_hip_matmul_weight* weight) {
    if (!weight) return CHARLOTTE_HIP_MATMUL_OK;
    Status s = CHARLOTTE_HIP_MATMUL_OK;
    if (weight->owned && weight->piece) {
        (void)hipSetDevice(weight->ctx->device);
        if (hipFree(weight->piece) != hipSuccess) s = CHARLOTTE_HIP_MATMUL_HIP_ERROR;
    }
    delete weight;
    return s;
}

const void* charlotte_hip_matmul_weight_device(const charlotte_hip_matmul_weight* weight) {
    return weight ? weight->piece : nullptr;
}

uint32_t charlotte_hip_matmul_split_tokens(uint32_t epilogue, uint64_t rows, uint64_t columns,
                                           charlotte_hip_matmul_split_gate gate) {
    return split_tokens_of(epilogue, rows, columns, gate);
}

uint64_t charlotte_hip_matmul_range_sum_floats(uint32_t epilogue, uint64_t rows, uint64_t columns,
                                               charlotte_hip_matmul_split_gate gate) {
    const uint32_t split = split_tokens_of(epilogue, rows, columns, gate);
    return split < 2 ? 0 : uint64_t{split} * rows * 32;
}

charlotte_hip_matmul_status charlotte_hip_matmul_plan_launch(const charlotte_hip_matmul_desc* desc,
                                                             const charlotte_hip_matmul_target* target,
                                                             charlotte_hip_matmul_split_gate gate,
                                                             uint64_t range_sums_bytes, uint32_t tokens,
                                                             charlotte_hip_matmul_plan* out, char* message,
                                                             uint64_t message_bytes) {
    if (message && message_bytes) message[0] = 0;
    if (!target || !out || target->compute_units == 0) return CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT;
    *out = charlotte_hip_matmul_plan{};
    chm::Product a{};
    uint32_t format = 0;
    Verdict v = describe(desc, tokens, nullptr, &a, &format);
    chm::Plan plan;
    if (v.ok())
        v = plan_product(a, format, Target{target->compute_units, target->gemm_path, target->gemv_path,
                                           target->workspace_bytes},
                         gate, range_sums_bytes, &plan);
    if (!v.ok()) {
        if (message && message_bytes) {
            const size_t n = std::min<uint64_t>(v.message.size(), message_bytes - 1);
            std::memcpy(message, v.message.data(), n);
            message[n] = 0;
        }
        return v.status;
    }
    out->kernel = plan.kernel;
    out->launches = plan.launches;
    out->canonical = plan.canonical ? 1u : 0u;
    out->rows = a.last_token ? 1u : a.tokens;
    out->lanes_a_row = plan.lanes;
    out->groups_a_lane = plan.span;
    out->steps_a_wave = plan.steps;
    out->tile_tokens = plan.tile_tokens;
    out->tile_rows = plan.tile_rows;
    out->chunks = plan.chunks;
    out->tiles = plan.tiles;
    out->workgroups = plan.workgroups;
    return CHARLOTTE_HIP_MATMUL_OK;
}

// Runs a planned product on ctx's device; `range_sums` serves a split plan.
// No allocation: every buffer is the caller's or the library's static one.
static Status run_plan(charlotte_hip_matmul_context* ctx, const chm::Product& a, uint32_t format, const chm::Plan& plan,
                       float* range_sums, void* stream) {
    if (plan.kernel == chm::kNoKernel) return ok(ctx);
    if (hipError_t e = hipSetDevice(ctx->device); e != hipSuccess) return hip_fail(ctx, e, "launch: hipSetDevice");
    auto* s = static_cast<hipStream_t>(stream);
    hipError_t e;
    switch (plan.kernel) {
        case chm::kGemmMfma: e = chm::launch_gemm_mfma(a, format, plan, ctx->workspace, s); break;
        case chm::kGemmTiled: e = chm::launch_gemm_canonical(a, format, plan, nullptr, s); break;
        case chm::kGemmShort: e = chm::launch_gemm_short(a, format, plan, s); break;
        case chm::kGemmExact: e = chm::launch_gemm_exact(a, format, plan, nullptr, s); break;
        case chm::kGemmExactSplit: e = chm::launch_gemm_exact(a, format, plan, range_sums, s); break;
        case chm::kGemmExactShort: e = chm::launch_gemm_exact_short(a, format, plan, s); break;
        case chm::kGemmSplit: e = chm::launch_gemm_canonical(a, format, plan, range_sums, s); break;
        default: e = chm::launch_gemv(a, format, plan, ctx->compute_units, s); break;
    }
    if (e != hipSuccess) return hip_fail(ctx, e, "launch");
    return ok(ctx);
}

static Target target_of(const charlotte_hip_matmul_context* ctx) {
    return Target{ctx->compute_units, ctx->gemm_path, ctx->gemv_path, ctx->workspace ? ctx->workspace_bytes : 0};
}

charlotte_hip_matmul_status charlotte_hip_matmul_launch(charlotte_hip_matmul_context* ctx,
                                                        const charlotte_hip_matmul_desc* desc,
                                                        charlotte_hip_matmul_split_gate gate, void* range_sums,
                                                        uint64_t range_sums_bytes, uint32_t tokens, void* stream) {
    if (!ctx) return CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT;
    chm::Product a{};
    uint32_t format = 0;
    Verdict v = describe(desc, tokens, ctx, &a, &format);
    chm::Plan plan;
    if (v.ok()) v = plan_product(a, format, target_of(ctx), gate, range_sums ? range_sums_bytes : 0, &plan);
    if (!v.ok()) return fail(ctx, v.status, v.message);
    if ((plan.kernel == chm::kGemmSplit || plan.kernel == chm::kGemmExactSplit) &&
        reinterpret_cast<uintptr_t>(range_sums) % 4 != 0)
        return fail(ctx, CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT, "launch: range_sums not 4-byte aligned");
    return run_plan(ctx, a, format, plan, static_cast<float*>(range_sums), stream);
}

charlotte_hip_matmul_status charlotte_hip_matmul_launch_static(charlotte_hip_matmul_context* ctx,
                                                               const charlotte_hip_matmul_desc* desc,
                                                               charlotte_hip_matmul_split_gate gate, uint32_t tokens,
                                                               void* stream) {
    if (!ctx) return CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT;
    chm::Product a{};
    uint32_t format = 0;
    Verdict v = describe(desc, tokens, ctx, &a, &format);
    chm::Plan plan;
    // Planned as the ordinary launch plans with a buffer of the static
    // array's size: a step whose range sums would not fit it runs the tiled
    // form, whose bits are the split's (the same order of addition).
    if (v.ok())
        v = plan_product(a, format, target_of(ctx), gate, CHARLOTTE_HIP_MATMUL_STATIC_SCRATCH_BYTES, &plan);
    if (!v.ok()) return fail(ctx, v.status, v.message);
    return run_plan(ctx, a, format, plan, ctx->scratch, stream);
}

charlotte_hip_matmul_status charlotte_hip_matmul_gather(charlotte_hip_matmul_context* ctx,
                                                        const charlotte_hip_matmul_gather_desc* desc,
                                                        uint32_t tokens, void* stream) {
    if (!ctx) return CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT;
    if (!desc) return fail(ctx, CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT, "gather: no descriptor");
    const charlotte_hip_matmul_gather_desc& d = *desc;
    const charlotte_hip_matmul_weight* t = d.table;
    if (!t) return fail(ctx, CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT, "gather: no table");
    if (t->ctx != ctx) return fail(ctx, CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT, "gather: a table of another context");
    if (tokens == 0) return fail(ctx, CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT, "gather: a step of no tokens");
    if (!d.fed && !d.ids) return fail(ctx, CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT, "gather: no identifiers");
    if (!d.hidden || reinterpret_cast<uintptr_t>(d.hidden) % 16 != 0)
        return fail(ctx, CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT, "gather: hidden missing or not 16-byte aligned");
    if (d.first_row + t->rows > 0x100000000ull)
        return fail(ctx, CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT, "gather: rows past 2^32");
    if (static_cast<uint64_t>(tokens) * (t->columns / 32) * 8 > 0xFFFFFFFFull * 256)
        return fail(ctx, CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT, "gather: too many rows a step");
    chm::Gather g{};
    g.piece = t->piece;
    g.blocks = t->blocks;
    g.ids = d.ids;
    g.fed = d.fed;
    g.hidden = d.hidden;
    g.tokens = tokens;
    g.groups = static_cast<uint32_t>(t->columns / 32);
    g.first_row = static_cast<uint32_t>(d.first_row);
    g.row_count = static_cast<uint32_t>(t->rows);
    g.media = d.media ? 1u : 0u;
    g.media_token = d.media_token;
    g.scale = d.scale;
    if (hipError_t e = hipSetDevice(ctx->device); e != hipSuccess) return hip_fail(ctx, e, "gather: hipSetDevice");
    if (hipError_t e = chm::launch_gather(g, t->type, static_cast<hipStream_t>(stream)); e != hipSuccess)
        return hip_fail(ctx, e, "gather");
    return ok(ctx);
}

charlotte_hip_matmul_status charlotte_hip_matmul_gather_positions(charlotte_hip_matmul_context* ctx,
                                                                  const charlotte_hip_matmul_weight* table,
                                                                  uint32_t positions, uint32_t grid_columns,
                                                                  uint32_t tokens, float* output, void* stream) {
    if (!ctx) return CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT;
    if (!table) return fail(ctx, CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT, "gather positions: no table");
    if (table->ctx != ctx)
        return fail(ctx, CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT, "gather positions: a table of another context");
    if (table->type != CHARLOTTE_HIP_MATMUL_F32)
        return fail(ctx, CHARLOTTE_HIP_MATMUL_UNSUPPORTED_TYPE, "gather positions: the table is not F32");
    if (positions == 0 || table->rows != 2ull * positions)
        return fail(ctx, CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT, "gather positions: the table is not 2 x positions rows");
    if (grid_columns == 0 || grid_columns > positions || tokens == 0 ||
        tokens > static_cast<uint64_t>(grid_columns) * positions)
        return fail(ctx, CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT, "gather positions: a grid the table does not cover");
    if (!output || reinterpret_cast<uintptr_t>(output) % 16 != 0)
        return fail(ctx, CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT, "gather positions: output missing or not 16-byte aligned");
    chm::Gather g{};
    g.piece = table->piece;
    g.blocks = table->blocks;
    g.hidden = output;
    g.tokens = tokens;
    g.groups = static_cast<uint32_t>(table->columns / 32);
    g.positions = positions;
    g.grid_columns = grid_columns;
    if (hipError_t e = hipSetDevice(ctx->device); e != hipSuccess)
        return hip_fail(ctx, e, "gather positions: hipSetDevice");
    if (hipError_t e = chm::launch_gather_positions(g, static_cast<hipStream_t>(stream)); e != hipSuccess)
        return hip_fail(ctx, e, "gather positions");
    return ok(ctx);
}

charlotte_hip_matmul_status charlotte_hip_matmul_gguf_open(const char* path, charlotte_hip_matmul_gguf** out,
                                                           uint32_t* read_error) {
    if (!path || !out) return CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT;
    *out = nullptr;
    auto* g = new (std::nothrow) charlotte_hip_matmul_gguf;
    if (!g) return CHARLOTTE_HIP_MATMUL_OUT_OF_MEMORY;
    int os_error = 0;
    const chm::GgufError e = g->file.open(path, &os_error);
    if (read_error) *read_error = static_cast<uint32_t>(e);
    if (os_error != 0) {
        delete g;
        return CHARLOTTE_HIP_MATMUL_IO_ERROR;
    }
    if (e != chm::GgufError::kOk) {
        delete g;
        return CHARLOTTE_HIP_MATMUL_BAD_FILE;
    }
    *out = g;
    return CHARLOTTE_HIP_MATMUL_OK;
}

charlotte_hip_matmul_status charlotte_hip_matmul_gguf_read(const void* bytes, uint64_t size,
                                                           charlotte_hip_matmul_gguf** out, uint32_t* read_error) {
    if (!out || (!bytes && size)) return CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT;
    *out = nullptr;
    auto* g = new (std::nothrow) charlotte_hip_matmul_gguf;
    if (!g) return CHARLOTTE_HIP_MATMUL_OUT_OF_MEMORY;
    static const uint8_t kEmpty = 0;
    const chm::GgufError e = g->file.index.read(bytes ? static_cast<const uint8_t*>(bytes) : &kEmpty, size);
    if (read_error) *read_error = static_cast<uint32_t>(e);
    if (e != chm::GgufError::kOk) {
        delete g;
        return CHARLOTTE_HIP_MATMUL_BAD_FILE;
    }
    *out = g;
    return CHARLOTTE_HIP_MATMUL_OK;
}

const char* charlotte_hip_matmul_gguf_error_string(uint32_t read_error) {
    return chm::gguf_error_string(static_cast<chm::GgufError>(read_error));
}

charlotte_hip_matmul_status charlotte_hip_matmul_gguf_close(charlotte_hip_matmul_gguf* file) {
    delete file;
    return CHARLOTTE_HIP_MATMUL_OK;
}

uint64_t charlotte_hip_matmul_gguf_tensor_count(const charlotte_hip_matmul_gguf* file) {
    return file ? file->file.index.tensors.size() : 0;
}

charlotte_hip_matmul_status charlotte_hip_matmul_gguf_tensor_at(const charlotte_hip_matmul_gguf* file, uint64_t index,
                                                                charlotte_hip_matmul_gguf_tensor* out) {
    if (!file || !out || index >= file->file.index.tensors.size()) return CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT;
    const chm::GgufTensor& t = file->file.index.tensors[index];
    out->name = t.name.c_str();
    out->gguf_type = t.type;
    out->dimension_count = t.dimension_count;
    for (int d = 0; d < 4; ++d) out->dimensions[d] = t.dimensions[d];
    out->element_count = t.elements;
    out->offset = t.offset;
    out->bytes = t.bytes;
    return CHARLOTTE_HIP_MATMUL_OK;
}

int64_t charlotte_hip_matmul_gguf_find(const charlotte_hip_matmul_gguf* file, const char* name) {
    return file && name ? file->file.index.find(name) : -1;
}

const void* charlotte_hip_matmul_gguf_bytes(const charlotte_hip_matmul_gguf* file) {
    return file ? file->file.index.bytes : nullptr;
}

charlotte_hip_matmul_status charlotte_hip_matmul_gguf_upload(charlotte_hip_matmul_context* ctx,
                                                             const charlotte_hip_matmul_gguf* file, uint64_t index,
                                                             charlotte_hip_matmul_weight** out) {
    if (!ctx) return CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT;
    if (!file || !out || index >= file->file.index.tensors.size())
        return fail(ctx, CHARLOTTE_HIP_MATMUL_INVALID_ARGUMENT, "gguf upload: no such tensor");
    const chm::GgufTensor& t = file->file.index.tensors[index];
    if (!known(t.type))
        return fail(ctx, CHARLOTTE_HIP_MATMUL_UNSUPPORTED_TYPE,
                    "gguf upload: " + t.name + " is GGUF type " + std::to_string(t.type));
    const uint64_t columns = t.dimensions[0];
    const uint64_t rows = columns ? t.elements / columns : 0;
    const charlotte_hip_matmul_status s = charlotte_hip_matmul_weight_upload(
        ctx, t.type, rows, columns, file->file.index.bytes + t.offset, t.bytes, out);
    if (s != CHARLOTTE_HIP_MATMUL_OK) ctx->error = "gguf upload of " + t.name + ": " + ctx->error;
    return s;
}

}  // extern "C"
