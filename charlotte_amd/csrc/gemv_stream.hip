// Decode of Q6_K rows of K = 1,152 (G = 36 groups) — the LM head of Gemma
// 3 1B and its QKV and output projections — streamed through LDS.
//
// The mapping is gemv_quarters' (4 lanes a row, lane j owning ranges
// 8j .. 8j + 7 = groups 9j .. 9j + 8), but the bytes arrive differently: a
// wave works 16 rows at a time (a step), and a step's four streams are
// contiguous in the piece (16 rows x 36 groups: lo 9,216 bytes, hi 4,608,
// scales 1,152, d 144 — the step starts on a super-block, 576 groups being 72
// of them). A wave copies a step into its LDS stage with
// global_load_lds_dwordx4 — 64 lanes x 16 consecutive bytes an instruction,
// whole 1 KB runs, no register waiting — then, once it has landed, reads its
// lanes' share into registers, starts the next step's copy into the same
// stage, and decodes from registers: the copy of one step runs under the
// decode of the one before. Stages are wave-private: no workgroup barrier;
// the wait for a step is one s_waitcnt on the wave's own count. Two
// workgroups of four waves a CU (two waves a SIMD) fit the LDS.
//
// x is staged once in LDS; a lane reads its slice a group at a time. A row's
// total is its 32 range sums added in order from zero: lane j holds sums
// 8j .. 8j + 7; lane 0 adds its eight to zero, passes the partial total to
// lane 1 (a quad permute), which adds its eight, and so on — the canonical
// order, so the bits are every other kernel's.
//
// The LIMBS form (the GEMV path INT8_LIMBS, limbs.hpp) streams the same
// bytes but stages x as int8 limb records and decodes a group with 24
// v_dot4_i32_i8 in place of 32 exact weights and their fma chain — about
// half the VALU work a step, which the copies feel twice: fewer instruction
// cycles, and a higher clock (the SIMDs' load throttles it). A lane's nine
// groups sum into one float from zero; the quad adds its four by two DPP
// moves. Not the canonical bits: within 1e-5 of them.
#include <algorithm>

#include "plan.hpp"
#include "product.hpp"
#include "stream.hpp"

namespace chm {

constexpr int kStreamWaves = 4;
constexpr uint32_t kStepRows = 16;
constexpr uint32_t kStepGroups = kStepRows * 36;  // 576
// A step's 16-byte chunks a stream: lo 576, hi 288, scales 72, d 9 (144
// bytes: 72 super-blocks).
constexpr uint32_t kLoChunks = kStepGroups, kHiChunks = kStepGroups / 2, kScChunks = kStepGroups / 8, kDChunks = 9;

// A lane's share of a step, as held in registers between the stage and the
// decode: its nine groups' lo and hi, their scale pairs, the two d's.
struct StepRun {
    u32x4s_t lo[9];
    u32x2s_t hi[9];
    uint32_t sc[9];
    uint32_t d_first, d_next;
};

template <bool FULL, bool LIMBS>
__global__ __launch_bounds__(256, 2) void gemv_stream(Product a, uint32_t steps, uint32_t common) {
    __shared__ u32x4s_t lo_a[kStreamWaves][kLoChunks];
    __shared__ u32x4s_t hi_a[kStreamWaves][kHiChunks];
    __shared__ u32x4s_t sc_a[kStreamWaves][kScChunks];
    __shared__ u32x4s_t d_a[kStreamWaves][kDChunks];
    // x: four slices of 72 float4 and one of padding each; or (LIMBS) four
    // slices of 9 group records and 4 dwords of padding each (the same size)
    __shared__ u32x4s_t x_stage[292];
    float4* const xs = reinterpret_cast<float4*>(x_stage);

    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: scalar branches
    const uint32_t rho = lane >> 2, j = lane & 3u;
    const uint32_t waves = gridDim.x * kStreamWaves;
    const uint32_t token = a.last_token ? a.tokens - 1 : 0;

    struct Stage {
        u32x4s_t *lo, *hi, *sc, *d;
    };
    const Stage sa{lo_a[wave], hi_a[wave], sc_a[wave], d_a[wave]};


    auto issue = [&](uint32_t step, const Stage& st) {
        u32x4s_t *lo = st.lo, *hi = st.hi, *sc = st.sc, *d = st.d;
        const Piece w = piece_of(a, step * kStepRows);
        const uint64_t n = w.blocks;
        copy_stream<kLoChunks>(w.piece + 576ull * w.row, lo, lane);
        copy_stream<kHiChunks>(w.piece + 128 * n + 288ull * w.row, hi, lane);
        copy_stream<kScChunks>(w.piece + 192 * n + 72ull * w.row, sc, lane);
        copy_stream<kDChunks>(w.piece + 208 * n + 9ull * w.row, d, lane);
    };
    const uint32_t lg = 36 * rho + 9 * j;  // the lane's first group within a step
    // The stage's reads are written as instructions the compiler does not
    // look into: it would otherwise wait for every copy in flight into any
    // stage before them (it cannot tell the two stages' copies apart across
    // the loop). The waits around them are explicit: the copies' before,
    // lgkmcnt(0) after.
    auto take = [&](StepRun& run, const Stage& st) {
        const uint32_t lo_at = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(st.lo)) + 16 * lg;
        const uint32_t hi_at = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(st.hi)) + 8 * lg;
        const uint32_t sc_at = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(st.sc)) + 2 * lg;
        const uint32_t d_at = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(st.d)) + 2 * (lg >> 3);
#define CHM_LDS_B128(dst, addr, off) \
    __asm__ __volatile__("ds_read_b128 %0, %1 offset:" #off : "=v"(dst) : "v"(addr))
#define CHM_LDS_B64(dst, addr, off) __asm__ __volatile__("ds_read_b64 %0, %1 offset:" #off : "=v"(dst) : "v"(addr))
#define CHM_LDS_U16(dst, addr, off) __asm__ __volatile__("ds_read_u16 %0, %1 offset:" #off : "=v"(dst) : "v"(addr))
        CHM_LDS_B128(run.lo[0], lo_at, 0);
        CHM_LDS_B128(run.lo[1], lo_at, 16);
        CHM_LDS_B128(run.lo[2], lo_at, 32);
        CHM_LDS_B128(run.lo[3], lo_at, 48);
        CHM_LDS_B128(run.lo[4], lo_at, 64);
        CHM_LDS_B128(run.lo[5], lo_at, 80);
        CHM_LDS_B128(run.lo[6], lo_at, 96);
        CHM_LDS_B128(run.lo[7], lo_at, 112);
        CHM_LDS_B128(run.lo[8], lo_at, 128);
        CHM_LDS_B64(run.hi[0], hi_at, 0);
        CHM_LDS_B64(run.hi[1], hi_at, 8);
        CHM_LDS_B64(run.hi[2], hi_at, 16);
        CHM_LDS_B64(run.hi[3], hi_at, 24);
        CHM_LDS_B64(run.hi[4], hi_at, 32);
        CHM_LDS_B64(run.hi[5], hi_at, 40);
        CHM_LDS_B64(run.hi[6], hi_at, 48);
        CHM_LDS_B64(run.hi[7], hi_at, 56);
        CHM_LDS_B64(run.hi[8], hi_at, 64);
        CHM_LDS_U16(run.sc[0], sc_at, 0);
        CHM_LDS_U16(run.sc[1], sc_at, 2);
        CHM_LDS_U16(run.sc[2], sc_at, 4);
        CHM_LDS_U16(run.sc[3], sc_at, 6);
        CHM_LDS_U16(run.sc[4], sc_at, 8);
        CHM_LDS_U16(run.sc[5], sc_at, 10);
        CHM_LDS_U16(run.sc[6], sc_at, 12);
        CHM_LDS_U16(run.sc[7], sc_at, 14);
        CHM_LDS_U16(run.sc[8], sc_at, 16);
        CHM_LDS_U16(run.d_first, d_at, 0);
        CHM_LDS_U16(run.d_next, d_at, 2);
        // The reads have landed before anything uses their registers: the
        // wait claims to modify every one of them, so no use can move above it.
        __asm__ __volatile__("s_waitcnt lgkmcnt(0)"
                             : "+v"(run.lo[0]), "+v"(run.lo[1]), "+v"(run.lo[2]), "+v"(run.lo[3]), "+v"(run.lo[4]),
                               "+v"(run.lo[5]), "+v"(run.lo[6]), "+v"(run.lo[7]), "+v"(run.lo[8])
                             :
                             : "memory");
        __asm__ __volatile__(""
                             : "+v"(run.hi[0]), "+v"(run.hi[1]), "+v"(run.hi[2]), "+v"(run.hi[3]), "+v"(run.hi[4]),
                               "+v"(run.hi[5]), "+v"(run.hi[6]), "+v"(run.hi[7]), "+v"(run.hi[8]));
        __asm__ __volatile__(""
                             : "+v"(run.sc[0]), "+v"(run.sc[1]), "+v"(run.sc[2]), "+v"(run.sc[3]), "+v"(run.sc[4]),
                               "+v"(run.sc[5]), "+v"(run.sc[6]), "+v"(run.sc[7]), "+v"(run.sc[8]), "+v"(run.d_first),
                               "+v"(run.d_next));
#undef CHM_LDS_B128
#undef CHM_LDS_B64
#undef CHM_LDS_U16
    };
    // One step: the lane's nine groups, its eight range sums, the row's total
    // by the quad chain, the output.
    auto decode_exact = [&](uint32_t step, const StepRun& run) {
        float sums[8];
        float s = 0.0f;
        // x a group ahead: group i + 1's words are read before group i's
        // products, so the reads' latency runs under them.
        float4 xa[2][8];
#pragma unroll
        for (int v = 0; v < 8; ++v) xa[0][v] = xs[73 * j + v];
#pragma unroll
        for (int i = 0; i < 9; ++i) {
            if (i + 1 < 9) {
#pragma unroll
                for (int v = 0; v < 8; ++v) xa[(i + 1) & 1][v] = xs[73 * j + 8 * (i + 1) + v];
            }
            float xg[32];
#pragma unroll
            for (int v = 0; v < 8; ++v) {
                const float4 q = xa[i & 1][v];
                xg[4 * v] = q.x, xg[4 * v + 1] = q.y, xg[4 * v + 2] = q.z, xg[4 * v + 3] = q.w;
            }
            const uint32_t lw[4] = {run.lo[i][0], run.lo[i][1], run.lo[i][2], run.lo[i][3]};
            const uint32_t hw[2] = {run.hi[i][0], run.hi[i][1]};
            const uint32_t dbits = ((lg + i) >> 3) == (lg >> 3) ? run.d_first : run.d_next;
            s = chain_q6_k(lw, hw, run.sc[i], dbits, xg, s);
            // Range 8j + m is group 9j + m alone for m < 7, and groups
            // 9j + 7 and 9j + 8 for m = 7 (floor(36 r / 32) at r = 8j + m):
            // the same for every lane.
            if (i < 7 || i == 8) {
                sums[i < 7 ? i : 7] = s;
                s = 0.0f;
            }
        }
        // The quad chain: total = ((0 + sums of lane 0) + sums of lane 1) ...
        float total = 0.0f;
#pragma unroll
        for (int step_lane = 0; step_lane < 4; ++step_lane) {
            float t = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, total), 0x90, 0xF, 0xF,
                                                                           false));  // quad_perm [0, 0, 1, 2]
            if (step_lane == 0) t = 0.0f;
#pragma unroll
            for (int k = 0; k < 8; ++k) t = t + sums[k];
            if (j == static_cast<uint32_t>(step_lane)) total = t;
        }
        const uint32_t p = step * kStepRows + rho;
        if (j == 3 && p < a.rows) emit<FULL>(a, p, 0, a.last_token ? a.tokens - 1 : 0, total, 0.0f);
    };
    // LIMBS: the lane's nine groups into one sum from zero, record i + 1 read
    // while group i's products run; the quad's four sums added by DPP
    // (lanes 0 + 1 and 2 + 3, then the pairs: every lane the same total).
    auto decode_limbs = [&](uint32_t step, const StepRun& run) {
        const u32x4s_t* records = x_stage + 73 * j;
        u32x4s_t g[2][8];
#pragma unroll
        for (int v = 0; v < 8; ++v) g[0][v] = records[v];
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 9; ++i) {
            if (i + 1 < 9) {
#pragma unroll
                for (int v = 0; v < 8; ++v) g[(i + 1) & 1][v] = records[8 * (i + 1) + v];
            }
            const uint32_t lw[4] = {run.lo[i][0], run.lo[i][1], run.lo[i][2], run.lo[i][3]};
            const uint32_t hw[2] = {run.hi[i][0], run.hi[i][1]};
            const uint32_t dbits = ((lg + i) >> 3) == (lg >> 3) ? run.d_first : run.d_next;
            s = group_limbs_q6_k(lw, hw, run.sc[i], half_to_float(dbits), g[i & 1], s);
        }
        float total = s + __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, s), 0xB1, 0xF, 0xF,
                                                                              false));  // quad_perm [1, 0, 3, 2]
        total = total + __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, total), 0x4E, 0xF,
                                                                           0xF, false));  // quad_perm [2, 3, 0, 1]
        const uint32_t p = step * kStepRows + rho;
        if (j == 3 && p < a.rows) emit<FULL>(a, p, 0, a.last_token ? a.tokens - 1 : 0, total, 0.0f);
    };

    // One step in flight a wave (two waves a SIMD): the next step's copy is
    // issued as soon as this one is out of the stage.
    // The first step's copy is issued before x is staged, so the two round
    // trips overlap (the barrier below waits for both).
    uint32_t step = blockIdx.x * kStreamWaves + wave;
    if (step < steps) issue(step, sa);
    // x in LDS, clamped where the product is clipped; lane j reads its slice
    // (groups 9j .. 9j + 8) a group at a time, lanes of one j the same words.
    // Slices sit 73 float4 apart, so the four a read takes start in
    // different banks.
    // The stores are written as instructions the compiler does not look
    // into: it would otherwise wait for the copy just issued before any LDS
    // store (it cannot tell x from the stage). Their wait is explicit.
    if constexpr (LIMBS) {
        // group g's record: slice g / 9, record g % 9; four lanes a group
        const uint32_t t = threadIdx.x;
        if (t < 4 * 36) {
            const uint32_t group = t >> 2, part = t & 3u;
            const float4* src =
                reinterpret_cast<const float4*>(a.x + static_cast<uint64_t>(token) * 1152 + 32 * group + 8 * part);
            const uint32_t base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(x_stage));
            stage_limbs(clamp_input(a, src[0]), clamp_input(a, src[1]), part,
                        base + 16 * (73 * (group / 9) + 8 * (group % 9)));
        }
        __asm__ __volatile__("s_waitcnt lgkmcnt(0)" ::: "memory");
        __syncthreads();
    } else {
        const float4* src = reinterpret_cast<const float4*>(a.x + static_cast<uint64_t>(token) * 1152);
        const float4 x0 = src[threadIdx.x], x1 = src[min(threadIdx.x + 256, 287u)];
        const uint32_t base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(xs));
        auto bits = [](float4 q) {
            return u32x4s_t{__float_as_uint(q.x), __float_as_uint(q.y), __float_as_uint(q.z), __float_as_uint(q.w)};
        };
        const u32x4s_t c0 = bits(clamp_input(a, x0));
        const uint32_t v0 = threadIdx.x, v1 = threadIdx.x + 256;
        __asm__ __volatile__("ds_write_b128 %0, %1" : : "v"(base + 16 * (v0 + v0 / 72)), "v"(c0));
        if (v1 < 288) {
            const u32x4s_t c1 = bits(clamp_input(a, x1));
            __asm__ __volatile__("ds_write_b128 %0, %1" : : "v"(base + 16 * (v1 + v1 / 72)), "v"(c1));
        }
        __asm__ __volatile__("s_waitcnt lgkmcnt(0)" ::: "memory");
        __syncthreads();
    }
    if (step >= steps) return;
    while (true) {
        __builtin_amdgcn_s_waitcnt(kVmcnt0);
        __asm__ __volatile__("" ::: "memory");
        StepRun run;
        take(run, sa);
        // Steps below `common` are dealt to every wave in turn; the rest to
        // the first half of the grid alone (w < waves / 2), whose waves are
        // the CUs' first workgroups: they win the SIMDs' issue arbitration
        // and finish ~15% sooner than the second ones when dealt the same.
        uint32_t next = step + waves;
        if (next >= common) {
            const uint32_t fast = waves / 2, w = blockIdx.x * kStreamWaves + wave;
            next = step < common ? (w < fast ? common + w : steps) : step + fast;
        }
        if (next < steps) issue(next, sa);
        if constexpr (LIMBS)
            decode_limbs(step, run);
        else
            decode_exact(step, run);
        if (next >= steps) break;
        step = next;
    }
}

// Whether the streamed kernel takes the product: Q6_K, K = 1,152, every
// member's rows and first row a whole number of steps (so a step lies in one
// member and starts on a super-block), and a plain or any epilogue.
bool gemv_stream_takes(const Product& a, uint32_t format) {
    if (format != kQ6_K || a.groups != 36) return false;
    for (uint32_t m = 0; m < a.members; ++m)
        if (a.m[m].rows % kStepRows != 0 || a.m[m].row_offset % kStepRows != 0) return false;
    if (a.epilogue == kGated) return false;  // gated rows interleave the members
    return true;
}

hipError_t launch_gemv_stream(const Product& a, uint32_t compute_units, bool limbs, hipStream_t stream) {
    const uint32_t steps = a.rows / kStepRows;
    const uint32_t blocks = std::min<uint32_t>(2 * compute_units, (steps + kStreamWaves - 1) / kStreamWaves);
    const bool plain = plain_epilogue(a);
    // One round's worth of steps, the last, on the first half of the grid
    // alone: C2 (8 steps a wave) 49.6 -> 48.5 and 51.0 -> 49.7 us canonical,
    // the INT8_LIMBS form unchanged (A/B on one box).
    const uint32_t waves = blocks * kStreamWaves;
    const uint32_t common = steps >= 2 * waves ? steps - waves : steps;
    if (limbs) {
        if (plain)
            hipLaunchKernelGGL((gemv_stream<false, true>), dim3(blocks), dim3(256), 0, stream, a, steps, common);
        else
            hipLaunchKernelGGL((gemv_stream<true, true>), dim3(blocks), dim3(256), 0, stream, a, steps, common);
    } else if (plain) {
        hipLaunchKernelGGL((gemv_stream<false, false>), dim3(blocks), dim3(256), 0, stream, a, steps, common);
    } else {
        hipLaunchKernelGGL((gemv_stream<true, false>), dim3(blocks), dim3(256), 0, stream, a, steps, common);
    }
    return hipGetLastError();
}

}  // namespace chm
