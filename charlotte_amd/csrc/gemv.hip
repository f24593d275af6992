// Decode: the matrix-vector product, one token, bound by reading each weight
// once from HBM. Every output in the canonical order, so its bits are the
// prefill tile's and the CPU restatement's.
//
// Mapping: L lanes a row. Lane j of a row owns ranges [32j/L, 32(j+1)/L) —
// groups [Gj/L, G(j+1)/L), at most SPAN of them — and runs each range's chain
// from zero; a wave takes 64/L rows a step and `steps` steps. L = 32 is the
// reference's mapping (matmul.wgsl:207-243): a half-wave reads a row's 32
// adjacent groups, coalesced. It balances when 32 divides G (K = 1,024,
// 2,048, 3,072); for K = 1,152 (G = 36) four ranges hold two groups and the
// rest one, so L = 32 leaves 44% of the lanes idle, and L = 4 gives every
// lane exactly 9 groups — 8 ranges, 144 contiguous code bytes.
//
// x: lane j's slice never changes, so with SPAN <= 3 groups it is loaded into
// registers once; otherwise the workgroup stages all of x in LDS once,
// interleaved by range so a half-wave's lanes read consecutive words (L = 32;
// the two half-waves read the same words: a broadcast).
// Each step loads all of its groups' bytes before decoding any, so a wave
// has a step's weights in flight at once.
// Range sums meet in LDS, 33 floats a row (padded against bank conflicts);
// then lane i adds row i's 32 sums in order from zero and writes the output.
#include <algorithm>

#include "decode.hpp"
#include "plan.hpp"
#include "product.hpp"
#include "stream.hpp"

namespace chm {

// Workgroups a CU is asked to hold at once, as launch bounds: the L = 32
// kernel's registers allow 4 waves a SIMD at SPAN <= 2 as it stands; the L = 4
// Q6_K kernel holds a 9-group run (65 registers) and spills past 128.
constexpr int kRangesMinBlocks = 2;
constexpr int kQuartersMinBlocks = 3;

constexpr int kWaves = 4;     // waves a workgroup
constexpr int kPad = 33;      // a row's 32 range sums, padded
constexpr int kRowPad = 36;   // gemv_ranges: the same, each row 16-byte aligned

constexpr int kWaveRows = 64; // rows a wave covers at most (steps * 64 / L)
constexpr uint32_t kMaxStagedK = 8192;
constexpr int kChunkGroups = 8;  // past kMaxStagedK: groups a range x is staged for at a time

// The range sums a wave writes to LDS are read back by lanes of the same wave
// only. A wave's LDS operations execute in order, so ordering the compiler's
// view of them is all that is needed: no workgroup barrier, whose fence would
// also wait for every outstanding global load.
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The outputs of a wave's rows first .. first + count - 1, lane i holding
// row first + i's total (first even, so a gated product's gate and up totals
// are adjacent lanes). Every lane of the wave calls it.
template <bool FULL>
__device__ __forceinline__ void finish_rows(const Product& a, uint32_t first, uint32_t count, float total) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t p = first + lane;
    float partner = 0.0f;
    if (FULL && a.epilogue == kGated) partner = __shfl_xor(total, 1);
    if (lane < count && p < a.rows) emit<FULL, true>(a, p, 0, a.last_token ? a.tokens - 1 : 0, total, partner);
}

// L = 32: lane r of a half-wave owns range r — at most SPAN groups, its
// chain from zero over them, and no other range; its range sum goes to LDS.
// Rows a batch: B steps' loads are issued before any is decoded, so a wave
// keeps B rows' bytes in flight rather than one; B never exceeds a wave's
// steps, so every row loaded is decoded. The unquantized formats hold 16 or
// 32 dwords a group, so fewer rows a batch keep the registers in bounds.
template <uint32_t F>
constexpr int batch_of(int span) {
    if constexpr (F == kF32) return span >= 2 ? 1 : 2;
    if constexpr (F == kF16 || F == kBF16) return span >= 3 ? 1 : span == 2 ? 2 : 4;
    return span >= 3 ? 2 : span == 2 ? 4 : 8;
}

template <uint32_t F, int SPAN, bool XREG, bool FULL, int B>
__global__ __launch_bounds__(256, kRangesMinBlocks) void gemv_ranges(Product a, uint32_t steps, uint32_t tiles) {
    // Dynamic LDS: each wave's range sums, then x when it is staged rather
    // than held in registers. A workgroup is kWaves waves, or one (small
    // products with x in registers: ranges_waves).
    extern __shared__ float4 dynamic_lds[];
    const uint32_t waves_a_block = blockDim.x >> 6;
    float* const partials = reinterpret_cast<float*>(dynamic_lds);
    float4* const xs4 = dynamic_lds + waves_a_block * (kWaveRows * kRowPad / 4);

    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t half = lane >> 5, r = lane & 31u;
    const uint32_t G = a.groups;
    const uint32_t g0 = range_lo(r, G), g1 = range_lo(r + 1, G);
    const uint32_t token = a.last_token ? a.tokens - 1 : 0;
    const float* x = a.x + static_cast<uint64_t>(token) * G * 32;

    Raw<F> raw[B][SPAN];
    // Every lane issues the same loads on every path — rows past the
    // product read its last row, groups past the lane's range the row's last
    // group, unused — so a decode waits for its own loads.
    auto load_row = [&](Raw<F> (&r)[SPAN], uint32_t wave_first, uint32_t step) {
        const uint32_t p = min(wave_first + step * 2 + half, a.rows - 1);
        const Piece w = piece_of(a, p);
        const uint64_t row0 = static_cast<uint64_t>(w.row) * G;
#pragma unroll
        for (int i = 0; i < SPAN; ++i) r[i].load(w.piece, w.blocks, row0 + min(g0 + i, G - 1));
    };
    // Staged x: the first tile's first row is issued before x is read and
    // its other rows after, so x's round trip overlaps the weights'. x in
    // registers: x's loads go out first, the rows' behind them — measured
    // faster for the small products this form serves (Q4_0 3,072 x 1,024:
    // 3.81 -> 3.53 us; the Qwen3 0.6B decode step 563 -> 496 us), where the
    // row first (x behind it), x coalesced through LDS, or every kernel
    // argument fetched in one batch of scalar loads measured no better. (The
    // grid never exceeds the tiles, so every workgroup has a first tile.)
    const uint32_t first_wave_row = (blockIdx.x * waves_a_block + wave) * steps * 2;
    if constexpr (!XREG) load_row(raw[0], first_wave_row, 0);

    float xr[XREG ? SPAN * 32 : 1];
    if constexpr (XREG) {
        // All of the slice's loads first, then the clamp where the product is
        // clipped, so the loads are in flight together.
#pragma unroll
        for (int i = 0; i < SPAN; ++i) {
            if (g0 + i < g1) {
                const float4* src = reinterpret_cast<const float4*>(x + (g0 + i) * 32);
#pragma unroll
                for (int v = 0; v < 8; ++v) {
                    const float4 q = src[v];
                    xr[i * 32 + 4 * v + 0] = q.x;
                    xr[i * 32 + 4 * v + 1] = q.y;
                    xr[i * 32 + 4 * v + 2] = q.z;
                    xr[i * 32 + 4 * v + 3] = q.w;
                }
            }
        }
        if (clipped(a)) {
            const float lo = *a.clip[0], hi = *a.clip[1];
#pragma unroll
            for (int k = 0; k < SPAN * 32; ++k) xr[k] = clamp_to(xr[k], lo, hi);
        }
    } else {
        // Staged range-interleaved: float4 v of group g0(r) + i of range r at
        // xs4[256 i + 32 v + r], so the 32 lanes of a half-wave, one a range,
        // read 32 consecutive float4 (range-major, they would all fall in the
        // same banks). Thread t stages range t % 32, float4 t / 32 of each of
        // its range's groups; every load is issued before any is stored.
        const float4* src = reinterpret_cast<const float4*>(x);
        const uint32_t sr = threadIdx.x & 31u, sv = threadIdx.x >> 5;
        const uint32_t s0 = range_lo(sr, G), s1 = range_lo(sr + 1, G);
        float4 xv[SPAN];
#pragma unroll
        for (int k = 0; k < SPAN; ++k) xv[k] = src[min(s0 + k, G - 1) * 8 + sv];
#pragma unroll
        for (int k = 0; k < SPAN; ++k)
            xs4[256 * k + threadIdx.x] = s0 + k < s1 ? clamp_input(a, xv[k]) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        __syncthreads();
    }
    if constexpr (XREG) load_row(raw[0], first_wave_row, 0);
#pragma unroll
    for (int b = 1; b < B; ++b) load_row(raw[b], first_wave_row, b);

    float* mine = partials + wave * (kWaveRows * kRowPad);
    bool loaded = true;  // the first batch already is
    for (uint32_t tile = blockIdx.x; tile < tiles; tile += gridDim.x) {
        const uint32_t wave_first = (tile * waves_a_block + wave) * steps * 2;
        for (uint32_t step0 = 0; step0 < steps; step0 += B) {
            if (!loaded) {
#pragma unroll
                for (int b = 0; b < B; ++b) load_row(raw[b], wave_first, step0 + b);
            }
            loaded = false;
#pragma unroll
            for (int b = 0; b < B; ++b) {
                const uint32_t slot = (step0 + b) * 2 + half;
                if (step0 + b >= steps) break;
                float s = 0.0f;
                if (wave_first + slot < a.rows) {
#pragma unroll
                    for (int i = 0; i < SPAN; ++i) {
                        if (g0 + i < g1) {
                            if constexpr (XREG) {
                                s = raw[b][i].chain(xr + 32 * i, s);
                            } else {
                                float xg[32];
                                const float4* src = xs4 + 256 * i + r;
#pragma unroll
                                for (int v = 0; v < 8; ++v) {
                                    const float4 q = src[32 * v];
                                    xg[4 * v] = q.x;
                                    xg[4 * v + 1] = q.y;
                                    xg[4 * v + 2] = q.z;
                                    xg[4 * v + 3] = q.w;
                                }
                                s = raw[b][i].chain(xg, s);
                            }
                        }
                    }
                }
                mine[slot * kRowPad + r] = s;  // an empty range's sum is zero
            }
        }
        wave_sync();
        float total = 0.0f;
        if (lane < steps * 2 && wave_first + lane < a.rows) total = ordered_total(mine + lane * kRowPad);
        finish_rows<FULL>(a, wave_first, steps * 2, total);
        wave_sync();  // the sums are read before the next tile writes them
    }
}

// A lane's run of SPAN groups from gi0. Q4_0 and Q6_K load a run's streams in
// few wide loads (below); Q4_1 and Q8_0 load each group as the L = 32 kernel
// does.
template <uint32_t F, int SPAN>
struct Run {
    Raw<F> g[SPAN];
    __device__ __forceinline__ void load(const uint8_t* piece, uint64_t n, uint64_t gi0) {
#pragma unroll
        for (int i = 0; i < SPAN; ++i) g[i].load(piece, n, gi0 + i);
    }
    __device__ __forceinline__ float chain(int i, uint64_t, const float* x, float s) const { return g[i].chain(x, s); }
};

template <int SPAN>
struct Run<kQ4_0, SPAN> {
    uint32_t w[SPAN][4];
    uint32_t d[SPAN];
    __device__ __forceinline__ void load(const uint8_t* piece, uint64_t n, uint64_t gi0) {
        const uint4* c = reinterpret_cast<const uint4*>(piece + 16 * gi0);
        const uint16_t* s = reinterpret_cast<const uint16_t*>(piece + 16 * n + 2 * gi0);
#pragma unroll
        for (int i = 0; i < SPAN; ++i) {
            const uint4 q = c[i];
            w[i][0] = q.x;
            w[i][1] = q.y;
            w[i][2] = q.z;
            w[i][3] = q.w;
            d[i] = s[i];
        }
    }
    __device__ __forceinline__ float chain(int i, uint64_t, const float* x, float s) const {
        return chain_q4_0(w[i], d[i], x, s);
    }
};

// Q6_K's 9 groups from a lane's run: lo, hi, scales contiguous from group gi0,
// and the two super-blocks' d the run touches (9 groups from gi0 = 9m span
// super-blocks gi0 / 8 and gi0 / 8 + 1).
template <int SPAN>
struct Run<kQ6_K, SPAN> {
    // The lane's run of SPAN groups in few wide loads:
    //   lo     SPAN 16-byte loads (16 bytes a group, 16-byte aligned);
    //   hi     8 bytes a group from an 8-byte-aligned start: the 16-byte-
    //          aligned window holding it, and its phase there (0 or 2 dwords);
    //   scales 2 bytes a group from a 2-byte-aligned start: the 8-byte-aligned
    //          window holding it, realigned once with v_alignbyte;
    //   d      the run touches super-blocks gi0 / 8 and, at most, the next
    //          (SPAN <= 9): two dwords from a 4-byte-aligned start, pulled back
    //          so they never pass the piece's end, (210 n + 3) & ~3.
    // Every read lies inside the piece's layout (its streams run on past each
    // window's slack: hi into the scales, scales into the d's).
    static_assert(SPAN <= 9, "a run spans at most two super-blocks");
    static constexpr int kHiWords = (8 * SPAN + 8 + 15) / 16 * 4;
    static constexpr int kScWords = (2 * SPAN + 6 + 7) / 8 * 2;
    static constexpr int kScAligned = (2 * SPAN + 3) / 4;
    uint32_t lo[SPAN][4];
    uint32_t hiw[kHiWords];
    uint32_t sc[kScAligned];
    uint32_t dw[2];
    uint32_t hi_phase, d_byte;
    uint64_t first_block;
    __device__ __forceinline__ void load(const uint8_t* piece, uint64_t n, uint64_t gi0) {
        const uint4* l = reinterpret_cast<const uint4*>(piece + 16 * gi0);
#pragma unroll
        for (int i = 0; i < SPAN; ++i) {
            const uint4 q = l[i];
            lo[i][0] = q.x;
            lo[i][1] = q.y;
            lo[i][2] = q.z;
            lo[i][3] = q.w;
        }
        const uint64_t hi_at = 128 * n + 8 * gi0;
        const uint4* h = reinterpret_cast<const uint4*>(piece + (hi_at & ~uint64_t{15}));
        hi_phase = static_cast<uint32_t>(hi_at & 15) >> 2;
#pragma unroll
        for (int i = 0; i < kHiWords / 4; ++i) {
            const uint4 q = h[i];
            hiw[4 * i] = q.x;
            hiw[4 * i + 1] = q.y;
            hiw[4 * i + 2] = q.z;
            hiw[4 * i + 3] = q.w;
        }
        const uint64_t sc_at = 192 * n + 2 * gi0;
        const uint2* c = reinterpret_cast<const uint2*>(piece + (sc_at & ~uint64_t{7}));
        uint32_t scw[kScWords];
#pragma unroll
        for (int i = 0; i < kScWords / 2; ++i) {
            const uint2 q = c[i];
            scw[2 * i] = q.x;
            scw[2 * i + 1] = q.y;
        }
        const uint32_t sc_byte = static_cast<uint32_t>(sc_at & 7);  // 0, 2, 4 or 6
        const bool skip = sc_byte >= 4;
#pragma unroll
        for (int k = 0; k < kScAligned; ++k) {
            const uint32_t a0 = skip ? scw[k + 1] : scw[k];
            // The last aligned dword's high half is never used; its index is
            // held inside the window.
            const uint32_t a1 = skip ? scw[k + 2 < kScWords ? k + 2 : kScWords - 1] : scw[k + 1];
            sc[k] = __builtin_amdgcn_alignbyte(a1, a0, sc_byte & 3);
        }
        first_block = gi0 / 8;
        const uint64_t d_at = 208 * n + 2 * first_block;
        const uint64_t end = (210 * n + 3) & ~uint64_t{3};
        uint64_t at = d_at & ~uint64_t{3};
        if (at + 8 > end) at = end - 8;
        const uint32_t* dp = reinterpret_cast<const uint32_t*>(piece + at);
        dw[0] = dp[0];
        dw[1] = dp[1];
        d_byte = static_cast<uint32_t>(d_at - at);
    }
    __device__ __forceinline__ float chain(int i, uint64_t gi, const float* x, float s) const {
        const uint32_t h[2] = {hi_phase == 0 ? hiw[2 * i] : hiw[2 * i + 2],
                               hi_phase == 0 ? hiw[2 * i + 1] : hiw[2 * i + 3]};
        const uint32_t scales = (sc[i >> 1] >> (16 * (i & 1))) & 0xFFFFu;
        const uint32_t byte = d_byte + 2 * static_cast<uint32_t>(gi / 8 - first_block);
        const uint64_t both = (static_cast<uint64_t>(dw[1]) << 32) | dw[0];
        const uint32_t d = static_cast<uint32_t>(both >> (8 * byte)) & 0xFFFFu;
        return chain_q6_k(lo[i], h, scales, d, x, s);
    }
};

// x in LDS for the L = 4 kernel: slice j (groups SPAN j .. SPAN j + SPAN - 1)
// at float4 SPAN 8 j + j — one float4 of padding a slice, so the 4 slices a
// read takes start in different banks.
template <int SPAN>
__device__ __forceinline__ uint32_t x_slot(uint32_t v) {
    return v + v / (8 * SPAN);
}

// L = 4: lane j of a row owns ranges 8j .. 8j + 7, exactly G / 4 = SPAN
// groups (G = 4 SPAN, G >= 32, so no range is empty). Its run's bytes are
// contiguous. (Loading the next step's runs during the current decode, two
// run buffers in turn, measured slower.)

template <uint32_t F, int SPAN, bool FULL>
__global__ __launch_bounds__(256, kQuartersMinBlocks) void gemv_quarters(Product a, uint32_t steps, uint32_t tiles) {
    __shared__ float partials[kWaves][kWaveRows * kPad];
    extern __shared__ float4 xs4[];

    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t rho = lane >> 2, j = lane & 3u;
    const uint32_t G = a.groups;
    const uint32_t g0 = SPAN * j;
    const uint32_t token = a.last_token ? a.tokens - 1 : 0;
    const float* x = a.x + static_cast<uint64_t>(token) * G * 32;

    float* mine = partials[wave];
    // Step n of this wave: tile blockIdx.x + (n / steps) gridDim.x, step n % steps.
    const uint32_t total_steps = (tiles - blockIdx.x + gridDim.x - 1) / gridDim.x * steps;
    auto row_of = [&](uint32_t n) -> uint32_t {
        const uint32_t tile = blockIdx.x + (n / steps) * gridDim.x;
        return (tile * kWaves + wave) * steps * 16 + (n % steps) * 16 + rho;
    };
    // Every step issues the same loads — a row past the product reads the
    // last row, unused — so the count of loads in flight is the same on every
    // path and a decode waits for its own step's loads only.
    auto load = [&](Run<F, SPAN>& run, uint32_t n) {
        const uint32_t p = min(row_of(n < total_steps ? n : total_steps - 1), a.rows - 1);
        const Piece w = piece_of(a, p);
        run.load(w.piece, w.blocks, static_cast<uint64_t>(w.row) * G + g0);
    };
    // The first step's run is loaded before x is staged, so the two round
    // trips overlap.
    Run<F, SPAN> first;
    load(first, 0);  // the grid never exceeds the tiles: every wave has a step
    {
        // G = 4 SPAN groups, 32 SPAN float4: a fixed count a thread, every
        // load issued before any is stored.
        constexpr int kPer = (32 * SPAN + 255) / 256;
        const float4* src = reinterpret_cast<const float4*>(x);
        float4 xv[kPer];
#pragma unroll
        for (int k = 0; k < kPer; ++k) xv[k] = src[min(threadIdx.x + 256 * k, G * 8 - 1)];
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const uint32_t v = threadIdx.x + 256 * k;
            if (v < G * 8) xs4[x_slot<SPAN>(v)] = clamp_input(a, xv[k]);
        }
    }
    const float4* xl = xs4 + x_slot<SPAN>(8 * g0);
    // Which of the run's groups end a range; the run's first range is 8j.
    uint32_t ends = 0;
#pragma unroll
    for (int i = 0; i < SPAN; ++i) {
        const uint32_t g = g0 + i;
        const uint32_t r = (32 * g + 31) / G;  // the range holding g
        if (g + 1 == range_lo(r + 1, G)) ends |= 1u << i;
    }
    __syncthreads();

    auto decode = [&](const Run<F, SPAN>& run, uint32_t n) {
        const uint32_t p = row_of(n);
        const uint32_t slot = (n % steps) * 16 + rho;
        float* sums = mine + slot * kPad;
        if (p < a.rows) {
            const uint64_t first_gi = static_cast<uint64_t>(piece_of(a, p).row) * G + g0;
            float s = 0.0f;
            uint32_t r = 8 * j;
#pragma unroll
            for (int i = 0; i < SPAN; ++i) {
                float xg[32];
#pragma unroll
                for (int v = 0; v < 8; ++v) {
                    const float4 q = xl[8 * i + v];
                    xg[4 * v] = q.x;
                    xg[4 * v + 1] = q.y;
                    xg[4 * v + 2] = q.z;
                    xg[4 * v + 3] = q.w;
                }
                s = run.chain(i, first_gi + i, xg, s);
                if (ends & (1u << i)) {
                    sums[r] = s;
                    s = 0.0f;
                    ++r;
                }
            }
        }
        if (n % steps == steps - 1) {  // a tile's last step: its rows' totals
            wave_sync();
            const uint32_t tile_first = p - slot;
            float total = 0.0f;
            if (lane < steps * 16 && tile_first + lane < a.rows) {
                const float* rs = mine + lane * kPad;
#pragma unroll
                for (int k = 0; k < 32; ++k) total = total + rs[k];
            }
            finish_rows<FULL>(a, tile_first, steps * 16, total);
            wave_sync();
        }
    };
    for (uint32_t n = 0; n < total_steps; ++n) {
        if (n > 0) load(first, n);
        decode(first, n);
    }
}

// Past K = 8,192 (a range holds more than 8 groups): x is staged in LDS 8
// groups a range at a time (32 KB, range-interleaved as gemv_ranges stages
// it), and every row of the tile continues its chain over each chunk before
// the next is staged. Lane r of a half-wave owns range r of its row; a wave
// takes STEPS steps of two rows, so a lane holds STEPS chains across the
// chunks. A chunk's groups are loaded NB at a time for every step before any
// is decoded. Range sums meet in LDS and add in order, as in gemv_ranges.
template <uint32_t F>
constexpr int chunk_batch() {
    return F == kF32 ? 1 : F == kF16 || F == kBF16 ? 2 : 4;
}

template <uint32_t F, bool FULL, int STEPS>
__global__ __launch_bounds__(256, 2) void gemv_chunked(Product a, uint32_t tiles) {
    __shared__ float partials[kWaves][kWaveRows * kPad];
    __shared__ float4 xs4[kChunkGroups * 256];
    constexpr int NB = chunk_batch<F>();

    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t half = lane >> 5, r = lane & 31u;
    const uint32_t G = a.groups;
    const uint32_t g0 = range_lo(r, G), g1 = range_lo(r + 1, G);
    const uint32_t span = (G + 31) / 32;  // the most groups a range holds
    const uint32_t token = a.last_token ? a.tokens - 1 : 0;
    const float4* x4 = reinterpret_cast<const float4*>(a.x + static_cast<uint64_t>(token) * G * 32);
    // Staging role: range sr, float4 sv of each of its groups.
    const uint32_t sr = threadIdx.x & 31u, sv = threadIdx.x >> 5;
    const uint32_t s0 = range_lo(sr, G), s1 = range_lo(sr + 1, G);
    float* mine = partials[wave];

    for (uint32_t tile = blockIdx.x; tile < tiles; tile += gridDim.x) {
        const uint32_t wave_first = (tile * kWaves + wave) * STEPS * 2;
        Piece rows[STEPS];
#pragma unroll
        for (int st = 0; st < STEPS; ++st) rows[st] = piece_of(a, min(wave_first + 2 * st + half, a.rows - 1));
        float s[STEPS];
#pragma unroll
        for (int st = 0; st < STEPS; ++st) s[st] = 0.0f;
        for (uint32_t i0 = 0; i0 < span; i0 += kChunkGroups) {
            __syncthreads();  // every lane is done with the previous chunk
            float4 xv[kChunkGroups];
#pragma unroll
            for (int k = 0; k < kChunkGroups; ++k) xv[k] = x4[min(s0 + i0 + k, G - 1) * 8 + sv];
#pragma unroll
            for (int k = 0; k < kChunkGroups; ++k)
                xs4[256 * k + threadIdx.x] =
                    s0 + i0 + k < s1 ? clamp_input(a, xv[k]) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            __syncthreads();
#pragma unroll
            for (int k0 = 0; k0 < kChunkGroups; k0 += NB) {
                Raw<F> raw[STEPS][NB];
#pragma unroll
                for (int st = 0; st < STEPS; ++st) {
                    const uint64_t row0 = static_cast<uint64_t>(rows[st].row) * G;
#pragma unroll
                    for (int k = 0; k < NB; ++k)
                        raw[st][k].load(rows[st].piece, rows[st].blocks, row0 + min(g0 + i0 + k0 + k, G - 1));
                }
#pragma unroll
                for (int k = 0; k < NB; ++k) {
                    if (g0 + i0 + k0 + k < g1) {
                        float xg[32];
                        const float4* src = xs4 + 256 * (k0 + k) + r;
#pragma unroll
                        for (int v = 0; v < 8; ++v) {
                            const float4 q = src[32 * v];
                            xg[4 * v] = q.x;
                            xg[4 * v + 1] = q.y;
                            xg[4 * v + 2] = q.z;
                            xg[4 * v + 3] = q.w;
                        }
#pragma unroll
                        for (int st = 0; st < STEPS; ++st) s[st] = raw[st][k].chain(xg, s[st]);
                    }
                }
            }
        }
#pragma unroll
        for (int st = 0; st < STEPS; ++st) mine[(2 * st + half) * kPad + r] = s[st];  // an empty range's is zero
        wave_sync();
        float total = 0.0f;
        if (lane < STEPS * 2 && wave_first + lane < a.rows) {
            const float* sums = mine + lane * kPad;
#pragma unroll
            for (int q = 0; q < 32; ++q) total = total + sums[q];
        }
        finish_rows<FULL>(a, wave_first, STEPS * 2, total);
        wave_sync();  // the sums are read before the next tile writes them
    }
}

// Workgroups of `kernel` a CU holds at once with `lds` bytes of dynamic LDS.
template <typename K>
static uint32_t resident(K kernel, size_t lds) {
    int blocks = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, kernel, 256, lds) != hipSuccess || blocks < 1) blocks = 1;
    return static_cast<uint32_t>(blocks);
}

template <uint32_t F, int SPAN, bool XREG, bool FULL, int B>
static void launch_ranges(const Product& a, uint32_t steps, uint32_t tiles, uint32_t waves, size_t x_lds,
                          uint32_t compute_units, hipStream_t stream) {
    const size_t lds = waves * kWaveRows * kRowPad * sizeof(float) + x_lds;
    thread_local size_t cached_lds = ~size_t{0};
    thread_local uint32_t per_cu = 1;
    if (cached_lds != lds) {
        int blocks = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, gemv_ranges<F, SPAN, XREG, FULL, B>, 64 * waves,
                                                         lds) != hipSuccess ||
            blocks < 1)
            blocks = 1;
        per_cu = static_cast<uint32_t>(blocks), cached_lds = lds;
    }
    const dim3 grid(std::min(tiles, per_cu * compute_units));
    hipLaunchKernelGGL((gemv_ranges<F, SPAN, XREG, FULL, B>), grid, dim3(64 * waves), lds, stream, a, steps, tiles);
}

// A grid of at most the workgroups the GPU holds at once, each looping over
// tiles, so no tail round runs part-empty.
template <uint32_t F, int L, int SPAN, bool XREG, bool FULL>
static void go_epilogue(const Product& a, uint32_t steps, uint32_t tiles, uint32_t waves, uint32_t compute_units,
                        hipStream_t stream) {
    // x staged: L = 32, SPAN float4 a thread (range-interleaved); L = 4, x in
    // order with a pad.
    const size_t lds = XREG ? 0
                       : L == 32 ? static_cast<size_t>(SPAN) * 256 * sizeof(float4)
                                 : (static_cast<size_t>(a.groups) * 32 + 16) * sizeof(float);
    if constexpr (L == 32) {
        // Steps are a power of two, and so is the batch: the batch is the
        // smaller, so no load is issued for a row the wave does not decode.
        constexpr uint32_t most = batch_of<F>(SPAN);
        const uint32_t b = std::min(steps, most);
        if (b == 1) {
            launch_ranges<F, SPAN, XREG, FULL, 1>(a, steps, tiles, waves, lds, compute_units, stream);
        } else if constexpr (most >= 2) {
            if (b == 2) {
                launch_ranges<F, SPAN, XREG, FULL, 2>(a, steps, tiles, waves, lds, compute_units, stream);
            } else if constexpr (most >= 4) {
                if (b == 4)
                    launch_ranges<F, SPAN, XREG, FULL, 4>(a, steps, tiles, waves, lds, compute_units, stream);
                else if constexpr (most >= 8)
                    launch_ranges<F, SPAN, XREG, FULL, 8>(a, steps, tiles, waves, lds, compute_units, stream);
            }
        }
    } else {
        thread_local size_t cached_lds = ~size_t{0};
        thread_local uint32_t per_cu = 1;
        if (cached_lds != lds) per_cu = resident(gemv_quarters<F, SPAN, FULL>, lds), cached_lds = lds;
        const dim3 grid(std::min(tiles, per_cu * compute_units));
        hipLaunchKernelGGL((gemv_quarters<F, SPAN, FULL>), grid, dim3(256), lds, stream, a, steps, tiles);
    }
}

template <uint32_t F, int L, int SPAN, bool XREG>
static void go(const Product& a, uint32_t steps, uint32_t tiles, uint32_t waves, uint32_t compute_units,
               hipStream_t stream) {
    if (plain_epilogue(a))
        go_epilogue<F, L, SPAN, XREG, false>(a, steps, tiles, waves, compute_units, stream);
    else
        go_epilogue<F, L, SPAN, XREG, true>(a, steps, tiles, waves, compute_units, stream);
}

template <uint32_t F, int STEPS>
static void go_chunked(const Product& a, uint32_t tiles, uint32_t compute_units, hipStream_t stream) {
    const bool plain = plain_epilogue(a);
    auto kernel = plain ? gemv_chunked<F, false, STEPS> : gemv_chunked<F, true, STEPS>;
    thread_local uint32_t per_cu[2] = {0, 0};
    if (per_cu[plain] == 0) per_cu[plain] = resident(kernel, 0);
    const dim3 grid(std::min(tiles, per_cu[plain] * compute_units));
    hipLaunchKernelGGL(kernel, grid, dim3(256), 0, stream, a, tiles);
}

template <uint32_t F>
static hipError_t launch_format(const Product& a, const Plan& plan, uint32_t cus, hipStream_t stream) {
    const uint32_t tiles = static_cast<uint32_t>(plan.tiles);
    if (plan.kernel == kGemvChunked) {
        switch (plan.steps) {
            case 1: go_chunked<F, 1>(a, tiles, cus, stream); break;
            case 2: go_chunked<F, 2>(a, tiles, cus, stream); break;
            case 4: go_chunked<F, 4>(a, tiles, cus, stream); break;
            default: return hipErrorInvalidValue;
        }
        return hipGetLastError();
    }
    if (plan.kernel == kGemvQuarters) {
        if constexpr (!plain_values(F)) {
            go<F, 4, 9, false>(a, plan.steps, tiles, plan.waves, cus, stream);
            return hipGetLastError();
        }
        return hipErrorInvalidValue;
    }
    switch (plan.span) {
        case 1: go<F, 32, 1, true>(a, plan.steps, tiles, plan.waves, cus, stream); break;
        case 2: go<F, 32, 2, true>(a, plan.steps, tiles, plan.waves, cus, stream); break;
        case 3:
            if constexpr (F != kF32) go<F, 32, 3, true>(a, plan.steps, tiles, plan.waves, cus, stream);
            else return hipErrorInvalidValue;
            break;
        default:
            // x staged in LDS: the quantized formats only (the others take
            // the chunked kernel past three groups a lane).
            if constexpr (!plain_values(F)) {
                if (plan.span == 4) go<F, 32, 4, false>(a, plan.steps, tiles, plan.waves, cus, stream);
                else if (plan.span == 6) go<F, 32, 6, false>(a, plan.steps, tiles, plan.waves, cus, stream);
                else if (plan.span == 8) go<F, 32, 8, false>(a, plan.steps, tiles, plan.waves, cus, stream);
                else return hipErrorInvalidValue;
            } else {
                return hipErrorInvalidValue;
            }
    }
    return hipGetLastError();
}

// The decode's kernel and shape:
//   - Q6_K at K = 1,152, 1,024 or 2,048 in whole steps: the LDS-streamed
//     kernels (the INT8_LIMBS form there when asked);
//   - Q4_0 at K = 1,024, 2,048, 4,096 or 8,192, 2^20 groups or more, in
//     whole steps: the LDS-streamed kernel (the INT8_LIMBS form at K =
//     1,024 and 2,048 when asked);
//   - Q4_0 at K = 9,216 .. 16,384 in whole 1,024s: the LDS-streamed kernel
//     with a lane a range (gemv_wide.hip);
//   - quantized K = 1,152 otherwise: 4 lanes a row, 9 groups each;
//   - other K up to 8,192: the reference's 32 lanes a row, x in registers
//     while a lane's slice is at most 3 groups, else staged whole in LDS
//     (a lane's 4, 6 or 8 groups: 5 and 7 take the next size's kernel);
//   - past 8,192, F16 and BF16 past 3,072 and F32 past 2,048 (their groups
//     are 64 or 128 bytes, too many registers for a lane's whole slice): x
//     staged a chunk of 8 groups a range at a time.
bool plan_gemv(const Product& a, uint32_t format, uint32_t compute_units, bool limbs, Plan* plan) {
    *plan = Plan{};
    plan->launches = 1;
    plan->tile_tokens = 1;
    const uint32_t G = a.groups;
    if (G == 0 || a.rows == 0 || compute_units == 0) return false;
    if (gemv_stream_takes(a, format) || gemv_stream8_takes(a, format)) {
        const bool stream = G == 36;
        const uint32_t step_rows = stream ? 16 : 64 / (G / 8);
        plan->kernel = stream ? kGemvStream : kGemvStream8;
        plan->limbs = limbs;
        plan->canonical = !limbs;
        plan->lanes = stream ? 4 : G / 8;
        plan->span = stream ? 9 : 8;
        plan->steps = 1;
        plan->tile_rows = step_rows;
        plan->tiles = a.rows / step_rows;
        plan->workgroups = std::min<uint64_t>(2ull * compute_units, (plan->tiles + 3) / 4);
        return true;
    }
    if (gemv_stream4_takes(a, format)) {
        const uint32_t step_rows = 64 / (G / 8);
        plan->kernel = kGemvStream4;
        // the limbs form at K = 1,024 and 2,048 only: at 4,096 and 8,192 it
        // measured slower than the canonical decode (21.4 against 20.4 us,
        // 37.9 against 33.7, plain copies); at 1,024 it is ~10% faster with
        // non-temporal copies (Q4_0 head 19.6 against 21.7 us)
        plan->limbs = limbs && G <= 64;
        plan->canonical = !plan->limbs;
        plan->lanes = G / 8;
        plan->span = 8;
        plan->steps = 1;
        plan->tile_rows = step_rows;
        plan->tiles = a.rows / step_rows;
        plan->workgroups = gemv_stream4_workgroups(G, compute_units, plan->tiles);
        return true;
    }
    if (gemv_wide_takes(a, format)) {
        plan->kernel = kGemvWide;
        plan->lanes = 32;
        plan->span = G / 32;
        plan->steps = 1;
        plan->tile_rows = 2;
        plan->tiles = (a.rows + 1) / 2;
        plan->workgroups = gemv_wide_workgroups(compute_units, plan->tiles);
        return true;
    }
    if (G * 32 > kMaxStagedK || (format == kF32 && G > 64) || (plain_values(format) && G > 96)) {
        plan->kernel = kGemvChunked;
        plan->lanes = 32;
        plan->span = (G + 31) / 32;
        // Steps a wave: the fewest (1, 2 or 4) that bring the grid down to
        // two workgroups a CU.
        uint32_t steps = 1;
        while (steps < 4 && static_cast<uint64_t>(steps) * kWaves * 2 * 2 * compute_units < a.rows) steps *= 2;
        plan->steps = steps;
        plan->tile_rows = kWaves * 2 * steps;
        plan->tiles = (a.rows + plan->tile_rows - 1) / plan->tile_rows;
        plan->workgroups = std::min<uint64_t>(plan->tiles, 2ull * compute_units);
        return true;
    }
    if (G == 36 && !plain_values(format)) {
        plan->kernel = kGemvQuarters;
        plan->lanes = 4;
        plan->span = 9;
    } else {
        const uint32_t span = (G + 31) / 32;
        plan->kernel = kGemvRanges;
        plan->lanes = 32;
        plan->span = span <= 4 ? span : span <= 6 ? 6 : 8;
        plan->xreg = span <= 3;
    }
    const uint32_t rows_a_step = 64 / plan->lanes;
    const uint32_t max_steps = kWaveRows / rows_a_step;
    if (plan->lanes == 4) {
        // Steps a wave: the most, up to max_steps, that still gives every CU
        // about 8 waves.
        const uint32_t steps = a.rows / (rows_a_step * compute_units * 8);
        plan->steps = steps < 1 ? 1 : steps > max_steps ? max_steps : steps;
    } else {
        // L = 32: a power of two of steps a wave, the fewest that bring the
        // grid down to one workgroup a CU — two for products of 2^20 groups
        // or more. A small product is bound by its workgroups' dispatch and
        // one memory round trip, so fewer workgroups with more rows each
        // finish sooner (Q4_0 3,072 x 1,024: 384 workgroups 5.0 us, 192
        // 4.3 us, 96 4.8 us); a large one needs the second workgroup's loads
        // in flight.
        const uint64_t per_cu = static_cast<uint64_t>(a.rows) * G >= (1u << 20) ? 2 : 1;
        const uint64_t target = per_cu * compute_units * kWaves * rows_a_step;
        uint32_t steps = 1;
        while (steps < max_steps && steps * target < a.rows) steps *= 2;
        // Past one round of tiles on the resident workgroups (two a CU), the
        // fewer steps whose rounds leave the fewest rows on the busiest
        // workgroup: 151,936 rows at 32 steps are 594 tiles on 512
        // workgroups, 82 of which run a second round (512 rows for the
        // busiest); at 8 steps, 2,374 tiles, 320 rows (Q4_0 head: 28.5 ->
        // 26 us).
        const uint64_t resident = 2ull * compute_units;
        auto makespan = [&](uint32_t st) {
            const uint64_t rows_a_tile = uint64_t{kWaves} * st * rows_a_step;
            const uint64_t tiles = (a.rows + rows_a_tile - 1) / rows_a_tile;
            return (tiles + resident - 1) / resident * rows_a_tile;
        };
        uint32_t best = steps;
        const uint64_t tiles_now = (a.rows + uint64_t{kWaves} * steps * rows_a_step - 1) / (uint64_t{kWaves} * steps * rows_a_step);
        if (tiles_now > resident)
            for (uint32_t st = steps / 2; st >= 8; st /= 2)
                if (makespan(st) * 100 < makespan(best) * 97) best = st;
        plan->steps = best;
        // A small product with x in registers (under 2^20 groups: one
        // workgroup a CU at most) runs its waves as workgroups of one: they
        // spread over every CU rather than four to a CU on three quarters of
        // them (Q4_0 3,072 x 1,024: 4.03 -> 3.81 us; the Qwen3 0.6B decode
        // step 633 -> 589 us). A large one keeps four a workgroup (the Q4_0
        // head of 151,936 rows: 23.0 against 24.1 us).
        if (plan->xreg && per_cu == 1) plan->waves = 1;
    }
    plan->tile_rows = plan->waves * plan->steps * rows_a_step;
    plan->tiles = (a.rows + plan->tile_rows - 1) / plan->tile_rows;
    plan->workgroups = plan->tiles;  // at most; the launch caps it at what the GPU holds
    return true;
}

hipError_t launch_gemv(const Product& a, uint32_t format, const Plan& plan, uint32_t compute_units,
                       hipStream_t stream) {
    if (plan.kernel == kGemvStream) return launch_gemv_stream(a, compute_units, plan.limbs, stream);
    if (plan.kernel == kGemvStream8) return launch_gemv_stream8(a, compute_units, plan.limbs, stream);
    if (plan.kernel == kGemvStream4) return launch_gemv_stream4(a, compute_units, plan.limbs, stream);
    if (plan.kernel == kGemvWide) return launch_gemv_wide(a, compute_units, stream);
    switch (format) {
        case kQ4_0: return launch_format<kQ4_0>(a, plan, compute_units, stream);
        case kQ4_1: return launch_format<kQ4_1>(a, plan, compute_units, stream);
        case kQ8_0: return launch_format<kQ8_0>(a, plan, compute_units, stream);
        case kQ6_K: return launch_format<kQ6_K>(a, plan, compute_units, stream);
        case kF32: return launch_format<kF32>(a, plan, compute_units, stream);
        case kF16: return launch_format<kF16>(a, plan, compute_units, stream);
        case kBF16: return launch_format<kBF16>(a, plan, compute_units, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace chm
