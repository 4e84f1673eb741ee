// k_gemv.hip — weight-streaming decode GEMV (M <= 16 tokens) for gfx950.
//
// One wave computes RTW consecutive 16-row tiles of one problem against all its (<= 16)
// tokens with v_mfma_i32_16x16x64_i8, streaming the tiles' K/256 weight tiles (T16K256
// layout, 1 KiB each: one 16-byte load per lane) from HBM. The activation operands of a
// k tile are loaded once per stage and shared by the RTW row tiles, so more weight bytes
// are in flight per register. Codes are trit + 2, so the MFMAs accumulate sum(code * x)
// and the epilogue subtracts 2 * rowsum. Four accumulators per row tile make the unpack
// 5 VALU ops per weight word instead of 7:
//   j=0: w & 0x03030303 (codes)          -> a0      j=1: w & 0x0C0C0C0C (4 * codes)  -> a1
//   j=2: w & 0x30303030 (16 * codes)     -> a2      j=3: (w >> 6) & 0x03030303       -> a3
//   acc = a0 + a3 + (a1 >> 2) + (a2 >> 4) - 2 * rowsum       (shifts divide exact multiples)
//
// Memory: raw buffer loads. Lanes of tokens t >= M and row tiles past the matrix use
// out-of-range offsets/resources, which the buffer unit answers with zeros and no memory
// traffic (no branches around loads). A rolling pipeline keeps kDepth k-tile stages in
// flight per wave; with the k-tile count known at compile time (the common widths) the
// loop is fully unrolled and the vmcnt waits only cover the stage being consumed.
//
// Epilogue (reference order, src/int8_act_test.cpp:233): y = (tau[n] * s[t]) * float(acc),
// then y + bias[n] as a separate rounding (compiled with -ffp-contract=off).
#include "common.hpp"
#include "gemv_tile.hpp"


namespace nnhip
{
namespace
{

constexpr int kBlock = 256;                 // 4 waves

template <int kRTW>
struct Stage
{
    v4i w[kRTW];  // 4 weight words of this lane, per row tile
    v4i x[4];     // activation bytes for MFMA j = 0..3 (register path only)
};

template <int kRTW>
struct Src
{
    __amdgpu_buffer_rsrc_t rw[kRTW];  // one resource per row tile (num_records = KT KiB, 0 past N)
    __amdgpu_buffer_rsrc_t rx;
    uint32_t voff_w, voff_x;
    const uint8_t* xl;  // LDS path: this lane's activation row
    uint32_t sw0, sw1;  // LDS path: byte offsets of this lane's units (g, 4 + g) in a 128-byte group
};

template <bool LDS, int kRTW>
__device__ __forceinline__ void load_stage(Stage<kRTW>& st, const Src<kRTW>& s, int kt)
{
#pragma unroll
    for (int r = 0; r < kRTW; ++r) st.w[r] = ld16<kNT>(s.rw[r], s.voff_w, (uint32_t)kt * 1024u);
    if constexpr (!LDS)
    {
#pragma unroll
        for (int j = 0; j < 4; ++j) st.x[j] = ld16(s.rx, s.voff_x, (uint32_t)kt * 256u + 64u * j);
    }
}

template <int kRTW>
__device__ __forceinline__ void read_x_lds(v4i (&x)[4], const Src<kRTW>& s, int kt)
{
#pragma unroll
    for (int j = 0; j < 4; ++j) x[j] = *reinterpret_cast<const v4i*>(s.xl + kt * 256 + (j >> 1) * 128 + ((j & 1) ? s.sw1 : s.sw0));
}

// Copy the listed activation blocks into LDS (whole block cooperates), then barrier. Unit u
// (16 bytes) of token row t lands at unit u ^ (t & 7) of its 128-byte group, so the 16 token rows
// an MFMA operand reads sit in 8 distinct bank groups (without it, rows Kp apart share banks).
// The 16-wave blocks (up to 152 KiB of activations) copy by buffer->LDS DMA, one KiB of LDS per
// instruction (lane l fills LDS unit 64q + l from the source unit that belongs there), all of a
// block's instructions in flight together and one wait at the barrier: copied through
// registers, each 16-byte load waited for its store, one memory round trip per 16 KiB of the
// block's staging (M=16 sweep 5460 -> 5570 GB/s). The 4-wave blocks (at most 48 KiB, a few KiB
// at M=1) keep the register copy, measured alike or slightly faster there.
template <int kThreads = kBlock>
__device__ __forceinline__ void stage_x(uint8_t* lds, const XStage* __restrict__ xs, int n_x)
{
    if constexpr (kThreads < 1024)
    {
        for (int e = 0; e < n_x; ++e)
        {
            const XStage x = xs[e];
            for (uint32_t off = threadIdx.x * 16u; off < x.bytes; off += kThreads * 16u)
            {
                const uint32_t t = off / x.row, u = (off - t * x.row) >> 4;
                const uint32_t dst = t * x.row + (((u & ~7u) | ((u ^ t) & 7u)) << 4);
                *reinterpret_cast<v4i*>(lds + x.lds_off + dst) = *reinterpret_cast<const v4i*>(x.src + off);
            }
        }
        __syncthreads();
        return;
    }
    typedef __attribute__((address_space(3))) void lds_void;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const uint32_t lane = threadIdx.x & 63u;
    for (int e = 0; e < n_x; ++e)
    {
        const XStage x = xs[e];
        const __amdgpu_buffer_rsrc_t rx = rsrc(x.src, x.bytes);
        const uint32_t upr = x.row >> 4;  // 16-byte units per token row
        const uint32_t nq = (x.bytes + 1023u) >> 10;
        for (uint32_t q = (uint32_t)wave; q < nq; q += kThreads / kWave)
        {
            const uint32_t L = q * 64u + lane;  // LDS unit of this lane
            if (L * 16u < x.bytes)              // lanes past the block leave the LDS after it alone
            {
                const uint32_t t = L / upr, u = L - t * upr;
                const uint32_t src = t * x.row + (((u & ~7u) | ((u ^ t) & 7u)) << 4);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_void*)(lds + x.lds_off + q * 1024u), 16, src, 0, 0,
                                                         0);
            }
        }
    }
    __syncthreads();
}

// Loads are unconditional: a stage past the last k tile reads beyond its resource
// (num_records = KT KiB), which returns zero words (code 0: no contribution). On the LDS
// path the activations of stage kt+1 are read from LDS while stage kt computes (LDS reads
// count on lgkmcnt, so they never wait behind the weight stream).
template <bool LDS, int kRTW, int kDepth, int KT_FIXED, int kThreads = kBlock, bool kStage = false>
__device__ __forceinline__ void gemv_stream(int KT, const Src<kRTW>& s, Acc (&acc)[kRTW], uint8_t* lds = nullptr,
                                            const XStage* __restrict__ xs = nullptr, int n_x = 0)
{
    Stage<kRTW> st[kDepth];
#pragma unroll
    for (int u = 0; u < kDepth; ++u) load_stage<LDS>(st[u], s, u);
    // kStage: the block's activation staging (and its barrier) runs here, behind the first
    // weight stages of the wave's first item, so their memory latency overlaps it
    if constexpr (kStage) stage_x<kThreads>(lds, xs, n_x);
    v4i xc[4], xn[4];
    if constexpr (LDS) read_x_lds(xc, s, 0);
    if constexpr (KT_FIXED > 0)
    {
#pragma unroll
        for (int kt = 0; kt < KT_FIXED; ++kt)
        {
            if constexpr (LDS)
            {
                if (kt + 1 < KT_FIXED) read_x_lds(xn, s, kt + 1);
                compute_stage<kRTW, true>(st[kt % kDepth].w, xc, acc);
#pragma unroll
                for (int j = 0; j < 4; ++j) xc[j] = xn[j];
            }
            else
            {
                compute_stage<kRTW, true>(st[kt % kDepth].w, st[kt % kDepth].x, acc);
            }
            if (kt + kDepth < KT_FIXED) load_stage<LDS>(st[kt % kDepth], s, kt + kDepth);
            // keep the stage order: later stages' MFMAs must not be hoisted above these loads
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    else
    {
        for (int kt = 0; kt < KT; kt += kDepth)
        {
#pragma unroll
            for (int u = 0; u < kDepth; ++u)
            {
                // zero words past KT: adds nothing (the LDS read stays inside the staged row)
                if constexpr (LDS)
                {
                    if (kt + u + 1 < KT) read_x_lds(xn, s, kt + u + 1);
                    compute_stage<kRTW, true>(st[u].w, xc, acc);
#pragma unroll
                    for (int j = 0; j < 4; ++j) xc[j] = xn[j];
                }
                else
                {
                    compute_stage<kRTW, true>(st[u].w, st[u].x, acc);
                }
                load_stage<LDS>(st[u], s, kt + u + kDepth);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
}

// Item = row tiles rt0 .. rt0 + kRTW - 1 of problem p. LDS path: the problem's activations
// were staged at lds + p.xlds; tokens t >= M read token 0's row (their columns are never
// stored), so no lane needs zeros.
template <bool LDS, int kRTW, int kDepth, int kThreads = kBlock, bool kStage = false>
__device__ __forceinline__ void gemv_item(const GemvProblem& p, int rt0, int lane, uint8_t* lds,
                                          const XStage* __restrict__ xs = nullptr, int n_x = 0)
{
    const int g = lane >> 4, t = lane & 15;
    const int RT = (p.N + 15) / 16;
    const uint32_t Kp = (uint32_t)p.KT * kTileK;
    Src<kRTW> s;
#pragma unroll
    for (int r = 0; r < kRTW; ++r)
    {
        const int rt = rt0 + r < RT ? rt0 + r : RT - 1;
        s.rw[r] = rsrc(p.rp + (size_t)rt * p.KT * 64, rt0 + r < RT ? (uint32_t)p.KT * 1024u : 0u);
    }
    s.voff_w = (uint32_t)lane * 16u;
    if constexpr (LDS)
    {
        // operand j of k tile kt is 16-byte column 16 kt + 4 j + g: unit (4 (j & 1) + g) ^ (tr & 7) of
        // the 128-byte group 2 kt + (j >> 1) in the staged row tr (the identity for M = 1)
        const int tr = t < p.M ? t : 0;
        s.xl = lds + p.xlds + tr * Kp;
        s.sw0 = 16u * (uint32_t)(g ^ (tr & 7));
        s.sw1 = 16u * (uint32_t)((4 + g) ^ (tr & 7));
    }
    else
    {
        s.rx = rsrc(p.xi, (uint32_t)p.M * Kp);
        s.voff_x = t < p.M ? (uint32_t)t * Kp + 16u * g : kOOB;
    }

    // Epilogue operands: unconditional buffer loads issued before the weight stream (rows
    // past N and tokens past M read 0), so they have landed by the end of the item. The tile
    // is computed transposed (compute_stage<kT>): lane 16 g + r holds tokens tb + i (tb = 4 g,
    // i = 0..3) of row r of each row tile.
    const uint32_t tb = 4u * (uint32_t)g, rl = (uint32_t)t;
    const __amdgpu_buffer_rsrc_t rtau = rsrc(p.tau, (uint32_t)p.N * 4u);
    const __amdgpu_buffer_rsrc_t rbias = rsrc(p.bias ? p.bias : p.tau, p.bias ? (uint32_t)p.N * 4u : 0u);
    const __amdgpu_buffer_rsrc_t rrs = rsrc(p.rowsum, (uint32_t)p.M * 4u), rs = rsrc(p.s, (uint32_t)p.M * 4u);
    int rs2[4];
    float sv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
    {
        const uint32_t to = tb + i < (uint32_t)p.M ? (tb + i) * 4u : kOOB;
        rs2[i] = 2 * __builtin_bit_cast(int, __builtin_amdgcn_raw_buffer_load_b32(rrs, to, 0, 0));
        sv[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, to, 0, 0));
    }
    float tv[kRTW], bv[kRTW];
#pragma unroll
    for (int r = 0; r < kRTW; ++r)
    {
        const uint32_t n = (uint32_t)(rt0 + r) * 16u + rl;
        tv[r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rtau, n * 4u, 0, 0));
        bv[r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rbias, n * 4u, 0, 0));
    }

    Acc acc[kRTW];
#pragma unroll
    for (int r = 0; r < kRTW; ++r) acc[r].a0 = acc[r].a1 = acc[r].a2 = acc[r].a3 = v4i{0, 0, 0, 0};
    switch (p.KT)
    {
    case 4: gemv_stream<LDS, kRTW, kDepth, 4, kThreads, kStage>(4, s, acc, lds, xs, n_x); break;
    case 10: gemv_stream<LDS, kRTW, kDepth, 10, kThreads, kStage>(10, s, acc, lds, xs, n_x); break;
    case 16: gemv_stream<LDS, kRTW, kDepth, 16, kThreads, kStage>(16, s, acc, lds, xs, n_x); break;
    case 27: gemv_stream<LDS, kRTW, kDepth, 27, kThreads, kStage>(27, s, acc, lds, xs, n_x); break;
    default: gemv_stream<LDS, kRTW, kDepth, 0, kThreads, kStage>(p.KT, s, acc, lds, xs, n_x); break;
    }

    // Masked lanes store out of range (the output is below 2 GiB, so kOOB + 16 is past it): dropped
    // by the buffer unit. With M a multiple of 4 a lane's four tokens are one 16-byte store (the 16
    // lanes of a row tile write its 16 x 16 block as 1 KiB contiguous), written through the L2
    // (kPolicySys): the M = 16 sweep writes 44 MB of outputs beside 527 MB of weights, and left
    // dirty in the L2 they cost 101.2-101.8 against 97.9-98.8 us. Otherwise (M = 1: 64 bytes per
    // row tile) one store per token with the default policy.
    const __amdgpu_buffer_rsrc_t ry = rsrc(p.y, (uint32_t)p.N * (uint32_t)p.M * 4u);
#pragma unroll
    for (int r = 0; r < kRTW; ++r)
    {
        const uint32_t n = (uint32_t)(rt0 + r) * 16u + rl;
        float y[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
        {
            const int a = acc_sum(acc[r], i) - rs2[i];
            y[i] = (tv[r] * sv[i]) * (float)a;
            if (p.bias) y[i] = y[i] + bv[r];
        }
        const bool live = n < (uint32_t)p.N && tb < (uint32_t)p.M;
        const uint32_t base = n * (uint32_t)p.M + tb;
        if ((p.M & 3) == 0)
        {
            __builtin_amdgcn_raw_buffer_store_b128(
                u32x4{__builtin_bit_cast(uint32_t, y[0]), __builtin_bit_cast(uint32_t, y[1]),
                      __builtin_bit_cast(uint32_t, y[2]), __builtin_bit_cast(uint32_t, y[3])},
                ry, live ? base * 4u : kOOB, 0, kPolicySys);
        }
        else
        {
#pragma unroll
            for (int i = 0; i < 4; ++i)
            {
                if (i >= p.M) break;  // uniform: no store that every lane would drop
                const uint32_t off = (live && tb + i < (uint32_t)p.M) ? (base + i) * 4u : kOOB;
                __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, y[i]), ry, off, 0, 0);
            }
        }
    }
}

// Single problem: static assignment of items to waves.
template <bool LDS, int kRTW, int kDepth>
__global__ __launch_bounds__(kBlock) void k_gemv(GemvProblem p, int n_items, XStage xs)
{
    extern __shared__ __align__(16) uint8_t lds[];
    if constexpr (LDS) stage_x(lds, &xs, 1);
    const int lane = threadIdx.x & 63;
    const int waves = gridDim.x * (kBlock / kWave);
    const int first = __builtin_amdgcn_readfirstlane(blockIdx.x * (kBlock / kWave) + (threadIdx.x >> 6));
    for (int item = first; item < n_items; item += waves) gemv_item<LDS, kRTW, kDepth>(p, item * kRTW, lane, lds);
}

// Grouped: wave w processes the items wave_items[wave_start[w] .. wave_start[w+1]) (each
// item = problem << 20 | first row tile). The host balances the per-wave lists by cost
// once, at group creation, so the kernel needs no atomics or memset and can be replayed.
// kThreads = 1024 (16 waves sharing one staging, one block per CU) for an activation block too
// large for four 4-wave blocks per CU.
template <bool LDS, int kRTW, int kDepth, int kThreads = kBlock>
__global__ __launch_bounds__(kThreads) void k_gemv_grouped(const GemvProblem* __restrict__ probs,
                                                           const uint32_t* __restrict__ wave_start,
                                                           const uint32_t* __restrict__ wave_items,
                                                           int n_waves, const XStage* __restrict__ xs,
                                                           int n_x)
{
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(blockIdx.x * (kThreads / kWave) + (threadIdx.x >> 6));
    const uint32_t b = w < n_waves ? wave_start[w] : 0u, e = w < n_waves ? wave_start[w + 1] : 0u;
    // 16-wave blocks (DMA staging of up to 152 KiB): every wave joins the block's staging barrier
    // once, inside its first item after that item's first weight loads are issued (or alone when
    // it has no items), so the weights' memory latency overlaps the staging (M=16 sweep +1 %).
    // 4-wave blocks stage first: there the register copy's waits also waited for the weights and
    // left the pipeline empty after the barrier (M=1 sweep -3 % with the overlap).
    constexpr bool kOverlap = LDS && kThreads >= 1024;
    if constexpr (LDS && !kOverlap) stage_x<kThreads>(lds, xs, n_x);
    if constexpr (kOverlap)
    {
        if (b == e)
        {
            stage_x<kThreads>(lds, xs, n_x);
            return;
        }
        const uint32_t it = wave_items[b];
        const GemvProblem p = probs[it >> 20];
        gemv_item<LDS, kRTW, kDepth, kThreads, true>(p, (int)(it & 0xFFFFFu), lane, lds, xs, n_x);
    }
    for (uint32_t i = kOverlap ? b + 1 : b; i < e; ++i)
    {
        const uint32_t it = wave_items[i];
        const GemvProblem p = probs[it >> 20];
        gemv_item<LDS, kRTW, kDepth>(p, (int)(it & 0xFFFFFu), lane, lds);
    }
}

// ---------------------------------------------------------------------------------------
// Deep decode GEMV for grids smaller than the device (a decode step's BitLinears: 160 - 864
// row tiles), over up to kGemvDeepMulti problems that share K, M and the activations (the
// q / k / v projections of one input). One 16-row tile per wave; the wave issues the loads of
// ALL its KT weight stages first (one memory latency instead of KT / depth of them), then the
// block stages the shared activations (M x Kp bytes, up to 160 KB) into LDS by buffer->LDS DMA
// while they land.
// LDS layout of the staged activations: token-major rows of Kp bytes with the 16-byte units of
// each 128-byte group permuted per token, unit u of row t holding column u ^ (t & 7). An MFMA
// operand read (lane = token t of 16-byte column c, 16 tokens) then touches 8 distinct bank
// groups per 8 lanes; without the permutation all 16 tokens of a column share banks (Kp is a
// multiple of 256 bytes) and the 16-way conflict made the MFMA loop 3-4x slower than its LDS
// bandwidth. Each DMA instruction still fetches one contiguous KiB of the activations (lane l
// takes the unit its LDS slot needs, a permutation within each 128-byte line). res != 0: y = epilogue + res[n, m] (the decoder's residual add, the same
// single rounding as a separate add). glu != 0: the rows are the interleaved gate/up rows of a
// gated FFN (16-row tile = gate rows 8t..8t+7, then up rows 8t..8t+7); lanes of the gate half
// take their up values from the lane 32 apart and store act(gate, up) as features 8t..8t+7 of
// h (glu_F, M) instead of Y.
struct GemvDeepArgs
{
    GemvProblem p[kGemvDeepMulti];
    int tile0[kGemvDeepMulti + 1];  // first row tile of each problem in the launch (prefix sums)
    int count;
    uint32_t xbytes;  // M * Kp: the activation bytes
};

inline size_t gemv_deep_lds_bytes(int M, int KT) { return round_up((size_t)M * KT * kTileK, 1024); }

template <int KT>
__global__ __launch_bounds__(kBlock) void k_gemv_deep(GemvDeepArgs da)
{
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int gt = __builtin_amdgcn_readfirstlane(blockIdx.x * (kBlock / kWave) + (threadIdx.x >> 6));
    int pi = 0;
#pragma unroll
    for (int j = 1; j < kGemvDeepMulti; ++j)
        if (j < da.count && gt >= da.tile0[j]) pi = j;
    const GemvProblem& p = da.p[pi];
    const int rt = gt - da.tile0[pi];
    const int n_tiles = da.tile0[pi + 1] - da.tile0[pi];
    const int g = lane >> 4, t = lane & 15;
    const uint32_t Kp = (uint32_t)KT * kTileK;
    const bool live = gt < da.tile0[da.count];

    // 1. all weight stages of the tile (a tile past the matrix reads zero words)
    const __amdgpu_buffer_rsrc_t rw = rsrc(p.rp + (size_t)(live ? rt : 0) * KT * 64, live ? (uint32_t)KT * 1024u : 0u);
    v4i w[KT];
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) w[kt] = ld16<kNT>(rw, (uint32_t)lane * 16u, (uint32_t)kt * 1024u);

    // 2. epilogue operands (rows past N and tokens past M read 0)
    const __amdgpu_buffer_rsrc_t rtau = rsrc(p.tau, (uint32_t)p.N * 4u);
    const __amdgpu_buffer_rsrc_t rbias = rsrc(p.bias ? p.bias : p.tau, p.bias ? (uint32_t)p.N * 4u : 0u);
    const __amdgpu_buffer_rsrc_t rres = rsrc(p.res ? p.res : p.tau, p.res ? (uint32_t)p.N * (uint32_t)p.M * 4u : 0u);
    const uint32_t tok = t < p.M ? (uint32_t)t : 0x40000000u;
    const int rs2 = 2 * __builtin_bit_cast(int, __builtin_amdgcn_raw_buffer_load_b32(rsrc(p.rowsum, (uint32_t)p.M * 4u), tok * 4u, 0, 0));
    const float sv = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsrc(p.s, (uint32_t)p.M * 4u), tok * 4u, 0, 0));
    float tv[4], bv[4], rv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
    {
        const uint32_t n = (uint32_t)(rt * 16 + 4 * g + i);
        tv[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rtau, n * 4u, 0, 0));
        bv[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rbias, n * 4u, 0, 0));
        // residual (N, M), or token-major (M, N) when the output is
        const uint32_t rix = p.ytm ? (uint32_t)t * (uint32_t)p.N + n : n * (uint32_t)p.M + (uint32_t)t;
        const uint32_t ro = (n < (uint32_t)p.N && t < p.M) ? rix * 4u : 0xFFFFFFF0u;
        rv[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rres, ro, 0, 0));
    }

    // 3. activations into LDS by buffer->LDS DMA (1 KiB per instruction, no registers), issued
    //    behind the weight loads; __syncthreads waits for both and joins the waves
    {
        typedef __attribute__((address_space(3))) void lds_void;
        const __amdgpu_buffer_rsrc_t rx = rsrc(p.xi, da.xbytes);
        const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        const int nq = (int)((da.xbytes + 1023u) / 1024u);
        for (int q = wave; q < nq; q += kBlock / kWave)
        {
            // LDS unit L = (row t, unit u) takes column u ^ (t & 7) of row t (units past the
            // activations read zeros)
            const uint32_t L = (uint32_t)q * 64u + (uint32_t)lane;
            const uint32_t tr = L / (uint32_t)(KT * 16), u = L - tr * (uint32_t)(KT * 16);
            const uint32_t src = tr * Kp + ((u ^ (tr & 7u)) * 16u);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_void*)(lds + q * 1024), 16, src, 0, 0, 0);
        }
        __syncthreads();
    }

    // 4. MFMAs over the k tiles; tokens t >= M read token 0's row (their columns are never stored)
    Acc acc[1];
    acc[0].a0 = acc[0].a1 = acc[0].a2 = acc[0].a3 = v4i{0, 0, 0, 0};
    // operand j of stage kt is column c = 16 kt + 4 j + g: unit (4 (j & 1) + g) ^ (t & 7) of the
    // 128-byte group 2 kt + (j >> 1)
    const int tr = t < p.M ? t : 0;
    const uint8_t* xrow = lds + (size_t)tr * Kp;
    const int sw0 = 16 * (g ^ (tr & 7)), sw1 = 16 * ((4 + g) ^ (tr & 7));
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
    {
        v4i x[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            x[j] = *reinterpret_cast<const v4i*>(xrow + kt * 256 + (j >> 1) * 128 + ((j & 1) ? sw1 : sw0));
        const v4i w1[1] = {w[kt]};
        compute_stage<1>(w1, x, acc);
    }

    // 5. epilogue, the reference order: y = (tau * s) * float(acc) [+ bias] [+ residual]
    float y[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
    {
        const int a = acc[0].a0[i] + acc[0].a3[i] + (acc[0].a1[i] >> 2) + (acc[0].a2[i] >> 4) - rs2;
        y[i] = (tv[i] * sv) * (float)a;
        if (p.bias) y[i] = y[i] + bv[i];
        if (p.res) y[i] = y[i] + rv[i];
    }
    if (p.glu == 0)
    {
        const __amdgpu_buffer_rsrc_t ry = rsrc(p.y, (uint32_t)p.N * (uint32_t)p.M * 4u);
#pragma unroll
        for (int i = 0; i < 4; ++i)
        {
            const int n = rt * 16 + 4 * g + i;
            const uint32_t yix = p.ytm ? (uint32_t)t * (uint32_t)p.N + (uint32_t)n : (uint32_t)n * (uint32_t)p.M + (uint32_t)t;
            const uint32_t off = (live && n < p.N && t < p.M) ? yix * 4u : 0xFFFFFFF0u;
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, y[i]), ry, off, 0, 0);
        }
    }
    else
    {
        const __amdgpu_buffer_rsrc_t rh = rsrc(p.y, (uint32_t)p.glu_F * (uint32_t)p.M * 4u);
#pragma unroll
        for (int i = 0; i < 4; ++i)
        {
            const float up = __shfl_xor(y[i], 32, kWave);  // tile row 8 + 4g + i
            const int f = rt * 8 + 4 * g + i;
            const bool st = live && g < 2 && f < p.glu_F && t < p.M;
            const float hv = glu_one(y[i], up, p.glu - 1);
            const uint32_t ho = p.ytm ? (uint32_t)t * (uint32_t)p.glu_F + (uint32_t)f : (uint32_t)f * (uint32_t)p.M + (uint32_t)t;
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, hv), rh, st ? ho * 4u : 0xFFFFFFF0u, 0, 0);
        }
    }
    (void)n_tiles;
}

template <int KT>
hipError_t launch_deep_kt(hipStream_t st, const GemvDeepArgs& da)
{
    static bool attr = false;
    if (!attr)
    {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemv_deep<KT>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)kGemvDeepLds);
        if (e != hipSuccess) return e;
        attr = true;
    }
    const unsigned blocks = (unsigned)ceil_div((size_t)da.tile0[da.count], (size_t)(kBlock / kWave));
    // the last DMA instruction fills a whole KiB (lanes past the activations read zeros)
    const uint32_t lds_bytes = (uint32_t)gemv_deep_lds_bytes(da.p[0].M, da.p[0].KT);
    hipLaunchKernelGGL(k_gemv_deep<KT>, dim3(blocks), dim3(kBlock), lds_bytes, st, da);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------
// Split-k decode GEMV without epilogue: the integer dot products of slice ks of the k tiles,
// part[ks][t][n] = sum over the slice's k of code(n, k) * x(t, k) (the four MFMA sums combined,
// a0 + a3 + (a1 >> 2) + (a2 >> 4), each an exact integer of the slice), token-major so that a
// per-token epilogue kernel reads its row contiguously. The slice sums add up exactly to the
// whole-K sum, so (tau * s) * float(sum_ks part - 2 rowsum) is the deep GEMV's epilogue bit for
// bit. Block b takes slice b % S (the blocks of one XCD share one slice's activations in L2) and
// row group b / S (4 row tiles, one per wave); the slice's KTS k tiles (KTS_MAX at compile time,
// loads past the slice read zeros) and its activation columns (M x KTS x 256 bytes, the XOR-
// swizzled rows of the deep GEMV) are staged as there. For grids that would leave most CUs idle
// (N = 2560: 40 row groups of the deep GEMV).
template <int KTS_MAX>
__global__ __launch_bounds__(kBlock) void k_gemv_part(GemvProblem p, int S, int kts, int32_t* __restrict__ part)
{
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int ks = (int)(blockIdx.x % (unsigned)S);
    const int rg = (int)(blockIdx.x / (unsigned)S);
    const int rt = rg * (kBlock / kWave) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int RT = (p.N + 15) / 16;
    const int g = lane >> 4, t = lane & 15;
    const uint32_t Kp = (uint32_t)p.KT * kTileK;
    const int k0 = ks * kts;
    const int nk = min(kts, p.KT - k0);  // this slice's k tiles (>= 1)
    const bool live = rt < RT;

    // 1. the slice's weight stages (tiles past the slice or the matrix read zero words)
    const __amdgpu_buffer_rsrc_t rw =
        rsrc(p.rp + ((size_t)(live ? rt : 0) * p.KT + k0) * 64, live ? (uint32_t)nk * 1024u : 0u);
    v4i w[KTS_MAX];
#pragma unroll
    for (int kt = 0; kt < KTS_MAX; ++kt) w[kt] = ld16<kNT>(rw, (uint32_t)lane * 16u, (uint32_t)kt * 1024u);

    // 2. the slice's activation columns into LDS (row tr: Kr = KTS_MAX * 256 bytes, units
    //    permuted per token as in the deep GEMV); columns past the slice are multiplied by zeros
    constexpr uint32_t Kr = (uint32_t)KTS_MAX * kTileK;
    {
        typedef __attribute__((address_space(3))) void lds_void;
        const uint32_t xbytes = (uint32_t)p.M * Kp;
        const __amdgpu_buffer_rsrc_t rx = rsrc(p.xi, xbytes);
        const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        const int nq = (int)(((uint32_t)p.M * Kr + 1023u) / 1024u);
        for (int q = wave; q < nq; q += kBlock / kWave)
        {
            const uint32_t L = (uint32_t)q * 64u + (uint32_t)lane;
            const uint32_t tr = L / (uint32_t)(KTS_MAX * 16), u = L - tr * (uint32_t)(KTS_MAX * 16);
            const uint32_t col = (uint32_t)k0 * kTileK + ((u ^ (tr & 7u)) * 16u);
            const uint32_t src = tr < (uint32_t)p.M && col < Kp ? tr * Kp + col : 0x80000000u;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_void*)(lds + q * 1024), 16, src, 0, 0, 0);
        }
        __syncthreads();
    }

    // 3. MFMAs over the slice's k tiles (tokens t >= M read token 0's row; never stored)
    Acc acc[1];
    acc[0].a0 = acc[0].a1 = acc[0].a2 = acc[0].a3 = v4i{0, 0, 0, 0};
    const int tr = t < p.M ? t : 0;
    const uint8_t* xrow = lds + (size_t)tr * Kr;
    const int sw0 = 16 * (g ^ (tr & 7)), sw1 = 16 * ((4 + g) ^ (tr & 7));
#pragma unroll
    for (int kt = 0; kt < KTS_MAX; ++kt)
    {
        v4i x[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            x[j] = *reinterpret_cast<const v4i*>(xrow + kt * 256 + (j >> 1) * 128 + ((j & 1) ? sw1 : sw0));
        const v4i w1[1] = {w[kt]};
        compute_stage<1>(w1, x, acc);
    }

    // 4. the slice's sums, part[ks][t][n] (rows past N and tokens past M are not stored)
    const __amdgpu_buffer_rsrc_t rp = rsrc(part + (size_t)ks * p.M * p.N, (uint32_t)p.M * (uint32_t)p.N * 4u);
#pragma unroll
    for (int i = 0; i < 4; ++i)
    {
        const int n = rt * 16 + 4 * g + i;
        const int a = acc[0].a0[i] + acc[0].a3[i] + (acc[0].a1[i] >> 2) + (acc[0].a2[i] >> 4);
        const uint32_t off = (live && n < p.N && t < p.M) ? ((uint32_t)t * (uint32_t)p.N + (uint32_t)n) * 4u : 0xFFFFFFF0u;
        __builtin_amdgcn_raw_buffer_store_b32((uint32_t)a, rp, off, 0, 0);
    }
}

template <int KTS_MAX>
hipError_t launch_part_kts(hipStream_t st, const GemvProblem& p, int S, int kts, int32_t* part)
{
    static bool attr = false;
    const uint32_t lds_bytes = (uint32_t)round_up((size_t)p.M * KTS_MAX * kTileK, 1024);
    if (!attr)
    {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemv_part<KTS_MAX>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)kGemvDeepLds);
        if (e != hipSuccess) return e;
        attr = true;
    }
    const unsigned row_groups = (unsigned)ceil_div(ceil_div((size_t)p.N, 16), (size_t)(kBlock / kWave));
    hipLaunchKernelGGL(k_gemv_part<KTS_MAX>, dim3(row_groups * (unsigned)S), dim3(kBlock), lds_bytes, st, p, S, kts,
                       part);
    return hipGetLastError();
}

}  // namespace

// k tiles per slice for S slices, rounded up to a compiled width (0 when none fits)
static int gemv_part_width(int KT, int S)
{
    const int kts = (KT + S - 1) / S;
    static const int widths[] = {1, 2, 3, 4, 5, 7, 10, 14};
    for (int w : widths)
        if (w >= kts) return w;
    return 0;
}

bool gemv_part_ok(const GemvProblem& p, int S)
{
    if (S < 1 || S > 32 || p.M < 1 || p.M > kGemvMaxM || p.N < 1) return false;
    const int kts = (p.KT + S - 1) / S;
    if ((S - 1) * kts >= p.KT) return false;  // every slice holds at least one k tile
    const int w = gemv_part_width(p.KT, S);
    return w > 0 && round_up((size_t)p.M * w * kTileK, 1024) <= kGemvDeepLds;
}

hipError_t launch_gemv_part(hipStream_t st, const GemvProblem& p, int S, int32_t* part)
{
    const int kts = (p.KT + S - 1) / S;
    switch (gemv_part_width(p.KT, S))
    {
    case 1: return launch_part_kts<1>(st, p, S, kts, part);
    case 2: return launch_part_kts<2>(st, p, S, kts, part);
    case 3: return launch_part_kts<3>(st, p, S, kts, part);
    case 4: return launch_part_kts<4>(st, p, S, kts, part);
    case 5: return launch_part_kts<5>(st, p, S, kts, part);
    case 7: return launch_part_kts<7>(st, p, S, kts, part);
    case 10: return launch_part_kts<10>(st, p, S, kts, part);
    case 14: return launch_part_kts<14>(st, p, S, kts, part);
    default: return hipErrorInvalidValue;
    }
}

size_t gemv_grid_waves(size_t n_items, int num_cus, bool lds)
{
    // resident waves per CU for the variant, never more waves than work items
    const GemvVariant v = gemv_variant(lds);
    size_t blocks = ceil_div(n_items, (size_t)(kBlock / kWave));
    const size_t cap = (size_t)(num_cus > 0 ? num_cus : 256) * (v.waves_per_cu / (kBlock / kWave));
    if (blocks > cap)
    {
        blocks = cap;
        // a few items per wave: as many waves as give every wave the same count (4800 items on
        // 4096 waves would leave most waves idle while 704 run a second item)
        const size_t per = ceil_div(n_items, cap * (kBlock / kWave));
        if (per <= 4) blocks = ceil_div(ceil_div(n_items, per), (size_t)(kBlock / kWave));
    }
    if (blocks < 1) blocks = 1;
    return blocks * (kBlock / kWave);
}

bool gemv_deep_multi_ok(const GemvProblem* ps, int count, int num_cus)
{
    if (count < 1 || count > kGemvDeepMulti) return false;
    const GemvProblem& p = ps[0];
    size_t tiles = 0;
    for (int i = 0; i < count; ++i)
    {
        if (ps[i].K != p.K || ps[i].M != p.M || ps[i].xi != p.xi || ps[i].s != p.s || ps[i].rowsum != p.rowsum ||
            ps[i].N < 1)
            return false;
        tiles += ceil_div((size_t)ps[i].N, 16);
    }
    const bool kt_ok = p.KT == 4 || p.KT == 10 || p.KT == 16 || p.KT == 27;
    return kt_ok && p.M >= 1 && p.M <= kGemvMaxM && gemv_deep_lds_bytes(p.M, p.KT) <= kGemvDeepLds &&
           tiles <= (size_t)kGemvDeepMaxTilesPerCu * (size_t)(num_cus > 0 ? num_cus : 256);
}

bool gemv_deep_ok(const GemvProblem& p, int num_cus) { return gemv_deep_multi_ok(&p, 1, num_cus); }

hipError_t launch_gemv_deep_multi(hipStream_t st, const GemvProblem* ps, int count)
{
    GemvDeepArgs da{};
    da.count = count;
    da.tile0[0] = 0;
    for (int i = 0; i < count; ++i)
    {
        da.p[i] = ps[i];
        da.tile0[i + 1] = da.tile0[i] + (int)ceil_div((size_t)ps[i].N, 16);
    }
    for (int i = count; i < kGemvDeepMulti; ++i) da.tile0[i + 1] = da.tile0[count];
    da.xbytes = (uint32_t)ps[0].M * (uint32_t)ps[0].KT * kTileK;
    switch (ps[0].KT)
    {
    case 4: return launch_deep_kt<4>(st, da);
    case 10: return launch_deep_kt<10>(st, da);
    case 16: return launch_deep_kt<16>(st, da);
    case 27: return launch_deep_kt<27>(st, da);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemv_deep(hipStream_t st, const GemvProblem& p) { return launch_gemv_deep_multi(st, &p, 1); }

hipError_t launch_gemv(hipStream_t st, const GemvProblem& p, int num_cus)
{
    if (p.N == 0 || p.M == 0) return hipSuccess;
    if (p.glu == 0 && gemv_deep_ok(p, num_cus)) return launch_gemv_deep(st, p);
    const uint32_t xbytes = (uint32_t)p.M * (uint32_t)p.KT * kTileK;
    const bool lds = xbytes <= kGemvLdsBudget;
    const GemvVariant v = gemv_variant(lds);
    const size_t items = ceil_div(ceil_div((size_t)p.N, 16), (size_t)v.row_tiles);
    const unsigned blocks = (unsigned)(gemv_grid_waves(items, num_cus, lds) / (kBlock / kWave));
    GemvProblem q = p;
    if (lds)
    {
        q.xlds = 0;
        const XStage xs{p.xi, xbytes, 0, (uint32_t)p.KT * kTileK};
        hipLaunchKernelGGL((k_gemv<true, kLdsRTW, kLdsDepth>), dim3(blocks), dim3(kBlock), xbytes, st, q,
                           (int)items, xs);
    }
    else
    {
        q.xlds = -1;
        hipLaunchKernelGGL((k_gemv<false, kRegRTW, kRegDepth>), dim3(blocks), dim3(kBlock), 0, st, q,
                           (int)items, XStage{});
    }
    return hipGetLastError();
}

hipError_t launch_gemv_grouped(hipStream_t st, const GemvProblem* d_probs, const uint32_t* d_wave_start,
                               const uint32_t* d_wave_items, size_t n_waves, const XStage* d_xstage,
                               int n_xstage, uint32_t lds_bytes)
{
    if (n_waves == 0) return hipSuccess;
    if (n_xstage > 0 && lds_bytes > kGemvLdsBudget)
    {
        // one large activation block: 16 waves per block, one block per CU
        constexpr int kBig = 1024;
        static bool attr = false;
        if (!attr)
        {
            const hipError_t e = hipFuncSetAttribute(
                reinterpret_cast<const void*>(&k_gemv_grouped<true, kLdsRTW, kBigDepth, kBig>),
                hipFuncAttributeMaxDynamicSharedMemorySize, (int)kGemvLdsBigBudget);
            if (e != hipSuccess) return e;
            attr = true;
        }
        const unsigned blocks = (unsigned)ceil_div(n_waves, (size_t)(kBig / kWave));
        hipLaunchKernelGGL((k_gemv_grouped<true, kLdsRTW, kBigDepth, kBig>), dim3(blocks), dim3(kBig), lds_bytes, st,
                           d_probs, d_wave_start, d_wave_items, (int)n_waves, d_xstage, n_xstage);
        return hipGetLastError();
    }
    const unsigned blocks = (unsigned)ceil_div(n_waves, (size_t)(kBlock / kWave));
    if (n_xstage > 0)
        hipLaunchKernelGGL((k_gemv_grouped<true, kLdsRTW, kLdsDepth>), dim3(blocks), dim3(kBlock), lds_bytes,
                           st, d_probs, d_wave_start, d_wave_items, (int)n_waves, d_xstage, n_xstage);
    else
        hipLaunchKernelGGL((k_gemv_grouped<false, kRegRTW, kRegDepth>), dim3(blocks), dim3(kBlock), 0, st,
                           d_probs, d_wave_start, d_wave_items, (int)n_waves, d_xstage, 0);
    return hipGetLastError();
}

}  // namespace nnhip
