// k_gemm.hip — ternary x int8 prefill GEMM (M > 16 tokens) on gfx950 int8 MFMA.
//
// Y (N, M) = (tau[n] * s[m]) * float(sum_k trit(n,k) * q(m,k)) [+ bias[n]]
//
// Operands: weights in the T16K256 layout (1 KiB per 16 rows x 256 k, lane-ordered MFMA A
// operands: (word_q >> 2j) & 0x03030303 = codes of k = 256kt + 64j + 16g + 0..15), and
// token-major int8 activations xi (M, Kp). MFMAs accumulate sum(code * x); the epilogue
// subtracts 2 * rowsum[m] (codes are trit + 2).
//
// MFMA: v_mfma_i32_32x32x32_i8. On MI355X it sustains ~3.7 POP/s in a pure-MFMA loop against
// ~2.6 for the 16x16x64 shape, so the GEMM uses 32x32 tiles. Lane l of a 32x32x32 MFMA holds
// row l%32 (A) / token l%32 (B) and the 16 k of half l/32; for k0 = 64j + 32m it reads the
// T16K256 lane 16*(2m + l/32) + (row%16) of the row's tile and shifts by 2j, so the same tile
// layout feeds both the 16x16 GEMV and this GEMM.
// Tiling: one block per CU, kWavesN x kWavesM waves (default 2 x 4 = 8, two per SIMD so one
// wave's LDS reads and unpacking overlap the other's MFMAs). Block tile 256 rows (16 row
// tiles) x 128 tokens; default wave tile 128 rows x 32 tokens = 4 x 1 MFMA tiles of 32x32.
// Per 256-wide k tile ("stage") the block stages A (16 KiB, copied as is) and B (128 token
// rows of 256 B, 16-byte chunk c of token t stored at chunk c ^ (t & 15) so the 16 lanes of
// a ds_read_b128 hit 16 distinct bank groups) with buffer->LDS DMA loads (no register
// staging; out-of-range rows and tokens read as zeros). Three LDS slots form a ring: stage
// s+2 is issued at the top of stage s, so two k tiles of loads are in flight while one is
// multiplied; one barrier per stage. Waits on the DMA are explicit s_waitcnt vmcnt.
//
// Block order is XCD-aware: blocks are dealt round-robin to the 8 XCDs, and each XCD gets
// whole token blocks (all N for them), so a token block's activations stay in that XCD's L2.
#include "common.hpp"

namespace nnhip
{
namespace
{

typedef int v4i __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr uint32_t kM3 = 0x03030303u;
#ifndef NNHIP_GEMM_WAVES_N
#define NNHIP_GEMM_WAVES_N 4
#endif
#ifndef NNHIP_GEMM_WAVES_M
#define NNHIP_GEMM_WAVES_M 2
#endif
constexpr int kWavesN = NNHIP_GEMM_WAVES_N, kWavesM = NNHIP_GEMM_WAVES_M;
constexpr int kWaves = kWavesN * kWavesM;
constexpr int kThreads = 64 * kWaves;
constexpr int kBN = 256, kBM = 128;          // block tile (rows, tokens)
constexpr int kRowTiles = kBN / 16;          // 16
constexpr int kWaveRows = kBN / kWavesN, kWaveToks = kBM / kWavesM;
constexpr int kWaveRowBlocks = kWaveRows / 32, kWaveTokBlocks = kWaveToks / 32;  // 32x32 MFMA tiles
constexpr int kSlots = 3;
constexpr int kABytes = kRowTiles * 1024;    // 16 KiB
constexpr int kBBytes = kBM * kTileK;        // 32 KiB
constexpr int kSlotBytes = kABytes + kBBytes;
constexpr int kLdsBytes = kSlots * kSlotBytes;  // 144 KiB
// DMA instructions per wave per stage: A one row tile (1 KiB) each, B four token rows each
constexpr int kADma = kRowTiles / kWaves, kBDma = kBM / 4 / kWaves;
static_assert(kADma * kWaves == kRowTiles && kBDma * kWaves * 4 == kBM, "DMA split");
constexpr int kDmaPerStage = kADma + kBDma;  // 12
constexpr int kRsrcFlags = 0x00020000;

static_assert(kDmaPerStage < 63, "vmcnt range");

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kRsrcFlags);
}

typedef int v16i __attribute__((ext_vector_type(16)));

__device__ __forceinline__ v16i mfma32(v4i a, v4i b, v16i c)
{
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

// s_waitcnt vmcnt(N) with expcnt / lgkmcnt left open (gfx9 encoding)
template <int N>
__device__ __forceinline__ void wait_vmcnt()
{
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x70 | 0xF00);
}

// Workgroup barrier without a memory fence. __syncthreads() (and any workgroup fence, even
// one limited to LDS) makes the compiler wait for every outstanding buffer->LDS load
// (vmcnt(0)), which drains the DMA ring each stage. Here the caller's explicit vmcnt wait
// covers the one stage that must have landed, and every LDS read of a slot is consumed
// (lgkmcnt waited) before its wave reaches the barrier that lets the slot be refilled. The
// empty asm statements are compiler-only memory clobbers (no wait instructions): no load or
// store moves across the barrier.
__device__ __forceinline__ void lds_barrier()
{
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

struct Dma
{
    __amdgpu_buffer_rsrc_t ra, rb;
    uint32_t a_voff;    // lane * 16 within a row tile
    uint32_t b_voff[kBDma];
    uint32_t a_row0;    // first row tile (global) this wave copies
};

// Issue the DMA of k tile kt into LDS slot `slot`.
__device__ __forceinline__ void issue_stage(uint8_t* lds, const Dma& d, int slot, int kt, int KT)
{
    uint8_t* base = lds + slot * kSlotBytes;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
    for (int i = 0; i < kADma; ++i)
    {
        const int rt_local = wave * kADma + i;
        const uint32_t soff = ((d.a_row0 + rt_local) * (uint32_t)KT + (uint32_t)kt) * 1024u;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(d.ra, (lds_void*)(base + rt_local * 1024), 16, d.a_voff, soff, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < kBDma; ++i)
    {
        // this instruction fills token rows 4*(wave*kBDma + i) .. +3 (1 KiB)
        uint8_t* dst = base + kABytes + (wave * kBDma + i) * 1024;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(d.rb, (lds_void*)dst, 16, d.b_voff[i], (uint32_t)kt * kTileK, 0, 0);
    }
}

__global__ __launch_bounds__(kThreads) void k_gemm(GemvProblem p, int n_mblocks, int n_nblocks, int xcd_mode)
{
    extern __shared__ __align__(16) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wn = wave % kWavesN, wm = wave / kWavesN;
    const int g = lane >> 4, t = lane & 15;
    const int KT = p.KT;
    const uint32_t Kp = (uint32_t)KT * kTileK;
    const int RT = (p.N + 15) / 16;

    // ---- block -> (token block, row block)
    int mb, nb;
    const int b = blockIdx.x;
    if (xcd_mode)
    {
        const int xcd = b & 7, l = b >> 3;
        const int per_xcd = n_mblocks >> 3;  // token blocks per XCD
        mb = xcd * per_xcd + l / n_nblocks;
        nb = l % n_nblocks;
    }
    else
    {
        mb = b / n_nblocks;
        nb = b % n_nblocks;
    }
    const int m0 = mb * kBM;
    const int rt0 = nb * kRowTiles;

    // ---- DMA descriptors
    Dma d;
    d.ra = rsrc(p.rp, (uint32_t)RT * (uint32_t)KT * 1024u);  // rows past N read zero (code 0)
    d.rb = rsrc(p.xi, (uint32_t)p.M * Kp);                    // tokens past M read zero
    d.a_voff = (uint32_t)lane * 16u;
    d.a_row0 = (uint32_t)rt0;
#pragma unroll
    for (int i = 0; i < kBDma; ++i)
    {
        const int row = (wave * kBDma + i) * 4 + (lane >> 4);  // token row within the block
        const int pos = lane & 15;                             // chunk position in the LDS row
        const int c = pos ^ (row & 15);                        // global chunk stored there
        const int m = m0 + row;
        d.b_voff[i] = m < p.M ? (uint32_t)m * Kp + (uint32_t)c * 16u : 0x80000000u;
    }

    v16i acc[kWaveRowBlocks][kWaveTokBlocks];
#pragma unroll
    for (int i = 0; i < kWaveRowBlocks; ++i)
#pragma unroll
        for (int n = 0; n < kWaveTokBlocks; ++n) acc[i][n] = v16i{};

    const int h = lane >> 5, l32 = lane & 31;
    issue_stage(lds, d, 0, 0, KT);
    if (KT > 1) issue_stage(lds, d, 1, 1, KT);

    for (int s = 0; s < KT; ++s)
    {
        // stage s has landed once at most the next stage's DMAs are outstanding
        if (s + 1 < KT) wait_vmcnt<kDmaPerStage>();
        else wait_vmcnt<0>();
        lds_barrier();  // every wave's part of stage s is in LDS; stage s-1's slot is free
        if (s + 2 < KT) issue_stage(lds, d, (s + 2) % kSlots, s + 2, KT);

        const uint8_t* sa = lds + (s % kSlots) * kSlotBytes;
        const uint8_t* sb = sa + kABytes;
        // A words: row block rb covers row tiles wn*8 + 2rb + (l32 / 16); half m of the 64-k
        // group is T16K256 lane 16 * (2m + h) + l32 % 16
        v4i wa[kWaveRowBlocks][2];
#pragma unroll
        for (int rb = 0; rb < kWaveRowBlocks; ++rb)
#pragma unroll
            for (int m = 0; m < 2; ++m)
            {
                const int rt_local = wn * (kWaveRows / 16) + 2 * rb + (l32 >> 4);
                wa[rb][m] = *reinterpret_cast<const v4i*>(sa + rt_local * 1024 + (16 * (2 * m + h) + (l32 & 15)) * 16);
            }
#pragma unroll
        for (int j = 0; j < 4; ++j)
        {
#pragma unroll
            for (int m = 0; m < 2; ++m)
            {
                const int c = 4 * j + 2 * m + h;  // 16-byte chunk of this lane's k half
                v4i bf[kWaveTokBlocks];
#pragma unroll
                for (int n = 0; n < kWaveTokBlocks; ++n)
                {
                    const int row = wm * kWaveToks + n * 32 + l32;
                    bf[n] = *reinterpret_cast<const v4i*>(sb + row * kTileK + ((c ^ (row & 15)) << 4));
                }
#pragma unroll
                for (int rb = 0; rb < kWaveRowBlocks; ++rb)
                {
                    const v4i a = (v4i)((__builtin_bit_cast(u32x4, wa[rb][m]) >> (2 * j)) & kM3);
#pragma unroll
                    for (int n = 0; n < kWaveTokBlocks; ++n) acc[rb][n] = mfma32(a, bf[n], acc[rb][n]);
                }
            }
        }
    }

    // ---- epilogue. Operands come in with unconditional buffer loads (rows past N, tokens past M read 0),
    // issued together so the waits do not serialize; masked lanes store to an out-of-range
    // offset, which the buffer unit drops.
    const __amdgpu_buffer_rsrc_t rtau = rsrc(p.tau, (uint32_t)p.N * 4u);
    const __amdgpu_buffer_rsrc_t rbias = rsrc(p.bias ? p.bias : p.tau, p.bias ? (uint32_t)p.N * 4u : 0u);
    const __amdgpu_buffer_rsrc_t rs_r = rsrc(p.rowsum, (uint32_t)p.M * 4u);
    const __amdgpu_buffer_rsrc_t rs_s = rsrc(p.s, (uint32_t)p.M * 4u);
    const __amdgpu_buffer_rsrc_t ry = rsrc(p.y, (uint32_t)((size_t)p.N * p.M * 4u <= 0xFFFFFFFFull
                                                               ? (size_t)p.N * p.M * 4u : 0xFFFFFFFFull));
    int rs2[kWaveTokBlocks];
    float sv[kWaveTokBlocks];
#pragma unroll
    for (int n = 0; n < kWaveTokBlocks; ++n)
    {
        const uint32_t m = (uint32_t)(m0 + wm * kWaveToks + n * 32 + l32);
        rs2[n] = 2 * __builtin_bit_cast(int, __builtin_amdgcn_raw_buffer_load_b32(rs_r, m * 4u, 0, 0));
        sv[n] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs_s, m * 4u, 0, 0));
    }
    // 32x32 accumulator layout: element i of lane l is row 8*(i/4) + 4*(l/32) + i%4, token l%32.
    // One row block at a time: its 16 tau / bias values are loaded together, then stored.
#pragma unroll
    for (int rb = 0; rb < kWaveRowBlocks; ++rb)
    {
        const int row0 = (rt0 + wn * (kWaveRows / 16) + 2 * rb) * 16 + 4 * h;
        float tv[16], bv[16];
#pragma unroll
        for (int i = 0; i < 16; ++i)
        {
            const uint32_t row = (uint32_t)(row0 + 8 * (i >> 2) + (i & 3));
            tv[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rtau, row * 4u, 0, 0));
            bv[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rbias, row * 4u, 0, 0));
        }
#pragma unroll
        for (int n = 0; n < kWaveTokBlocks; ++n)
        {
            const int m = m0 + wm * kWaveToks + n * 32 + l32;
#pragma unroll
            for (int i = 0; i < 16; ++i)
            {
                const int row = row0 + 8 * (i >> 2) + (i & 3);
                const int a = acc[rb][n][i] - rs2[n];
                float y = (tv[i] * sv[n]) * (float)a;
                if (p.bias) y = y + bv[i];
                const uint32_t off = (row < p.N && m < p.M) ? ((uint32_t)row * (uint32_t)p.M + (uint32_t)m) * 4u
                                                             : 0xFFFFFFF0u;
                __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, y), ry, off, 0, 0);
            }
        }
    }
}

}  // namespace

hipError_t launch_gemm(hipStream_t st, const GemvProblem& p, int /*num_cus*/)
{
    if (p.N == 0 || p.M == 0) return hipSuccess;
    static bool attr_set = false;
    if (!attr_set)
    {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemm),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    const int n_mblocks = (int)ceil_div((size_t)p.M, kBM);
    const int n_nblocks = (int)ceil_div((size_t)p.N, kBN);
    const int xcd_mode = (n_mblocks % 8 == 0) ? 1 : 0;
    const unsigned blocks = (unsigned)(n_mblocks * n_nblocks);
    hipLaunchKernelGGL(k_gemm, dim3(blocks), dim3(kThreads), kLdsBytes, st, p, n_mblocks, n_nblocks, xcd_mode);
    return hipGetLastError();
}

}  // namespace nnhip
