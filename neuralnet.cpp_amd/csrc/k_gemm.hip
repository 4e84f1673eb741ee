// k_gemm.hip — ternary x int8 prefill GEMM (M > 16 tokens) on gfx950 int8 MFMA.
//
// Y (N, M) = (tau[n] * s[m]) * float(sum_k trit(n,k) * q(m,k)) [+ bias[n]]
//
// Operands: weights in the T16K256 layout (1 KiB per 16 rows x 256 k, lane-ordered MFMA A
// operands: (word_q >> 2j) & 0x03030303 = codes of k = 256kt + 64j + 16g + 0..15), and
// token-major int8 activations xi (M, Kp). MFMAs accumulate sum(code * x); the epilogue
// subtracts 2 * rowsum[m] (codes are trit + 2).
//
// MFMA: v_mfma_i32_32x32x32_i8 (32 cycles, 64 Ki ops). Lane l of a 32x32x32 MFMA holds row
// l%32 (A) / token l%32 (B) and the 16 k of half l/32; for k0 = 64j + 32m it reads the
// T16K256 lane 16*(2m + l/32) + (row%16) of the row's tile and shifts by 2j, so the same tile
// layout feeds both the 16x16 GEMV and this GEMM.
//
// Tiling: one block per CU, block tile kBN rows x kBM tokens, kWavesN x kWavesM output tiles,
// each shared by kKSplit waves (struct Gemm; three configurations, chosen per call by the
// estimated block rounds over the CUs). The large one, 256 x 128 with 4 x 1 x 2 waves, gives
// each pair of waves 64 rows x 128 tokens (2 x 4 MFMA tiles); the two waves of a pair take
// the two k halves of every 64-k group and add their partial sums through LDS at the end. So
// every unpacked weight fragment (the only VALU work of the loop) feeds four MFMAs, LDS reads
// are 0.75 KiB per MFMA, and two waves share each SIMD. 128 x 128 (2 x 2 x 2 waves) and
// 64 x 64 (2 x 2 x 1: one wave per SIMD, no k split) spread problems with few 256 x 128
// blocks over more CUs. Per 256-wide k tile ("stage") the block
// stages A (16 KiB, copied as is) and B (128 token rows of 256 B, 16-byte chunk c of token t
// stored at chunk c ^ (t & 15) so the 16 lanes of a ds_read_b128 hit 16 distinct bank
// groups) with buffer->LDS DMA loads (no register staging; out-of-range rows and tokens read
// as zeros).
//
// Pipeline: a ring of kSlots LDS slots (default 2: measured faster than 3, more DMA in flight
// only added contention); the DMA of stage s+kSlots may start as soon as every wave has
// finished reading stage s. It is issued by the first wave of each k-split pair only, in
// kDmaParts pieces: one right after that barrier, the rest between the MFMAs of the next
// stage's first steps (issued all at once, 48 DMA instructions per block stalled every wave on
// the full address FIFO of the texture unit). Within a stage the wave's 32-k steps are
// software-pipelined: the B fragments of step i+1 are read from LDS while the MFMAs of step i
// run (two register sets), and the A words plus the first B fragments of stage s+1 are read
// before the last MFMAs of stage s. The one barrier per stage sits in the last step, after
// the wave's own reads of the stage have landed and its own part of the next stage's DMA is
// complete (explicit vmcnt / lgkmcnt waits, no memory fence, so the DMA of later stages is not
// drained). Wave priorities fall step by step between barriers (s_setprio), so the two waves
// of a SIMD stay level instead of the older one finishing first and idling at the barrier.
// The epilogue operands (tau, s, rowsum, bias) are loaded before the k-split exchange.
//
// Block order is XCD-aware: blocks are dealt round-robin to the 8 XCDs, and each XCD gets
// whole token blocks (all N for them), so a token block's activations stay in that XCD's L2.
#include "common.hpp"

namespace nnhip
{
namespace
{

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr uint32_t kM3 = 0x03030303u;
constexpr int kRsrcFlags = 0x00020000;
// Cache-policy operand of the output stores: non-temporal. M=2048 x N=4096 x K=4096 33.6 against
// 35.2-35.4 us; the prefill products at 32768 tokens 476 against 510-515 us (2560 x 6912) and
// 1164-1166 against 1194-1205 us (13824 x 2560); write-through (sc1, sc0 sc1) was no faster.
constexpr int kGemmYPolicy = kPolicyNT;
// The gated epilogue's h is read by the next quantizer. When h fits well inside the 256 MiB
// memory-side cache (kGemmHKeepBytes) it is written through (sc0 sc1) so that it stays there:
// the quantization of C4's h (6912 x 2048, 57 MB) took 21.1-21.2 instead of 30.6-30.8 us after
// it (same-box A/B), fc1 unchanged within noise. Larger h (C5's prefill at 32768 tokens, 906 MB)
// stays non-temporal: written through, the prefill took 0.5 ms longer.
constexpr size_t kGemmHKeepBytes = size_t(128) << 20;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kRsrcFlags);
}

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

// s_waitcnt lgkmcnt(0) with vmcnt / expcnt left open
__device__ __forceinline__ void wait_lgkm0()
{
    __builtin_amdgcn_s_waitcnt(0xC07F);
}

// Workgroup barrier without a memory fence. __syncthreads() (and any workgroup fence, even
// one limited to LDS) makes the compiler wait for every outstanding buffer->LDS load
// (vmcnt(0)), which drains the DMA ring each stage. Here the caller's explicit waits cover
// what must have landed (its own DMA part of the next stage, its own LDS reads of this
// stage). The empty asm statements are compiler-only memory clobbers (no wait instructions):
// no load or store moves across the barrier.
__device__ __forceinline__ void lds_barrier()
{
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

#ifndef NNHIP_GEMM_WAVES_N
#define NNHIP_GEMM_WAVES_N 4
#endif
#ifndef NNHIP_GEMM_WAVES_M
#define NNHIP_GEMM_WAVES_M 1
#endif
#ifndef NNHIP_GEMM_KSPLIT
#define NNHIP_GEMM_KSPLIT 2
#endif
#ifndef NNHIP_GEMM_SLOTS
#define NNHIP_GEMM_SLOTS 2  // 256 x 128 tile: 2 slots measured faster than 3
#endif
// DMA issuing waves (default: the first wave of each k-split pair) and pieces per stage
#ifndef NNHIP_GEMM_DMA_WAVES
#define NNHIP_GEMM_DMA_WAVES (kWavesN * kWavesM)
#endif
#ifndef NNHIP_GEMM_DMA_PARTS
#define NNHIP_GEMM_DMA_PARTS 2
#endif
#ifndef NNHIP_GEMM_PRIO
#define NNHIP_GEMM_PRIO 1
#endif
// One configuration of the kernel: block tile kBN_ rows x kBM_ tokens, kWavesN_ x kWavesM_
// output tiles per block, each shared by kKSplit_ waves, a ring of kSlots_ LDS stages.
template <int kBN_, int kBM_, int kWavesN_, int kWavesM_, int kKSplit_, int kSlots_>
struct Gemm
{
    static constexpr int kWavesN = kWavesN_, kWavesM = kWavesM_;
    static constexpr int kKSplit = kKSplit_;   // waves sharing one output tile, splitting its k steps
    static constexpr int kWaves = kWavesN * kWavesM * kKSplit;
    static constexpr int kThreads = 64 * kWaves;
    static constexpr int kWavesPerSimd = kWaves / 4;
    static constexpr int kBN = kBN_, kBM = kBM_;        // block tile (rows, tokens)
    static constexpr int kRowTiles = kBN / 16;
    static constexpr int kWaveRows = kBN / kWavesN, kWaveToks = kBM / kWavesM;
    static constexpr int kRB = kWaveRows / 32, kTB = kWaveToks / 32;  // 32x32 MFMA tiles per wave
    static constexpr int kSteps = kTileK / 32;          // 8 MFMA k steps per stage
    static constexpr int kWaveSteps = kSteps / kKSplit; // steps one wave runs per stage
    static constexpr int kMs = 2 / kKSplit;             // k halves (of each 64-k group) one wave multiplies
    static constexpr int kSlots = kSlots_;               // LDS ring depth (stages in flight)
    static constexpr int kABytes = kRowTiles * 1024;
    static constexpr int kBBytes = kBM * kTileK;
    static constexpr int kSlotBytes = kABytes + kBBytes;
    // k split: one 32x32 partial sum is 16 ints x 64 lanes = 4 KiB; each wave hands over half its row blocks
    static constexpr int kPartBytes = kRB / 2 * kTB * 4096;
    static constexpr int kRingBytes = kSlots * kSlotBytes;
    static constexpr int kLdsMain = kKSplit == 2 && kWaves * kPartBytes > kRingBytes ? kWaves * kPartBytes : kRingBytes;
    static constexpr int kLdsBytes = kLdsMain;
    // DMA instructions per wave per stage: A one row tile (1 KiB) each, B four token rows each
    // Waves 0 .. kDmaWaves-1 issue the DMA (with the default k split, the first wave of each pair:
    // the older wave of its SIMD, which the issue arbiter favours and which reaches the stage
    // barrier first)
    static constexpr int kDmaWaves = NNHIP_GEMM_DMA_WAVES;
    static constexpr int kADma = kRowTiles / kDmaWaves, kBDma = kBM / 4 / kDmaWaves;
    static constexpr int kDmaPerStage = kADma + kBDma;
    // The DMA of one stage is issued in kDmaParts pieces: the first right after the barrier that
    // frees its slot, the others at the start of the next stage's first kDmaParts - 1 steps.
    static constexpr int kDmaParts = kDmaPerStage % NNHIP_GEMM_DMA_PARTS == 0 ? NNHIP_GEMM_DMA_PARTS : 1;
    static constexpr int kPartLoads = kDmaPerStage / kDmaParts;

    static_assert(kWaves % 4 == 0 && kRB >= 1 && kTB >= 1, "wave layout");
    static_assert(kKSplit == 1 || (kKSplit == 2 && kRB % 2 == 0), "k split pairs finish one half of the row blocks each");
    static_assert(kDmaWaves <= kWaves && kADma * kDmaWaves == kRowTiles && kBDma * kDmaWaves * 4 == kBM, "DMA split");
    static_assert(kSlots >= 2 && kSlots <= 6 && 4 * kDmaPerStage < 63, "vmcnt range");
    static_assert(kDmaParts >= 1 && kDmaPerStage % kDmaParts == 0 && kDmaParts <= kWaveSteps, "DMA parts");
    static_assert(kTB * 32 * kTileK <= 65536, "B fragment offsets fit the ds_read immediate");

    // Wait until this wave's DMA of a stage has landed when `later` stages have been issued after
    // it (loads complete in order, kDmaPerStage per stage).
    static __device__ __forceinline__ void wait_stage_landed(int later)
    {
        if (later <= 0) wait_vmcnt<0>();
        else if (later == 1) wait_vmcnt<kDmaPerStage>();
        else if (later == 2) wait_vmcnt<2 * kDmaPerStage>();
        else if (later == 3) wait_vmcnt<3 * kDmaPerStage>();
        else wait_vmcnt<4 * kDmaPerStage>();
    }

    // Issue priority of a wave at step position `pos` of a barrier interval (0 = the step right
    // after the barrier, kWaveSteps - 1 = the step before it). The issue arbiter serves the
    // higher priority first and the older wave on a tie, so without this the older wave of a SIMD
    // runs ahead and idles at the barrier while the younger one finishes alone. Falling priority
    // keeps the two waves of a SIMD at the same step.
    static __device__ __forceinline__ void step_prio(int pos)
    {
        if (!NNHIP_GEMM_PRIO) return;
        const int v = 3 - (pos * 4) / kWaveSteps;
        if (v >= 3) __builtin_amdgcn_s_setprio(3);
        else if (v == 2) __builtin_amdgcn_s_setprio(2);
        else if (v == 1) __builtin_amdgcn_s_setprio(1);
        else __builtin_amdgcn_s_setprio(0);
    }

    struct Dma
    {
        __amdgpu_buffer_rsrc_t ra, rb;
        uint32_t a_voff;    // lane * 16 within a row tile
        uint32_t b_voff[kBDma];
        uint32_t a_row0;    // first row tile (global) of the block
    };

    // Issue loads [lo, hi) of this wave's share of k tile kt's DMA into LDS slot `slot`: the
    // wave's kADma A row tiles come first, then its kBDma groups of four B token rows. lo and hi
    // are constants at every (unrolled) call site.
    static __device__ __forceinline__ void issue_loads(uint8_t* lds, const Dma& d, int slot, int kt, int KT, int lo, int hi)
    {
        uint8_t* base = lds + slot * kSlotBytes;
        const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        if (kDmaWaves < kWaves && wave >= kDmaWaves) return;
#pragma unroll
        for (int q = 0; q < kDmaPerStage; ++q)
        {
            if (q < lo || q >= hi) continue;
            if (q < kADma)
            {
                const int rt_local = wave * kADma + q;
                const uint32_t soff = ((d.a_row0 + rt_local) * (uint32_t)KT + (uint32_t)kt) * 1024u;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(d.ra, (lds_void*)(base + rt_local * 1024), 16, d.a_voff, soff, 0,
                                                         0);
            }
            else
            {
                // this instruction fills token rows 4*(wave*kBDma + i) .. +3 (1 KiB)
                const int i = q - kADma;
                uint8_t* dst = base + kABytes + (wave * kBDma + i) * 1024;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(d.rb, (lds_void*)dst, 16, d.b_voff[i], (uint32_t)kt * kTileK, 0,
                                                         0);
            }
        }
    }

    // The whole DMA of k tile kt (prologue stages).
    static __device__ __forceinline__ void issue_stage(uint8_t* lds, const Dma& d, int slot, int kt, int KT)
    {
        issue_loads(lds, d, slot, kt, KT, 0, kDmaPerStage);
    }

    // A words of one stage: row block rb, the wave's k half (T16K256 lane 16*(2m + h) + row%16;
    // the k half offset is part of p)
    static __device__ __forceinline__ void read_a(v4i (&dst)[kRB][kMs], const uint8_t* p)
    {
#pragma unroll
        for (int rb = 0; rb < kRB; ++rb)
#pragma unroll
            for (int m = 0; m < kMs; ++m) dst[rb][m] = *reinterpret_cast<const v4i*>(p + rb * 2048 + m * 512);
    }

    // B fragments of one step for the wave's kTB token blocks (32 token rows = 8 KiB apart)
    static __device__ __forceinline__ void read_b(v4i (&dst)[kTB], const uint8_t* p)
    {
#pragma unroll
        for (int n = 0; n < kTB; ++n) dst[n] = *reinterpret_cast<const v4i*>(p + n * 32 * kTileK);
    }

    struct Lane
    {
        uint32_t a_off;              // A read offset within a slot
        uint32_t b_off;              // B read offset within a slot (token row of block 0)
        uint32_t b_step[kWaveSteps]; // swizzled chunk offset of the wave's step i
    };

    // One stage: the wave's 32-k steps (all eight, or the four of its k half). P selects the
    // register set holding this stage's A words; the next stage's go to the other set.
    template <int P>
    static __device__ __forceinline__ void run_stage(int s, int KT, uint8_t* lds, const Dma& d, const Lane& ln,
                                              v4i (&wa)[2][kRB][kMs], v4i (&bf)[2][kTB], v16i (&acc)[kRB][kTB])
    {
        const uint8_t* slot = lds + (s % kSlots) * kSlotBytes;
#pragma unroll
        for (int i = 0; i < kWaveSteps; ++i)
        {
            const int j = i / kMs, m = i % kMs;  // 64-k group, and the k half within the wave's set
            const int cur = i & 1, nxt = cur ^ 1;
            if (i + 1 < kWaveSteps)
            {
                read_b(bf[nxt], slot + ln.b_off + ln.b_step[i + 1]);
            }
            else if (s + 1 < KT)
            {
                wait_lgkm0();  // this wave's reads of stage s have landed
                wait_stage_landed(min(KT - 2 - s, kSlots - 2));  // its part of stage s+1 has landed
                lds_barrier();  // all of stage s+1 is in LDS; nobody reads stage s's slot any more
                if (s + kSlots < KT) issue_loads(lds, d, s % kSlots, s + kSlots, KT, 0, kPartLoads);
                const uint8_t* nslot = lds + ((s + 1) % kSlots) * kSlotBytes;
                read_a(wa[P ^ 1], nslot + ln.a_off);
                read_b(bf[nxt], nslot + ln.b_off + ln.b_step[0]);
            }
            __builtin_amdgcn_sched_barrier(0);
            step_prio(i == kWaveSteps - 1 ? 0 : i + 1);
#pragma unroll
            for (int rb = 0; rb < kRB; ++rb)
            {
                const v4i a = (v4i)((__builtin_bit_cast(u32x4, wa[P][rb][m]) >> (2 * j)) & kM3);
#pragma unroll
                for (int n = 0; n < kTB; ++n) acc[rb][n] = mfma32(a, bf[cur][n], acc[rb][n]);
                if (rb == 0 && i + 1 < kDmaParts)
                {
                    // piece i+1 of the DMA of stage s+kSlots-1, whose first piece went out at the
                    // barrier of stage s-1 (stages below kSlots were issued whole in the prologue)
                    const int t = s + kSlots - 1;
                    __builtin_amdgcn_sched_barrier(0);
                    if (s >= 1 && t < KT)
                        issue_loads(lds, d, (s - 1) % kSlots, t, KT, (i + 1) * kPartLoads, (i + 2) * kPartLoads);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    // Epilogue operands of the row blocks a wave finishes (kRBf of them, from rb0 on), loaded
    // before the k-split exchange so that their latency hides behind it. The 32x32 accumulator
    // layout puts element i of lane l at row 8*(i/4) + 4*(l/32) + i%4, token l%32. Buffer loads:
    // rows past N and tokens past M read zero; without a bias the bias values are zero.
    static constexpr int kRBf = kRB / kKSplit;
    struct EpiOps
    {
        int rs2[kTB];        // 2 * rowsum of the lane's tokens
        float sv[kTB];       // activation scale of the lane's tokens
        float tv[kRBf][16];  // tau of the lane's accumulator rows
        float bv[kRBf][16];  // bias of the lane's accumulator rows
    };

    static __device__ __forceinline__ void load_epilogue(const GemvProblem& p, EpiOps& e, int rb0, int row_w, int tok_w, int h,
                                                  int l32)
    {
        const __amdgpu_buffer_rsrc_t rtau = rsrc(p.tau, (uint32_t)p.N * 4u);
        const __amdgpu_buffer_rsrc_t rs_r = rsrc(p.rowsum, (uint32_t)p.M * 4u);
        const __amdgpu_buffer_rsrc_t rs_s = rsrc(p.s, (uint32_t)p.M * 4u);
#pragma unroll
        for (int n = 0; n < kTB; ++n)
        {
            const uint32_t m = (uint32_t)(tok_w + n * 32 + l32);
            e.rs2[n] = 2 * __builtin_bit_cast(int, __builtin_amdgcn_raw_buffer_load_b32(rs_r, m * 4u, 0, 0));
            e.sv[n] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs_s, m * 4u, 0, 0));
        }
#pragma unroll
        for (int r = 0; r < kRBf; ++r)
        {
            const uint32_t row0 = (uint32_t)(row_w + (rb0 + r) * 32 + 4 * h);
#pragma unroll
            for (int i = 0; i < 16; ++i)
            {
                const uint32_t row = row0 + (uint32_t)(8 * (i >> 2) + (i & 3));
                e.tv[r][i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rtau, row * 4u, 0, 0));
            }
        }
        if (p.bias)
        {
            const __amdgpu_buffer_rsrc_t rbias = rsrc(p.bias, (uint32_t)p.N * 4u);
#pragma unroll
            for (int r = 0; r < kRBf; ++r)
            {
                const uint32_t row0 = (uint32_t)(row_w + (rb0 + r) * 32 + 4 * h);
#pragma unroll
                for (int i = 0; i < 16; ++i)
                {
                    const uint32_t row = row0 + (uint32_t)(8 * (i >> 2) + (i & 3));
                    e.bv[r][i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rbias, row * 4u, 0, 0));
                }
            }
        }
        else
        {
#pragma unroll
            for (int r = 0; r < kRBf; ++r)
#pragma unroll
                for (int i = 0; i < 16; ++i) e.bv[r][i] = 0.0f;
        }
    }

    // Index of row block rb (a compile-time loop index in [rb0, rb0 + nrb)) within EpiOps.
    static __device__ __forceinline__ int epi_slot(int rb) { return kRBf == 1 ? 0 : rb; }

    // Epilogue of a block that lies wholly inside Y: no masks; row offsets are scalar.
    template <bool kBias>
    static __device__ __forceinline__ void store_full(const GemvProblem& p, const v16i (&acc)[kRB][kTB], const EpiOps& e, int rb0,
                                               int nrb, int row_w, int tok_w, int h, int l32)
    {
        const __amdgpu_buffer_rsrc_t ry = rsrc(p.y, (uint32_t)p.N * (uint32_t)p.M * 4u);
        const uint32_t M4 = (uint32_t)p.M * 4u;
        // p.res: y + res[row][token], the residual read at the output's own index, all of a row
        // block's values requested in one round trip before the first add
        const bool has_res = p.res != nullptr;
        const __amdgpu_buffer_rsrc_t rres = rsrc(has_res ? p.res : p.y, has_res ? (uint32_t)p.N * (uint32_t)p.M * 4u : 0u);
#pragma unroll
        for (int rb = 0; rb < kRB; ++rb)
        {
            if (rb < rb0 || rb >= rb0 + nrb) continue;
            const int r = epi_slot(rb);
            const uint32_t row0 = (uint32_t)(row_w + rb * 32 + 4 * h);
            const uint32_t vbase = (row0 * (uint32_t)p.M + (uint32_t)(tok_w + l32)) * 4u;
#pragma unroll
            for (int i0 = 0; i0 < 16; i0 += 4)
            {
                // the residuals of 4 rows x kTB token groups in one round trip
                float rv[4][kTB];
                if (has_res)
                {
#pragma unroll
                    for (int j = 0; j < 4; ++j)
#pragma unroll
                        for (int n = 0; n < kTB; ++n)
                            rv[j][n] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                                     rres, vbase + (uint32_t)(n * 128),
                                                                     (8 * (i0 >> 2) + j) * (int)M4, 0));
                }
#pragma unroll
                for (int j = 0; j < 4; ++j)
                {
                    const int i = i0 + j;
                    const int soff = (8 * (i >> 2) + (i & 3)) * (int)M4;
#pragma unroll
                    for (int n = 0; n < kTB; ++n)
                    {
                        const int a = acc[rb][n][i] - e.rs2[n];
                        float y = (e.tv[r][i] * e.sv[n]) * (float)a;
                        if (kBias) y = y + e.bv[r][i];
                        if (has_res) y = y + rv[j][n];
                        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, y), ry,
                                                              vbase + (uint32_t)(n * 128), soff, kGemmYPolicy);
                    }
                }
            }
        }
    }

    // Epilogue of an edge block: rows past N and tokens past M are masked (their lanes store to
    // an out-of-range offset, which the buffer unit drops).
    static __device__ __forceinline__ void store_edge(const GemvProblem& p, const v16i (&acc)[kRB][kTB], const EpiOps& e, int rb0,
                                               int nrb, int row_w, int tok_w, int h, int l32)
    {
        const __amdgpu_buffer_rsrc_t ry = rsrc(p.y, (uint32_t)p.N * (uint32_t)p.M * 4u);
        // p.res: added per element (edge blocks are few; out-of-range lanes read 0 and store nothing)
        const __amdgpu_buffer_rsrc_t rres = rsrc(p.res ? p.res : p.y, p.res ? (uint32_t)p.N * (uint32_t)p.M * 4u : 0u);
#pragma unroll
        for (int rb = 0; rb < kRB; ++rb)
        {
            if (rb < rb0 || rb >= rb0 + nrb) continue;
            const int r = epi_slot(rb);
            const int row0 = row_w + rb * 32 + 4 * h;
#pragma unroll
            for (int n = 0; n < kTB; ++n)
            {
                const int m = tok_w + n * 32 + l32;
#pragma unroll
                for (int i = 0; i < 16; ++i)
                {
                    const int row = row0 + 8 * (i >> 2) + (i & 3);
                    const int a = acc[rb][n][i] - e.rs2[n];
                    float y = (e.tv[r][i] * e.sv[n]) * (float)a;
                    if (p.bias) y = y + e.bv[r][i];
                    const uint32_t off = (row < p.N && m < p.M) ? ((uint32_t)row * (uint32_t)p.M + (uint32_t)m) * 4u
                                                                 : 0xFFFFFFF0u;
                    if (p.res)
                        y = y + __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rres, off, 0, 0));
                    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, y), ry, off, 0, kGemmYPolicy);
                }
            }
        }
    }

    // Epilogue of the fused gated activation (p.glu != 0). Rows are in the interleaved GLU order
    // (16-row group t = gate rows of features 8t..8t+7, then their up rows), so accumulator element
    // i (row 8*(i/4) + 4h + i%4 of the 32-row block) and element i + 4 (8 rows below) are gate and
    // up of one feature when i/4 is even. Each is rescaled exactly as the plain epilogue does
    // ((tau * s) * float(acc) [+ bias]), then combined by glu_one; h (glu_F, M) gets the result.
    template <int kHPolicy>
    static __device__ __forceinline__ void store_glu(const GemvProblem& p, const v16i (&acc)[kRB][kTB], const EpiOps& e, int rb0,
                                              int nrb, int row_w, int tok_w, int h, int l32)
    {
        const __amdgpu_buffer_rsrc_t ry = rsrc(p.y, (uint32_t)p.glu_F * (uint32_t)p.M * 4u);
        const int act = p.glu - 1;
#pragma unroll
        for (int rb = 0; rb < kRB; ++rb)
        {
            if (rb < rb0 || rb >= rb0 + nrb) continue;
            const int r = epi_slot(rb);
            const int row0 = row_w + rb * 32 + 4 * h;
#pragma unroll
            for (int q = 0; q < 8; ++q)
            {
                const int i = (q / 4) * 8 + (q % 4);  // gate element: i / 4 in {0, 2}
                const uint32_t rg = (uint32_t)(row0 + 8 * (i >> 2) + (i & 3));
                const int f = 8 * (int)(rg / 16u) + (int)(rg % 16u);
#pragma unroll
                for (int n = 0; n < kTB; ++n)
                {
                    const int m = tok_w + n * 32 + l32;
                    float yg = (e.tv[r][i] * e.sv[n]) * (float)(acc[rb][n][i] - e.rs2[n]);
                    float yu = (e.tv[r][i + 4] * e.sv[n]) * (float)(acc[rb][n][i + 4] - e.rs2[n]);
                    if (p.bias)
                    {
                        yg = yg + e.bv[r][i];
                        yu = yu + e.bv[r][i + 4];
                    }
                    const float y = glu_one(yg, yu, act);
                    const bool in = f < p.glu_F && m < p.M;
                    const uint32_t off = in ? ((uint32_t)f * (uint32_t)p.M + (uint32_t)m) * 4u : 0xFFFFFFF0u;
                    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, y), ry, off, 0, kHPolicy);
                }
            }
        }
    }

    // k split: wave KS of a pair hands the partial sums of the row blocks its partner finishes to
    // the partner through LDS (put_partials), and after a barrier adds the partner's partials of
    // its own row blocks (add_partials).

    template <int KS>
    static __device__ __forceinline__ void put_partials(const v16i (&acc)[kRB][kTB], uint8_t* lds, int wave, int lane)
    {
        constexpr int kHalf = kRB / 2;
        v4i* mine = reinterpret_cast<v4i*>(lds + wave * kPartBytes);
#pragma unroll
        for (int r = 0; r < kHalf; ++r)
#pragma unroll
            for (int n = 0; n < kTB; ++n)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                {
                    const v16i& a = acc[(1 - KS) * kHalf + r][n];
                    mine[((r * kTB + n) * 4 + q) * 64 + lane] = v4i{a[4 * q], a[4 * q + 1], a[4 * q + 2], a[4 * q + 3]};
                }
    }

    template <int KS>
    static __device__ __forceinline__ void add_partials(v16i (&acc)[kRB][kTB], const uint8_t* lds, int wave, int lane)
    {
        constexpr int kHalf = kRB / 2;
        const v4i* theirs = reinterpret_cast<const v4i*>(lds + (wave ^ (kWavesN * kWavesM)) * kPartBytes);
#pragma unroll
        for (int r = 0; r < kHalf; ++r)
        {
            // all reads of the row block first (one LDS round trip), then the adds
            v4i o[kTB][4];
#pragma unroll
            for (int n = 0; n < kTB; ++n)
#pragma unroll
                for (int q = 0; q < 4; ++q) o[n][q] = theirs[((r * kTB + n) * 4 + q) * 64 + lane];
#pragma unroll
            for (int n = 0; n < kTB; ++n)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                {
                    v16i& a = acc[KS * kHalf + r][n];
                    a[4 * q] += o[n][q][0];
                    a[4 * q + 1] += o[n][q][1];
                    a[4 * q + 2] += o[n][q][2];
                    a[4 * q + 3] += o[n][q][3];
                }
        }
    }

    static __device__ __forceinline__ void body(const GemvProblem& p, int n_mblocks, int n_nblocks, int xcd_mode,
                                                bool h_keep)
    {
        extern __shared__ __align__(16) uint8_t lds[];
        const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
        const int wn = wave % kWavesN, wm = (wave / kWavesN) % kWavesM, ks = wave / (kWavesN * kWavesM);
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

        // ---- per-lane LDS read offsets
        const int h = lane >> 5, l32 = lane & 31;
        Lane ln;
        ln.a_off = (uint32_t)((wn * (kWaveRows / 16) + (l32 >> 4)) * 1024 + (16 * h + (l32 & 15)) * 16 +
                              (kKSplit == 2 ? ks * 512 : 0));
        ln.b_off = (uint32_t)(kABytes + (wm * kWaveToks + l32) * kTileK);
        const int rsw = h ^ (l32 & 15);  // token row % 16 is l32 % 16 for every token block
#pragma unroll
        for (int i = 0; i < kWaveSteps; ++i)
        {
            const int j = i / kMs, m = kKSplit == 2 ? ks : i % kMs;
            const int c0 = 4 * j + 2 * m;  // chunk of lane half 0 for step (j, m)
            ln.b_step[i] = (uint32_t)((c0 ^ rsw) << 4);
        }

        v16i acc[kRB][kTB];
#pragma unroll
        for (int i = 0; i < kRB; ++i)
#pragma unroll
            for (int n = 0; n < kTB; ++n) acc[i][n] = v16i{};

        // ---- prologue: three stages in flight, then stage 0's first reads
        issue_stage(lds, d, 0, 0, KT);
#pragma unroll
        for (int i = 1; i < kSlots; ++i)
            if (i < KT) issue_stage(lds, d, i, i, KT);
        wait_stage_landed(min(KT - 1, kSlots - 1));
        lds_barrier();
        v4i wa[2][kRB][kMs];
        v4i bf[2][kTB];
        read_a(wa[0], lds + ln.a_off);
        read_b(bf[0], lds + ln.b_off + ln.b_step[0]);

        int s = 0;
        for (; s + 1 < KT; s += 2)
        {
            run_stage<0>(s, KT, lds, d, ln, wa, bf, acc);
            run_stage<1>(s + 1, KT, lds, d, ln, wa, bf, acc);
        }
        if (s < KT) run_stage<0>(s, KT, lds, d, ln, wa, bf, acc);

        // ---- epilogue operands (issued before the k-split exchange, whose LDS round trip hides
        // their latency), then the exchange: the two waves of a pair swap partial sums through LDS;
        // wave ks finishes row blocks [ks * kRB / 2, (ks + 1) * kRB / 2).
        const int row_w = (rt0 + wn * (kWaveRows / 16)) * 16;
        const int tok_w = m0 + wm * kWaveToks;
        int rb0 = 0, nrb = kRB;
        if (kKSplit == 2)
        {
            rb0 = ks * (kRB / 2);
            nrb = kRB / 2;
        }
        wait_lgkm0();
        wait_vmcnt<0>();
        EpiOps e;
        load_epilogue(p, e, rb0, row_w, tok_w, h, l32);
        if (kKSplit == 2)
        {
            lds_barrier();  // every wave is done with the ring
            if (ks == 0) put_partials<0>(acc, lds, wave, lane);
            else put_partials<1>(acc, lds, wave, lane);
            lds_barrier();
            if (ks == 0) add_partials<0>(acc, lds, wave, lane);
            else add_partials<1>(acc, lds, wave, lane);
        }

        // ---- epilogue
        const bool full = rt0 * 16 + kBN <= p.N && m0 + kBM <= p.M;
        if (p.glu)
        {
            // one uniform branch over the whole epilogue (the store policy is an immediate)
            if (h_keep) store_glu<kPolicySys>(p, acc, e, rb0, nrb, row_w, tok_w, h, l32);
            else store_glu<kGemmYPolicy>(p, acc, e, rb0, nrb, row_w, tok_w, h, l32);
        }
        else if (full)
        {
            if (p.bias) store_full<true>(p, acc, e, rb0, nrb, row_w, tok_w, h, l32);
            else store_full<false>(p, acc, e, rb0, nrb, row_w, tok_w, h, l32);
        }
        else
        {
            store_edge(p, acc, e, rb0, nrb, row_w, tok_w, h, l32);
        }
    }
};

template <class G>
__global__ __launch_bounds__(G::kThreads) __attribute__((amdgpu_waves_per_eu(G::kWavesPerSimd, G::kWavesPerSimd))) void
k_gemm(GemvProblem p, int n_mblocks, int n_nblocks, int xcd_mode, int h_keep)
{
    G::body(p, n_mblocks, n_nblocks, xcd_mode, h_keep != 0);
}

}  // namespace

namespace
{

// The three block tiles: 256 x 128 (8 waves, k-split pairs, 2 slots) for large problems,
// 128 x 128 (8 waves, 64 x 64 per pair, 3 slots) and 64 x 64 (4 waves, one per SIMD, 6 slots:
// short stages need a deeper ring to cover memory latency) to spread small problems over the
// chip. gemm_tile_choice weighs block rounds over the CUs by the measured relative round times.
using GemmA = Gemm<256, 128, NNHIP_GEMM_WAVES_N, NNHIP_GEMM_WAVES_M, NNHIP_GEMM_KSPLIT, NNHIP_GEMM_SLOTS>;
using GemmB = Gemm<128, 128, 2, 2, 2, 3>;
using GemmC = Gemm<64, 64, 2, 2, 1, 6>;

template <class G>
hipError_t launch_cfg(hipStream_t st, const GemvProblem& p, bool h_keep)
{
    static bool attr_set = false;
    if (!attr_set)
    {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemm<G>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, G::kLdsBytes);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    const int n_mblocks = (int)ceil_div((size_t)p.M, G::kBM);
    const int n_nblocks = (int)ceil_div((size_t)p.N, G::kBN);
    const int xcd_mode = (n_mblocks % 8 == 0) ? 1 : 0;
    const unsigned blocks = (unsigned)(n_mblocks * n_nblocks);
    hipLaunchKernelGGL(k_gemm<G>, dim3(blocks), dim3(G::kThreads), G::kLdsBytes, st, p, n_mblocks, n_nblocks,
                       xcd_mode, h_keep ? 1 : 0);
    return hipGetLastError();
}

// Estimated time of a configuration in units of one 256 x 128 block: rounds of blocks over the
// CUs times the block time relative to the 256 x 128 one.
double gemm_cost(const GemvProblem& p, int num_cus, int bn, int bm, double rel)
{
    const size_t blocks = ceil_div((size_t)p.N, (size_t)bn) * ceil_div((size_t)p.M, (size_t)bm);
    return (double)ceil_div(blocks, (size_t)num_cus) * rel;
}

}  // namespace

int gemm_tile_choice(const GemvProblem& p, int num_cus)
{
    const int cus = num_cus > 0 ? num_cus : 256;
    const double a = gemm_cost(p, cus, GemmA::kBN, GemmA::kBM, 1.0);
    const double b = gemm_cost(p, cus, GemmB::kBN, GemmB::kBM, kGemmRelB);
    const double c = gemm_cost(p, cus, GemmC::kBN, GemmC::kBM, kGemmRelC);
    if (a <= b && a <= c) return NNHIP_GEMM_TILE_256x128;
    return b <= c ? NNHIP_GEMM_TILE_128x128 : NNHIP_GEMM_TILE_64x64;
}

namespace
{

// The rows [rows0, N) of p as a problem of their own: the weight row tiles, the per-row scales,
// bias and residual, and the output rows move; the per-token inputs (codes, scales, row sums) are
// shared. rows0 is a multiple of 256 (16 row tiles; 128 gated features).
GemvProblem gemm_rows_from(const GemvProblem& p, int rows0)
{
    GemvProblem q = p;
    const size_t rt0 = (size_t)rows0 / 16;
    q.rp = p.rp + rt0 * (size_t)p.KT * 64;  // 1024 bytes = 64 x 16 per (row tile, k tile)
    q.tau = p.tau + rows0;
    if (p.bias) q.bias = p.bias + rows0;
    q.N = p.N - rows0;
    if (p.glu)
    {
        q.glu_F = p.glu_F - rows0 / 2;
        q.y = p.y + (size_t)(rows0 / 2) * (size_t)p.M;
    }
    else
    {
        q.y = p.y + (size_t)rows0 * (size_t)p.M;
        if (p.res) q.res = p.res + (size_t)rows0 * (size_t)p.M;
    }
    return q;
}

}  // namespace

GemmSplit gemm_split_choice(const GemvProblem& p, int num_cus)
{
    GemmSplit s{gemm_tile_choice(p, num_cus), 0, 0};
    const int cus = num_cus > 0 ? num_cus : 256;
    const int n_mb = (int)ceil_div((size_t)p.M, (size_t)GemmA::kBM);
    const int n_nb = (int)ceil_div((size_t)p.N, (size_t)GemmA::kBN);
    // the longest row-block prefix whose 256 x 128 blocks fill whole rounds of the CUs
    int r1 = n_nb - 1;
    while (r1 > 0 && ((long)r1 * n_mb) % cus != 0) --r1;
    if (r1 <= 0) return s;
    const double best = s.tile == NNHIP_GEMM_TILE_256x128   ? gemm_cost(p, cus, GemmA::kBN, GemmA::kBM, 1.0)
                        : s.tile == NNHIP_GEMM_TILE_128x128 ? gemm_cost(p, cus, GemmB::kBN, GemmB::kBM, kGemmRelB)
                                                            : gemm_cost(p, cus, GemmC::kBN, GemmC::kBM, kGemmRelC);
    const GemvProblem tail = gemm_rows_from(p, r1 * GemmA::kBN);
    const double tb = gemm_cost(tail, cus, GemmB::kBN, GemmB::kBM, kGemmRelB);
    const double tc = gemm_cost(tail, cus, GemmC::kBN, GemmC::kBM, kGemmRelC);
    const double split = (double)((long)r1 * n_mb / cus) + (tb <= tc ? tb : tc) + kGemmSplitCost;
    if (split < best) s = GemmSplit{NNHIP_GEMM_TILE_256x128, r1 * GemmA::kBN,
                                    tb <= tc ? NNHIP_GEMM_TILE_128x128 : NNHIP_GEMM_TILE_64x64};
    return s;
}

namespace
{

hipError_t launch_tile(hipStream_t st, const GemvProblem& p, int tile, bool h_keep)
{
    if (tile == NNHIP_GEMM_TILE_128x128) return launch_cfg<GemmB>(st, p, h_keep);
    if (tile == NNHIP_GEMM_TILE_64x64) return launch_cfg<GemmC>(st, p, h_keep);
    return launch_cfg<GemmA>(st, p, h_keep);
}

}  // namespace

hipError_t launch_gemm(hipStream_t st, const GemvProblem& p, int num_cus, int tile)
{
    if (p.N == 0 || p.M == 0) return hipSuccess;
    const bool h_keep = p.glu && (size_t)p.glu_F * (size_t)p.M * 4 <= kGemmHKeepBytes;
    if (tile == NNHIP_GEMM_TILE_AUTO)
    {
        const GemmSplit s = gemm_split_choice(p, num_cus);
        if (s.rows > 0)
        {
            GemvProblem head = p;
            head.N = s.rows;
            if (p.glu) head.glu_F = s.rows / 2;
            const hipError_t e = launch_cfg<GemmA>(st, head, h_keep);
            if (e != hipSuccess) return e;
            return launch_tile(st, gemm_rows_from(p, s.rows), s.tail_tile, h_keep);
        }
        tile = s.tile;
    }
    return launch_tile(st, p, tile, h_keep);
}

}  // namespace nnhip
