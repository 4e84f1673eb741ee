// k_ternary.hip — ternary x int8 kernels for gfx950: the load-time repacker and the
// MFMA prefill GEMM (the decode GEMV is in k_gemv.hip).
//
// Weights use the T16K256 layout (see include/nnhip.h, oracle/nn_oracle.c): one 1 KiB tile
// per 16 rows x 256 k, whose 64 lanes x 16 bytes are exactly the A operands of four
// v_mfma_i32_16x16x64_i8: for MFMA j (j = 0..3) lane l = 16g + r contributes the 16 codes
// (word_q >> 2j) & 0x03030303, q = 0..3, i.e. row r, k = 256kt + 64j + 16g + 0..15 in
// natural byte order; the B operand of lane l = 16g + t is the 16 activation bytes of
// token t at the same k. Codes are trit + 2 in {1,2,3}, so each MFMA accumulates
// sum(code * x) and the epilogue subtracts 2 * rowsum (rowsum = sum_k x for the token):
//     acc = sum_k (code - 2) * x = sum_k trit * x,   exact in int32.
// Epilogue (reference order, src/int8_act_test.cpp:233): y = (tau[n] * s[m]) * float(acc),
// then y + bias[n] as a separate rounding.
#include "common.hpp"

namespace nnhip
{
namespace
{

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr uint32_t kM3 = 0x03030303u;

__device__ __forceinline__ v4i mfma16(v4i a, v4i b, v4i c)
{
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// ------------------------------------------------------------------ repack / unrepack

// One thread per output word (rt, kt, lane l = 16g + r, q).
__global__ __launch_bounds__(256) void k_repack(const uint32_t* __restrict__ wq, size_t N, size_t K,
                                                size_t RT, size_t KT, uint32_t* __restrict__ rp)
{
    const size_t wpr = ceil_div(K, 16);
    const size_t total = RT * KT * kTileWords;
    for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (size_t)gridDim.x * blockDim.x)
    {
        const size_t tile = idx / kTileWords, within = idx % kTileWords;
        const size_t rt = tile / KT, kt = tile % KT;
        const size_t l = within / 4, q = within % 4;
        const size_t g = l / 16, r = l % 16;
        const size_t n = rt * 16 + r;
        uint32_t word = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j)
        {
            // k = 256kt + 64j + 16g + 4q + b, b = 0..3: all inside source word (k / 16)
            const size_t sw = 16 * kt + 4 * j + g;
            const uint32_t src = (n < N && sw < wpr) ? wq[n * wpr + sw] : 0xAAAAAAAAu;  // code 2
            const uint32_t codes = src >> (8 * q);  // codes for b = 0..3 in bits 2b
#pragma unroll
            for (int b = 0; b < 4; ++b) word |= ((codes >> (2 * b)) & 3u) << (8 * b + 2 * j);
        }
        rp[idx] = word;
    }
}

// One thread per reference word (n, wi): k = 16wi + e lives in lane 16*(wi%4) + r of tile
// (n/16, wi/16), at j = (wi%16)/4, word q = e/4, byte b = e%4.
__global__ __launch_bounds__(256) void k_unrepack(const uint32_t* __restrict__ rp, size_t N, size_t K,
                                                  size_t KT, uint32_t* __restrict__ wq)
{
    const size_t wpr = ceil_div(K, 16);
    const size_t total = N * wpr;
    for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (size_t)gridDim.x * blockDim.x)
    {
        const size_t n = idx / wpr, wi = idx % wpr;
        const size_t rt = n / 16, r = n % 16, kt = wi / 16, j = (wi % 16) / 4, g = wi % 4;
        const size_t l = 16 * g + r;
        const u32x4 src = reinterpret_cast<const u32x4*>(rp)[(rt * KT + kt) * 64 + l];
        const uint32_t s4[4] = {src.x, src.y, src.z, src.w};
        uint32_t word = 0;
#pragma unroll
        for (int e = 0; e < 16; ++e)
        {
            const uint32_t code = (s4[e / 4] >> (8 * (e % 4) + 2 * j)) & 3u;
            word |= code << (2 * e);
        }
        wq[idx] = word;
    }
}

// ------------------------------------------------------------------ prefill GEMM
//
// Block = 4 waves (2 x 2), block tile 128 rows x 128 tokens, wave tile 64 rows (4 row
// tiles) x 64 tokens (4 token tiles) = 16 MFMA output tiles of 16x16.
// Per 256-wide k tile:
//   * B (128 tokens x 256 bytes = 32 KiB) is staged in LDS, double-buffered, with the
//     16-byte chunk c of token row `tok` stored at chunk position c ^ (tok & 15) so the
//     ds_read_b128 of 16 lanes (16 tokens, same chunk) hit 16 distinct bank groups;
//   * A comes straight from the T16K256 tiles (one coalesced 16-byte load per lane per
//     row tile) and is unpacked in registers: a_j = (w >> 2j) & 0x03030303;
//   * the next k tile's A and B are loaded into registers while this one computes.
constexpr int kGemmBN = 128, kGemmBM = 128;
constexpr int kGemmThreads = 256;
constexpr int kBTileBytes = kGemmBM * kTileK;  // 32 KiB

__global__ __launch_bounds__(kGemmThreads) void k_gemm(GemvProblem p)
{
    extern __shared__ __align__(16) uint8_t lds[];  // 2 x 32 KiB
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int wn = wid & 1, wm = wid >> 1;
    const int g = lane >> 4, t = lane & 15;
    const int RT = (p.N + 15) / 16;
    const size_t Kp = (size_t)p.KT * kTileK;
    const int m0 = blockIdx.y * kGemmBM;
    const int rt0 = blockIdx.x * (kGemmBN / 16) + wn * 4;

    // global -> register staging of B: thread handles chunks ci = tid + 256*v, v = 0..7
    uint4 bstage[8];
    auto load_b = [&](int kt) {
#pragma unroll
        for (int v = 0; v < 8; ++v)
        {
            const int ci = tid + kGemmThreads * v;
            const int tok = ci >> 4, c = ci & 15;
            const int m = m0 + tok;
            if (m < p.M)
                bstage[v] = *reinterpret_cast<const uint4*>(p.xi + (size_t)m * Kp + (size_t)kt * kTileK +
                                                            c * 16);
            else
                bstage[v] = make_uint4(0, 0, 0, 0);
        }
    };
    auto store_b = [&](int buf) {
        uint8_t* base = lds + buf * kBTileBytes;
#pragma unroll
        for (int v = 0; v < 8; ++v)
        {
            const int ci = tid + kGemmThreads * v;
            const int tok = ci >> 4, c = ci & 15;
            *reinterpret_cast<uint4*>(base + tok * kTileK + ((c ^ (tok & 15)) << 4)) = bstage[v];
        }
    };
    u32x4 astage[4];
    auto load_a = [&](int kt) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
        {
            const int rt = rt0 + i;
            const u32x4 code2 = {0xAAAAAAAAu, 0xAAAAAAAAu, 0xAAAAAAAAu, 0xAAAAAAAAu};
            astage[i] = rt < RT ? p.rp[((size_t)rt * p.KT + kt) * 64 + lane] : code2;
        }
    };

    v4i acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int n = 0; n < 4; ++n) acc[i][n] = v4i{0, 0, 0, 0};

    load_b(0);
    load_a(0);
    store_b(0);
    __syncthreads();

    for (int kt = 0; kt < p.KT; ++kt)
    {
        const int buf = kt & 1;
        u32x4 acur[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) acur[i] = astage[i];
        if (kt + 1 < p.KT)
        {
            load_b(kt + 1);
            load_a(kt + 1);
        }
        const uint8_t* bl = lds + buf * kBTileBytes;
#pragma unroll
        for (int j = 0; j < 4; ++j)
        {
            v4i bf[4];
#pragma unroll
            for (int n = 0; n < 4; ++n)
            {
                const int tok = wm * 64 + n * 16 + t;
                const int c = 4 * j + g;
                bf[n] = *reinterpret_cast<const v4i*>(bl + tok * kTileK + ((c ^ (tok & 15)) << 4));
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
            {
                const u32x4 w = acur[i];
                const v4i a = v4i{(int)((w.x >> (2 * j)) & kM3), (int)((w.y >> (2 * j)) & kM3),
                                  (int)((w.z >> (2 * j)) & kM3), (int)((w.w >> (2 * j)) & kM3)};
#pragma unroll
                for (int n = 0; n < 4; ++n) acc[i][n] = mfma16(a, bf[n], acc[i][n]);
            }
        }
        if (kt + 1 < p.KT)
        {
            store_b(buf ^ 1);
            __syncthreads();
        }
    }

    // epilogue: lane (g, t) of output tile (i, n) holds rows 4g..4g+3, token t
#pragma unroll
    for (int n = 0; n < 4; ++n)
    {
        const int m = m0 + wm * 64 + n * 16 + t;
        if (m >= p.M) continue;
        const int rs2 = 2 * p.rowsum[m];
        const float sv = p.s[m];
#pragma unroll
        for (int i = 0; i < 4; ++i)
        {
#pragma unroll
            for (int r = 0; r < 4; ++r)
            {
                const int row = (rt0 + i) * 16 + 4 * g + r;
                if (row < p.N)
                {
                    const int a = acc[i][n][r] - rs2;
                    float y = __fmul_rn(__fmul_rn(p.tau[row], sv), (float)a);
                    if (p.bias) y = __fadd_rn(y, p.bias[row]);
                    p.y[(size_t)row * p.M + m] = y;
                }
            }
        }
    }
}

inline unsigned grid_cap(size_t n)
{
    size_t g = n < 1 ? 1 : n;
    if (g > (1u << 20)) g = 1u << 20;
    return (unsigned)g;
}

}  // namespace

hipError_t launch_repack(hipStream_t st, const uint32_t* wq, size_t N, size_t K, uint32_t* rp)
{
    const size_t RT = ceil_div(N, 16), KT = ceil_div(K, kTileK);
    const size_t total = RT * KT * kTileWords;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(k_repack, dim3(grid_cap(ceil_div(total, 256))), dim3(256), 0, st, wq, N, K, RT,
                       KT, rp);
    return hipGetLastError();
}

hipError_t launch_unrepack(hipStream_t st, const uint32_t* rp, size_t N, size_t K, uint32_t* wq)
{
    const size_t KT = ceil_div(K, kTileK);
    const size_t total = N * ceil_div(K, 16);
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(k_unrepack, dim3(grid_cap(ceil_div(total, 256))), dim3(256), 0, st, rp, N, K, KT,
                       wq);
    return hipGetLastError();
}

hipError_t launch_gemm(hipStream_t st, const GemvProblem& p, int /*num_cus*/)
{
    if (p.N == 0 || p.M == 0) return hipSuccess;
    const unsigned gx = (unsigned)ceil_div((size_t)p.N, kGemmBN);
    const unsigned gy = (unsigned)ceil_div((size_t)p.M, kGemmBM);
    hipLaunchKernelGGL(k_gemm, dim3(gx, gy), dim3(kGemmThreads), 2 * kBTileBytes, st, p);
    return hipGetLastError();
}

}  // namespace nnhip
