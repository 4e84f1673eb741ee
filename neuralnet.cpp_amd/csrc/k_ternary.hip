// k_ternary.hip — the load-time repacker of packed ternary weights into the T16K256 tile
// layout read by the decode GEMV (k_gemv.hip) and the prefill GEMM (k_gemm.hip).
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

}  // namespace nnhip
