// k_matq.hip — ternary x float GEMM on the reference packed container (f32 or f16
// activations, f32 accumulation): the reference's default BitLinear branch and its dX path.
//
//   matmul_q   Y (N, M)  = (tau o trit(wq)) . B,        wq (N, ceil(K/16)), B (K, M)
//   matmul_q_t Y (M, N)  = (tau o trit(A))^T . B,       A  (K, ceil(M/16)), B (K, N), tau per
//                                                        stored row k
//
// Both are HBM-bound GEMV shapes at decode (few tokens / few columns): the packed weights are
// read once (0.25 B per weight), the activations come from L2. The accumulation order is a
// lane-strided sum (lane l takes every 64th word or row) followed by a xor butterfly; the
// reference does not pin its order, only a tolerance of 1e-4 x max(1, |Y|) in f32
// (src/ternary_gemm_test.cpp:523-526).
#include "common.hpp"

namespace nnhip
{
namespace
{

constexpr int kMqBlock = 256;  // 4 waves
constexpr int kMqTok = 4;      // tokens (columns of B) per wave

__device__ __forceinline__ float load_act(const void* B, size_t idx, bool f16)
{
    return f16 ? (float)reinterpret_cast<const _Float16*>(B)[idx] : reinterpret_cast<const float*>(B)[idx];
}

__device__ __forceinline__ void store_out(void* Y, size_t idx, float v, bool f16)
{
    if (f16) reinterpret_cast<_Float16*>(Y)[idx] = (_Float16)v;
    else reinterpret_cast<float*>(Y)[idx] = v;
}

__device__ __forceinline__ float wave_fsum(float v)
{
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// One wave per (row n, chunk of kMqTok tokens); lane l sums the 16 k of words l, l+64, ...
__global__ __launch_bounds__(kMqBlock) void k_matmul_q(const uint32_t* __restrict__ wq, const float* __restrict__ tau,
                                                       const void* __restrict__ B, bool b16, size_t N, size_t K,
                                                       size_t M, void* __restrict__ Y, bool y16)
{
    const int lane = threadIdx.x & 63;
    const size_t n = (size_t)blockIdx.x * (kMqBlock / kWave) + (threadIdx.x >> 6);
    const size_t m0 = (size_t)blockIdx.y * kMqTok;
    if (n >= N) return;
    const size_t wpr = ceil_div(K, 16);
    const int mc = (int)(M - m0 < (size_t)kMqTok ? M - m0 : kMqTok);
    float acc[kMqTok] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (size_t w = (size_t)lane; w < wpr; w += kWave)
    {
        const uint32_t word = wq[n * wpr + w];
#pragma unroll
        for (int i = 0; i < 16; ++i)
        {
            const size_t k = 16 * w + (size_t)i;
            if (k >= K) break;
            const float t = (float)((int)((word >> (2 * i)) & 3u) - 2);
#pragma unroll
            for (int mm = 0; mm < kMqTok; ++mm)
                if (mm < mc) acc[mm] = __builtin_fmaf(t, load_act(B, k * M + m0 + mm, b16), acc[mm]);
        }
    }
#pragma unroll
    for (int mm = 0; mm < kMqTok; ++mm) acc[mm] = wave_fsum(acc[mm]);
    if (lane == 0)
        for (int mm = 0; mm < mc; ++mm) store_out(Y, n * M + m0 + mm, tau[n] * acc[mm], y16);
}

// One wave per (16 output rows m = 16c.., chunk of kMqTok columns of B); lane l takes stored
// rows k = l, l+64, ...: word A[k][c] holds trit(k, 16c + i) in bits 2i.
__global__ __launch_bounds__(kMqBlock) void k_matmul_q_t(const uint32_t* __restrict__ A, const float* __restrict__ tau,
                                                         const void* __restrict__ B, bool b16, size_t K, size_t M,
                                                         size_t N, void* __restrict__ Y, bool y16)
{
    const int lane = threadIdx.x & 63;
    const size_t c = (size_t)blockIdx.x * (kMqBlock / kWave) + (threadIdx.x >> 6);
    const size_t n0 = (size_t)blockIdx.y * kMqTok;
    const size_t wpa = ceil_div(M, 16);
    if (c >= wpa) return;
    const int nc = (int)(N - n0 < (size_t)kMqTok ? N - n0 : kMqTok);
    float acc[16][kMqTok];
#pragma unroll
    for (int i = 0; i < 16; ++i)
#pragma unroll
        for (int j = 0; j < kMqTok; ++j) acc[i][j] = 0.0f;
    for (size_t k = (size_t)lane; k < K; k += kWave)
    {
        const uint32_t word = A[k * wpa + c];
        const float tk = tau[k];
        float b[kMqTok];
#pragma unroll
        for (int j = 0; j < kMqTok; ++j) b[j] = j < nc ? load_act(B, k * N + n0 + j, b16) : 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i)
        {
            const float tt = tk * (float)((int)((word >> (2 * i)) & 3u) - 2);  // exact: trit in {-1,0,1}
#pragma unroll
            for (int j = 0; j < kMqTok; ++j) acc[i][j] = __builtin_fmaf(tt, b[j], acc[i][j]);
        }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i)
#pragma unroll
        for (int j = 0; j < kMqTok; ++j) acc[i][j] = wave_fsum(acc[i][j]);
    if (lane < 16)
    {
        const size_t m = 16 * c + (size_t)lane;
        if (m < M)
#pragma unroll
            for (int i = 0; i < 16; ++i)
                if (i == lane)
                    for (int j = 0; j < nc; ++j) store_out(Y, m * N + n0 + j, acc[i][j], y16);
    }
}

}  // namespace

hipError_t launch_matmul_q(hipStream_t st, const uint32_t* wq, const float* tau, const void* B, bool b16, size_t N,
                           size_t K, size_t M, void* Y, bool y16)
{
    if (N == 0 || M == 0) return hipSuccess;
    const dim3 grid((unsigned)ceil_div(N, (size_t)(kMqBlock / kWave)), (unsigned)ceil_div(M, (size_t)kMqTok));
    hipLaunchKernelGGL(k_matmul_q, grid, dim3(kMqBlock), 0, st, wq, tau, B, b16, N, K, M, Y, y16);
    return hipGetLastError();
}

hipError_t launch_matmul_q_t(hipStream_t st, const uint32_t* A, const float* tau, const void* B, bool b16, size_t K,
                             size_t M, size_t N, void* Y, bool y16)
{
    if (N == 0 || M == 0) return hipSuccess;
    const dim3 grid((unsigned)ceil_div(ceil_div(M, 16), (size_t)(kMqBlock / kWave)), (unsigned)ceil_div(N, (size_t)kMqTok));
    hipLaunchKernelGGL(k_matmul_q_t, grid, dim3(kMqBlock), 0, st, A, tau, B, b16, K, M, N, Y, y16);
    return hipGetLastError();
}

}  // namespace nnhip
