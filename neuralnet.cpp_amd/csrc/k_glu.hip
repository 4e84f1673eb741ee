// k_glu.hip — gated activations of the W1.58A8 feed-forward block (SwiGLU, ReLU^2-GLU) and
// the load-time interleave of a fused gate/up weight container.
//
// SwiGLU   h = (g * (1 / (1 + exp(-g)))) * u   include/neuralnet.cpp/compute_layer_mlp.hpp:317-328
// ReLU2GLU h = (r * r) * u, r = g > 0 ? g : 0  include/neuralnet.cpp/compute_layer_mlp.hpp:405-414
// evaluated in that order with IEEE-rounded operations (the build uses -ffp-contract=off).
// exp is glu_exp (common.hpp), so the kernels and the prefill GEMM's fused epilogue produce
// the same bits.
//
// Interleaved ("GLU") row order: 16-row group t holds gate rows 8t .. 8t+7, then up rows
// 8t .. 8t+7, so one T16K256 row tile carries both inputs of 8 features and the GEMM epilogue
// finds gate and up of a feature in the same lane. Rows of features >= F are padding
// (code 2 = trit 0, tau 0, bias 0).
#include "common.hpp"

namespace nnhip
{
namespace
{

__device__ __forceinline__ long glu_src_row(size_t r, size_t F)
{
    const size_t t = r / 16, i = r % 16;
    const size_t f = 8 * t + (i % 8);
    if (f >= F) return -1;
    return (long)(i < 8 ? f : F + f);
}

// One thread per (feature f, token m). interleaved: Y1 rows are in the GLU order, else gate
// rows [0, F) and up rows [F, 2F).
__global__ __launch_bounds__(256) void k_glu(const float* __restrict__ Y1, size_t F, size_t M, int act,
                                             bool interleaved, float* __restrict__ h)
{
    const size_t total = F * M;
    for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (size_t)gridDim.x * blockDim.x)
    {
        const size_t f = idx / M, m = idx % M;
        const size_t rg = interleaved ? 16 * (f / 8) + f % 8 : f;
        const size_t ru = interleaved ? rg + 8 : F + f;
        h[idx] = glu_one(Y1[rg * M + m], Y1[ru * M + m], act);
    }
}

// One thread per (interleaved row r, word w); thread w == 0 also moves tau / bias.
__global__ __launch_bounds__(256) void k_glu_interleave(const uint32_t* __restrict__ wq, const float* __restrict__ tau,
                                                        const float* __restrict__ bias, size_t F, size_t K,
                                                        uint32_t* __restrict__ wq_out, float* __restrict__ tau_out,
                                                        float* __restrict__ bias_out)
{
    const size_t wpr = ceil_div(K, 16), rows = 2 * round_up(F, 8);
    const size_t total = rows * wpr;
    for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (size_t)gridDim.x * blockDim.x)
    {
        const size_t r = idx / wpr, w = idx % wpr;
        const long src = glu_src_row(r, F);
        wq_out[idx] = src < 0 ? 0xAAAAAAAAu : wq[(size_t)src * wpr + w];
        if (w == 0)
        {
            tau_out[r] = src < 0 ? 0.0f : tau[src];
            if (bias_out) bias_out[r] = (src < 0 || !bias) ? 0.0f : bias[src];
        }
    }
}

unsigned grid_for(size_t n)
{
    const size_t b = ceil_div(n, (size_t)256);
    return (unsigned)(b < 8192 ? (b < 1 ? 1 : b) : 8192);
}

}  // namespace

hipError_t launch_glu(hipStream_t st, const float* Y1, size_t F, size_t M, int act, bool interleaved, float* h)
{
    if (F == 0 || M == 0) return hipSuccess;
    hipLaunchKernelGGL(k_glu, dim3(grid_for(F * M)), dim3(256), 0, st, Y1, F, M, act, interleaved, h);
    return hipGetLastError();
}

hipError_t launch_glu_interleave(hipStream_t st, const uint32_t* wq, const float* tau, const float* bias, size_t F,
                                 size_t K, uint32_t* wq_out, float* tau_out, float* bias_out)
{
    const size_t n = 2 * round_up(F, 8) * ceil_div(K, 16);
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_glu_interleave, dim3(grid_for(n)), dim3(256), 0, st, wq, tau, bias, F, K, wq_out, tau_out,
                       bias_out);
    return hipGetLastError();
}

}  // namespace nnhip
