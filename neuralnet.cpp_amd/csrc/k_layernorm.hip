// k_layernorm.hip — LayerNorm over the features of each token, on (F, M) feature-major
// activations: the reference's default SubLN norm type (FeedForward's subln_norm_type,
// include/neuralnet.cpp/compute_layer_feedforward.hpp:50-65) and its LayerNorm layer
// (include/neuralnet.cpp/compute_layer_mlp.hpp:462-545):
//   mean = sum_f x * fl(1/F); d = x - mean; var = sum_f d * d
//   sinv = 1 / sqrt(var * fl(1/F) + eps); out = (d * sinv) * gamma[f] + beta[f]
// every step rounded to fp32 (no contraction). The two sums run in one fixed order: 8 strided
// parts (part p holds the features f = p, p + 8, ... in ascending order), then the tree
// ((p0 + p1) + (p2 + p3)) + ((p4 + p5) + (p6 + p7)); oracle/nn_oracle.c restates that order.
//
// A 256-thread block holds 32 consecutive tokens: thread (part p, token t) = (tid / 32, tid % 32),
// so one wave reads 128 contiguous bytes of two feature rows per load. Three passes over the
// block's columns (sum, squared deviations, output); nothing is kept between them but the two
// per-token statistics in LDS. Not a hot path of this build: no fused int8 form.
#include "common.hpp"
#include "token_quant.hpp"

namespace nnhip
{
namespace
{

constexpr int kLnParts = 8, kLnTok = 32, kLnThreads = kLnParts * kLnTok;

__device__ __forceinline__ float ln_tree(const float (&v)[kLnParts][kLnTok], int t)
{
    const float a = __fadd_rn(__fadd_rn(v[0][t], v[1][t]), __fadd_rn(v[2][t], v[3][t]));
    const float b = __fadd_rn(__fadd_rn(v[4][t], v[5][t]), __fadd_rn(v[6][t], v[7][t]));
    return __fadd_rn(a, b);
}

__global__ __launch_bounds__(kLnThreads) void k_layernorm(const float* __restrict__ X, const float* __restrict__ gamma,
                                                          const float* __restrict__ beta, float eps, float inv_f,
                                                          int F, int M, float* __restrict__ out)
{
    __shared__ float part[kLnParts][kLnTok];
    __shared__ float stat[2][kLnTok];  // mean, 1 / sqrt(var / F + eps)
    const int t = threadIdx.x % kLnTok, p = threadIdx.x / kLnTok;
    const int m = blockIdx.x * kLnTok + t;
    const bool live = m < M;
    const size_t ld = (size_t)M;

    float s = 0.0f;
    if (live)
        for (int f = p; f < F; f += kLnParts) s = __fadd_rn(s, X[(size_t)f * ld + m]);
    part[p][t] = s;
    __syncthreads();
    if (p == 0) stat[0][t] = __fmul_rn(ln_tree(part, t), inv_f);
    __syncthreads();  // part is read before it is written again below
    const float mean = stat[0][t];

    float q = 0.0f;
    if (live)
        for (int f = p; f < F; f += kLnParts)
        {
            const float d = __fsub_rn(X[(size_t)f * ld + m], mean);
            q = __fadd_rn(q, __fmul_rn(d, d));
        }
    part[p][t] = q;
    __syncthreads();
    if (p == 0) stat[1][t] = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(__fmul_rn(ln_tree(part, t), inv_f), eps)));
    __syncthreads();
    const float sinv = stat[1][t];

    if (live)
        for (int f = p; f < F; f += kLnParts)
        {
            const size_t i = (size_t)f * ld + m;
            const float nrm = __fmul_rn(__fsub_rn(X[i], mean), sinv);
            out[i] = __fadd_rn(__fmul_rn(nrm, gamma[f]), beta[f]);
        }
}

}  // namespace

hipError_t launch_layernorm(hipStream_t st, const float* X, const float* gamma, const float* beta, float eps,
                            size_t F, size_t M, float* out)
{
    if (F == 0 || M == 0) return hipSuccess;
    const unsigned grid = (unsigned)ceil_div(M, (size_t)kLnTok);
    hipLaunchKernelGGL(k_layernorm, dim3(grid), dim3(kLnThreads), 0, st, X, gamma, beta, eps, 1.0f / (float)F, (int)F,
                       (int)M, out);
    return hipGetLastError();
}

}  // namespace nnhip
