// k_act.hip — activation-side kernels: fused [RMSNorm ->] per-token absmax -> int8
// quantization into the token-major layout the ternary GEMV/GEMM read, RMSNorm alone,
// and conversions between that layout and the reference int8 container.
//
// Both fused kernels evaluate the per-token sum of squares in one fixed order, the same
// as the oracle: 64 strided parts (feature f in part f % 64), each summed in ascending f,
// then the xor butterfly over 32,16,8,4,2,1. So the normalized values, the scale and the
// int8 codes are bit-identical to the unfused reference sequence.
#include "common.hpp"

#include <cmath>

namespace nnhip
{
namespace
{

constexpr int kBlock = 256;

__device__ __forceinline__ int quantize_one(float x, float s)
{
    if (s == 0.0f || isnan(x)) return 0;
    float v = __fdiv_rn(x, s);
    if (isnan(v)) return 0;
    v = fminf(fmaxf(v, -127.0f), 127.0f);
    return (int)roundf(v);
}

// Correctly rounded fp32 square root. v_sqrt_f32 alone is accurate to 1 ulp; the two
// fma residuals pick between its neighbours (the same correction LLVM's IEEE fsqrt
// lowering applies), so the result matches a host sqrtf bit for bit. Inputs here are
// ms + eps >= eps > 0 and far from the denormal range.
__device__ __forceinline__ float sqrt_rn(float v)
{
    float s = __builtin_sqrtf(v);
    if (!(v > 0.0f) || isinf(v)) return s;
    const float s_dn = __int_as_float(__float_as_int(s) - 1);
    const float s_up = __int_as_float(__float_as_int(s) + 1);
    const float r_dn = __builtin_fmaf(-s_dn, s, v);
    const float r_up = __builtin_fmaf(-s_up, s, v);
    if (r_dn <= 0.0f) s = s_dn;
    if (r_up > 0.0f) s = s_up;
    return s;
}

__device__ __forceinline__ float wave_max(float v)
{
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1)
    {
        const float o = __shfl_xor(v, off, kWave);
        v = o > v ? o : v;
    }
    return v;
}

__device__ __forceinline__ int wave_sum_i(int v)
{
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// out = (x * ri) * gamma  (two roundings, as RMSNorm's normed * gamma)
__device__ __forceinline__ float norm_val(float x, float ri, const float* gamma, size_t f, bool norm)
{
    if (!norm) return x;
    return __fmul_rn(__fmul_rn(x, ri), gamma[f]);
}

// ---------------------------------------------------------------------------------------
// Small M: one wave per token, lane l owns features l, l+64, ...
// mode: 0 = quantize (xi/s/rowsum/xq_ref), 1 = write normalized floats to `fout`.
__global__ __launch_bounds__(kBlock) void k_token_wave(const float* __restrict__ X,
                                                       const float* __restrict__ gamma, bool norm,
                                                       float eps, float inv_f, size_t K, size_t M,
                                                       size_t Kp, int mode, int8_t* __restrict__ xi,
                                                       float* __restrict__ s, int32_t* __restrict__ rowsum,
                                                       uint32_t* __restrict__ xq_ref,
                                                       float* __restrict__ fout)
{
    const int lane = threadIdx.x & 63;
    const size_t m = (size_t)blockIdx.x * (kBlock / kWave) + (threadIdx.x >> 6);
    if (m >= M) return;

    float ri = 1.0f;
    if (norm)
    {
        float part = 0.0f;
        for (size_t f = (size_t)lane; f < K; f += kWave)
        {
            const float x = X[f * M + m];
            part = __fadd_rn(part, __fmul_rn(x, x));
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) part = __fadd_rn(part, __shfl_xor(part, off, kWave));
        ri = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(__fmul_rn(part, inv_f), eps)));
    }

    if (mode == 1)
    {
        for (size_t f = (size_t)lane; f < K; f += kWave)
            fout[f * M + m] = norm_val(X[f * M + m], ri, gamma, f, norm);
        return;
    }

    float mx = 0.0f;
    for (size_t f = (size_t)lane; f < K; f += kWave)
    {
        const float a = fabsf(norm_val(X[f * M + m], ri, gamma, f, norm));
        mx = a > mx ? a : mx;
    }
    mx = wave_max(mx);
    const float sc = __fmul_rn(mx, 1.0f / 127.0f);

    int sum = 0;
    const size_t qpitch = ceil_div(M, 4) * 4;  // bytes per row of the reference container
    uint8_t* xr = reinterpret_cast<uint8_t*>(xq_ref);
    for (size_t f = (size_t)lane; f < Kp; f += kWave)
    {
        int q = 0;
        if (f < K) q = quantize_one(norm_val(X[f * M + m], ri, gamma, f, norm), sc);
        sum += q;
        xi[m * Kp + f] = (int8_t)q;
        if (xr && f < K) xr[f * qpitch + m] = (uint8_t)(q & 0xFF);
    }
    sum = wave_sum_i(sum);
    if (lane == 0)
    {
        s[m] = sc;
        rowsum[m] = sum;
    }
}

// ---------------------------------------------------------------------------------------
// Large M: 64 tokens per block (lane = token, coalesced rows of the (K, M) layout),
// 8 waves; wave w owns features f = 64*b + 8*w + j (j = 0..7), i.e. parts p = 8w + j.
constexpr int kTW = 8;  // waves per block

__global__ __launch_bounds__(kTW * kWave) void k_token_lanes(
    const float* __restrict__ X, const float* __restrict__ gamma, bool norm, float eps, float inv_f,
    size_t K, size_t M, size_t Kp, int mode, int8_t* __restrict__ xi, float* __restrict__ s,
    int32_t* __restrict__ rowsum, uint32_t* __restrict__ xq_ref, float* __restrict__ fout)
{
    __shared__ float part[64][kWave];  // [p][token]
    __shared__ float pmax[kTW][kWave];
    __shared__ int psum[kTW][kWave];

    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const size_t m = (size_t)blockIdx.x * kWave + lane;
    const bool active = m < M;
    const size_t nb = Kp / 64;

    float ri = 1.0f;
    if (norm)
    {
        float acc[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
        if (active)
            for (size_t b = 0; b < nb; ++b)
            {
#pragma unroll
                for (int j = 0; j < 8; ++j)
                {
                    const size_t f = 64 * b + 8 * w + j;
                    if (f < K)
                    {
                        const float x = X[f * M + m];
                        acc[j] = __fadd_rn(acc[j], __fmul_rn(x, x));
                    }
                }
            }
#pragma unroll
        for (int j = 0; j < 8; ++j) part[8 * w + j][lane] = acc[j];
        __syncthreads();
        // butterfly tree on the lower halves: v[p] = v[p] + v[p + off] for p < off
        float v[64];
#pragma unroll
        for (int p = 0; p < 64; ++p) v[p] = part[p][lane];
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1)
#pragma unroll
            for (int p = 0; p < off; ++p) v[p] = __fadd_rn(v[p], v[p + off]);
        ri = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(__fmul_rn(v[0], inv_f), eps)));
    }

    if (mode == 1)
    {
        if (active)
            for (size_t b = 0; b < nb; ++b)
#pragma unroll
                for (int j = 0; j < 8; ++j)
                {
                    const size_t f = 64 * b + 8 * w + j;
                    if (f < K) fout[f * M + m] = norm_val(X[f * M + m], ri, gamma, f, norm);
                }
        return;
    }

    float mx = 0.0f;
    if (active)
        for (size_t b = 0; b < nb; ++b)
#pragma unroll
            for (int j = 0; j < 8; ++j)
            {
                const size_t f = 64 * b + 8 * w + j;
                if (f < K)
                {
                    const float a = fabsf(norm_val(X[f * M + m], ri, gamma, f, norm));
                    mx = a > mx ? a : mx;
                }
            }
    pmax[w][lane] = mx;
    __syncthreads();
    float tmx = pmax[0][lane];
#pragma unroll
    for (int i = 1; i < kTW; ++i) tmx = pmax[i][lane] > tmx ? pmax[i][lane] : tmx;
    const float sc = __fmul_rn(tmx, 1.0f / 127.0f);

    int sum = 0;
    const size_t qpitch = ceil_div(M, 4) * 4;
    uint8_t* xr = reinterpret_cast<uint8_t*>(xq_ref);
    if (active)
        for (size_t b = 0; b < nb; ++b)
        {
            uint32_t lo = 0, hi = 0;
#pragma unroll
            for (int j = 0; j < 8; ++j)
            {
                const size_t f = 64 * b + 8 * w + j;
                int q = 0;
                if (f < K) q = quantize_one(norm_val(X[f * M + m], ri, gamma, f, norm), sc);
                sum += q;
                if (j < 4) lo |= (uint32_t)(q & 0xFF) << (8 * j);
                else hi |= (uint32_t)(q & 0xFF) << (8 * (j - 4));
                if (xr && f < K) xr[f * qpitch + m] = (uint8_t)(q & 0xFF);
            }
            *reinterpret_cast<uint2*>(xi + m * Kp + 64 * b + 8 * w) = make_uint2(lo, hi);
        }
    psum[w][lane] = sum;
    __syncthreads();
    if (w == 0 && active)
    {
        int t = 0;
#pragma unroll
        for (int i = 0; i < kTW; ++i) t += psum[i][lane];
        s[m] = sc;
        rowsum[m] = t;
    }
}

// Reference container (K, ceil(M/4)) -> token-major xi + rowsum. One block per token.
__global__ __launch_bounds__(kBlock) void k_from_container(const uint32_t* __restrict__ xq, size_t K,
                                                           size_t M, size_t Kp,
                                                           int8_t* __restrict__ xi,
                                                           int32_t* __restrict__ rowsum)
{
    __shared__ int red[kBlock / kWave];
    const size_t m = blockIdx.x;
    const size_t wpr = ceil_div(M, 4);
    const uint8_t* src = reinterpret_cast<const uint8_t*>(xq);
    int sum = 0;
    for (size_t k = threadIdx.x; k < Kp; k += kBlock)
    {
        int q = 0;
        if (k < K) q = (int)(int8_t)src[k * wpr * 4 + m];
        sum += q;
        xi[m * Kp + k] = (int8_t)q;
    }
    sum = wave_sum_i(sum);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = sum;
    __syncthreads();
    if (threadIdx.x == 0)
    {
        int t = 0;
        for (int i = 0; i < kBlock / kWave; ++i) t += red[i];
        rowsum[m] = t;
    }
}

// token-major xi -> reference container; one thread per output word.
__global__ __launch_bounds__(kBlock) void k_to_container(const int8_t* __restrict__ xi, size_t K,
                                                         size_t M, size_t Kp,
                                                         uint32_t* __restrict__ xq)
{
    const size_t wpr = ceil_div(M, 4);
    const size_t total = K * wpr;
    for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (size_t)gridDim.x * blockDim.x)
    {
        const size_t k = idx / wpr, wi = idx - k * wpr;
        uint32_t word = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b)
        {
            const size_t m = wi * 4 + b;
            if (m < M) word |= (uint32_t)(uint8_t)xi[m * Kp + k] << (8 * b);
        }
        xq[idx] = word;
    }
}

constexpr size_t kSmallM = 32;

}  // namespace

static hipError_t launch_token_kernel(hipStream_t st, const float* X, const float* gamma, bool norm,
                                      float eps, size_t K, size_t M, int mode, int8_t* xi, float* s,
                                      int32_t* rowsum, uint32_t* xq_ref, float* fout)
{
    if (M == 0) return hipSuccess;
    const float inv_f = 1.0f / (float)K;
    const size_t Kp = round_up(K, kTileK);
    if (M <= kSmallM)
    {
        const unsigned grid = (unsigned)ceil_div(M, kBlock / kWave);
        hipLaunchKernelGGL(k_token_wave, dim3(grid), dim3(kBlock), 0, st, X, gamma, norm, eps, inv_f,
                           K, M, Kp, mode, xi, s, rowsum, xq_ref, fout);
    }
    else
    {
        const unsigned grid = (unsigned)ceil_div(M, kWave);
        hipLaunchKernelGGL(k_token_lanes, dim3(grid), dim3(kTW * kWave), 0, st, X, gamma, norm, eps,
                           inv_f, K, M, Kp, mode, xi, s, rowsum, xq_ref, fout);
    }
    return hipGetLastError();
}

hipError_t launch_rmsnorm(hipStream_t st, const float* X, const float* gamma, float eps, size_t F,
                          size_t M, float* out)
{
    return launch_token_kernel(st, X, gamma, true, eps, F, M, 1, nullptr, nullptr, nullptr, nullptr,
                               out);
}

hipError_t launch_act_quant(hipStream_t st, const float* X, const float* gamma, bool norm, float eps,
                            size_t K, size_t M, int8_t* xi, float* s, int32_t* rowsum,
                            uint32_t* xq_ref)
{
    if (xq_ref && M % 4 != 0)
    {
        // tail bytes of the last word of each row must read 0: clear the container first
        const hipError_t e = launch_fill_u32(st, xq_ref, 0u, K * ceil_div(M, 4));
        if (e != hipSuccess) return e;
    }
    return launch_token_kernel(st, X, gamma, norm, eps, K, M, 0, xi, s, rowsum, xq_ref, nullptr);
}

hipError_t launch_act_from_container(hipStream_t st, const uint32_t* xq, size_t K, size_t M,
                                     int8_t* xi, int32_t* rowsum)
{
    if (M == 0) return hipSuccess;
    const size_t Kp = round_up(K, kTileK);
    hipLaunchKernelGGL(k_from_container, dim3((unsigned)M), dim3(kBlock), 0, st, xq, K, M, Kp, xi,
                       rowsum);
    return hipGetLastError();
}

hipError_t launch_act_to_container(hipStream_t st, const int8_t* xi, size_t K, size_t M, uint32_t* xq)
{
    const size_t wpr = ceil_div(M, 4);
    if (K == 0 || wpr == 0) return hipSuccess;
    const size_t Kp = round_up(K, kTileK);
    size_t g = ceil_div(K * wpr, (size_t)kBlock);
    if (g > (1u << 20)) g = 1u << 20;
    hipLaunchKernelGGL(k_to_container, dim3((unsigned)g), dim3(kBlock), 0, st, xi, K, M, Kp, xq);
    return hipGetLastError();
}

}  // namespace nnhip
