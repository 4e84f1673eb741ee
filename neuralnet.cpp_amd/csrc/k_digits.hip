// k_digits.hip — ternary x float products on the MFMA path: the reference's default BitLinear
// branch, matmul_q (f32 / f16 activations, include/neuralnet.cpp/compute_layer_bitlinear.hpp:464;
// src/ternary_gemm_test.cpp:253-289), on the repacked T16K256 weights.
//
// Each token m of B (K, M) becomes a 31-bit fixed point: with E_m the exponent of max_k |x|
// (max < 2^E_m), X = rint(x * 2^(30 - E_m)), |X| <= 2^30, written as four balanced base-256
// digits X = d0 + 256 d1 + 65536 d2 + 2^24 d3, every d in [-128, 127]. The digits are four int8
// "tokens" 4m .. 4m+3 for the ternary x int8 GEMV / GEMM, whose int32 sums are exact; run with
// unit scales its outputs are the exact integers A_p = sum_k trit * d_p (|A_p| <= 128 K < 2^24
// while K < 131072). The combine kernel forms T = sum_p A_p 256^p in int64 (exact) and
// Y = tau * (fl(T) * 2^(E_m - 30)): the only roundings are x to the fixed-point grid
// (<= 2^(E_m - 31) per element), the conversion of T and the multiply by tau — far inside the
// reference tolerance of f32 accumulation (1e-4 x max(1, max|Y|), src/ternary_gemm_test.cpp:503-516).
// A token holding NaN or +-inf takes an exact IEEE path in the combine kernel instead (per row:
// NaN if any NaN term, 0 x inf term or opposite infinities, else the infinity's sign), which is
// what the reference's per-term products give.
#include "common.hpp"

#include <cmath>

namespace nnhip
{
namespace
{

constexpr int kDigBlock = 256;
constexpr int32_t kSpecialToken = 0x7FFFFFFF;  // ex[m] of a token with a NaN or an infinity

__device__ __forceinline__ float load_b(const void* B, size_t idx, bool f16)
{
    return f16 ? (float)reinterpret_cast<const _Float16*>(B)[idx] : reinterpret_cast<const float*>(B)[idx];
}

// activation k of token m, times kscale[k] when given (one rounding: the transposed product's
// fl(tau_k * b), equal to the reference's fl(tau_k * trit) * b term by term)
__device__ __forceinline__ float load_bk(const void* B, const float* kscale, int k, int M, int m, bool f16)
{
    const float x = load_b(B, (size_t)k * M + m, f16);
    return kscale ? __fmul_rn(kscale[k], x) : x;
}

// One block per token: absmax (and non-finite detection), then the four digit rows. Each thread
// takes columns k = tid + kDigThreads * (8 i + u), eight independent loads in flight per step.
constexpr int kDigThreads = 1024;
constexpr int kDigUnroll = 8;

__global__ __launch_bounds__(kDigThreads) void k_digits(const void* __restrict__ B, bool f16,
                                                        const float* __restrict__ kscale, int K, int M, int Kp,
                                                        int8_t* __restrict__ xi, int32_t* __restrict__ rowsum,
                                                        int32_t* __restrict__ ex)
{
    constexpr int NW = kDigThreads / kWave;
    __shared__ float smax[NW];
    __shared__ int sbad[NW];
    __shared__ int ssum[4][NW];
    const int m = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    constexpr int STEP = kDigThreads * kDigUnroll;
    float mx = 0.0f;
    int bad = 0;
    for (int k0 = tid; k0 < K; k0 += STEP)
    {
        float v[kDigUnroll];
#pragma unroll
        for (int u = 0; u < kDigUnroll; ++u)
        {
            const int k = k0 + u * kDigThreads;
            v[u] = k < K ? load_bk(B, kscale, k, M, m, f16) : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < kDigUnroll; ++u)
        {
            const float a = fabsf(v[u]);
            bad |= !(a <= 3.4028234663852886e38f);  // NaN or inf
            mx = fmaxf(mx, a);
        }
    }
    for (int off = 32; off >= 1; off >>= 1)
    {
        mx = fmaxf(mx, __shfl_xor(mx, off, kWave));
        bad |= __shfl_xor(bad, off, kWave);
    }
    if (lane == 0)
    {
        smax[w] = mx;
        sbad[w] = bad;
    }
    __syncthreads();
    for (int i = 0; i < NW; ++i)
    {
        mx = fmaxf(mx, smax[i]);
        bad |= sbad[i];
    }
    int E = 0;
    (void)frexpf(mx, &E);  // mx < 2^E (E = 0 for mx = 0: every digit is 0)
    const int shift = 30 - E;
    int s[4] = {0, 0, 0, 0};
    int8_t* row = xi + (size_t)4 * m * Kp;
    for (int k0 = tid; k0 < Kp; k0 += STEP)
    {
        float v[kDigUnroll];
#pragma unroll
        for (int u = 0; u < kDigUnroll; ++u)
        {
            const int k = k0 + u * kDigThreads;
            v[u] = (k < K && !bad) ? load_bk(B, kscale, k, M, m, f16) : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < kDigUnroll; ++u)
        {
            const int k = k0 + u * kDigThreads;
            if (k >= Kp) continue;
            int X = (int)__builtin_rintf(ldexpf(v[u], shift));
            int d[4];
#pragma unroll
            for (int p = 0; p < 3; ++p)
            {
                d[p] = ((X + 128) & 255) - 128;
                X = (X - d[p]) >> 8;  // exact: X - d is a multiple of 256
            }
            d[3] = X;
#pragma unroll
            for (int p = 0; p < 4; ++p)
            {
                row[(size_t)p * Kp + k] = (int8_t)d[p];
                s[p] += d[p];
            }
        }
    }
#pragma unroll
    for (int p = 0; p < 4; ++p)
    {
        for (int off = 32; off >= 1; off >>= 1) s[p] += __shfl_xor(s[p], off, kWave);
        if (lane == 0) ssum[p][w] = s[p];
    }
    __syncthreads();
    if (tid < 4)
    {
        int t = 0;
        for (int i = 0; i < NW; ++i) t += ssum[tid][i];
        rowsum[4 * m + tid] = t;
    }
    if (tid == 0) ex[m] = bad ? kSpecialToken : E;
}

// Code (trit + 2) of row n, column k in the T16K256 layout.
__device__ __forceinline__ int code_at(const uint32_t* rp, int KT, int n, int k)
{
    const int rt = n >> 4, r = n & 15, kt = k >> 8, kk = k & 255;
    const int j = kk >> 6, g = (kk >> 4) & 3, q = (kk >> 2) & 3, b = kk & 3;
    const uint32_t word = rp[((size_t)rt * KT + kt) * 256 + 4 * (16 * g + r) + q];
    return (int)((word >> (8 * b + 2 * j)) & 3u);
}

// Y[n, m] from the digit products Yp (N, 4M): tau[n] * (fl(T) * 2^(E_m - 30)); a special token
// runs the IEEE evaluation of its non-finite terms over K.
__global__ __launch_bounds__(kDigBlock) void k_digit_combine(const float* __restrict__ Yp, const float* __restrict__ tau,
                                                             const int32_t* __restrict__ ex,
                                                             const uint32_t* __restrict__ rp, int KT,
                                                             const void* __restrict__ B, bool b16,
                                                             const float* __restrict__ kscale, int N, int K, int M,
                                                             void* __restrict__ Y, bool y16)
{
    const size_t idx = (size_t)blockIdx.x * kDigBlock + threadIdx.x;
    if (idx >= (size_t)N * M) return;
    const int n = (int)(idx / M), m = (int)(idx % M);
    const int E = ex[m];
    const float tn = tau ? tau[n] : 1.0f;
    float y;
    if (E != kSpecialToken)
    {
        const float4 d = *reinterpret_cast<const float4*>(Yp + ((size_t)n * M + m) * 4);
        const long long T = (long long)d.x + ((long long)d.y << 8) + ((long long)d.z << 16) + ((long long)d.w << 24);
        y = tn * ldexpf((float)T, E - 30);
    }
    else
    {
        // the finite terms cannot change a NaN or an infinite total: only the non-finite ones matter
        bool nan = false, pos = false, neg = false;
        for (int k = 0; k < K; ++k)
        {
            const float x = load_bk(B, kscale, k, M, m, b16);
            if (fabsf(x) <= 3.4028234663852886e38f) continue;
            const float tw = tn * (float)(code_at(rp, KT, n, k) - 2);
            if (x != x || tw != tw || tw == 0.0f)
                nan = true;
            else if ((tw > 0.0f) == (x > 0.0f))
                pos = true;
            else
                neg = true;
        }
        y = (nan || (pos && neg)) ? __builtin_nanf("") : (pos ? __builtin_inff() : -__builtin_inff());
    }
    if (y16)
        reinterpret_cast<_Float16*>(Y)[idx] = (_Float16)y;
    else
        reinterpret_cast<float*>(Y)[idx] = y;
}

}  // namespace

hipError_t launch_digits(hipStream_t st, const void* B, bool b16, const float* kscale, size_t K, size_t M, int8_t* xi,
                         int32_t* rowsum, int32_t* ex)
{
    const size_t Kp = round_up(K, kTileK);
    k_digits<<<dim3((unsigned)M), kDigThreads, 0, st>>>(B, b16, kscale, (int)K, (int)M, (int)Kp, xi, rowsum, ex);
    return hipGetLastError();
}

hipError_t launch_digit_combine(hipStream_t st, const float* Yp, const float* tau, const int32_t* ex,
                                const uint32_t* rp, const void* B, bool b16, const float* kscale, size_t N, size_t K,
                                size_t M, void* Y, bool y16)
{
    const size_t n = N * M;
    k_digit_combine<<<dim3((unsigned)ceil_div(n, kDigBlock)), kDigBlock, 0, st>>>(
        Yp, tau, ex, rp, (int)ceil_div(K, kTileK), B, b16, kscale, (int)N, (int)K, (int)M, Y, y16);
    return hipGetLastError();
}

}  // namespace nnhip
