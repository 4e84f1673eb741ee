// token_quant.hpp — the per-token [RMSNorm ->] absmax -> int8 quantizer passes of the
// one-token-per-block kernels, shared by k_act.hip (activations from a (K, M) matrix), k_gemv.hip
// (the split-k GEMV epilogue and residual add first) and k_decode.hip (the attention merge
// first). Every kernel evaluates the per-token sum of squares in one fixed order, the same as the
// oracle: 512 strided parts (feature f in part f % 512), each summed in ascending f, then the xor
// butterfly over 256, 128, ..., 1. So the normalized values, the scale and the int8 codes are
// bit-identical to the unfused reference sequence whichever kernel runs.
#pragma once

#include "common.hpp"

#include <cmath>

namespace nnhip
{
namespace
{

constexpr int kParts = 512;  // sum-of-squares parts
constexpr int kOneThreads = kOneThreadsHost;  // one-token kernels: thread t owns part t

__device__ __forceinline__ int quantize_one(float x, float s)
{
    if (s == 0.0f || isnan(x)) return 0;
    float v = __fdiv_rn(x, s);
    if (isnan(v)) return 0;
    v = fminf(fmaxf(v, -127.0f), 127.0f);
    return (int)roundf(v);
}

// Per-token reciprocal for the division-free codes: fl(1/s), 0 when s == 0 (every code is then
// 0, as quantize_one gives), +inf when 1/s overflows (every product is then flagged).
__device__ __forceinline__ float quant_rcp(float s)
{
    return s == 0.0f ? 0.0f : __fdiv_rn(1.0f, s);
}

// quantize_one(x, s) without a division in the common case, for callers whose scale comes from
// the same elements: with r = fl(1/s) and y = fl(x * r), when y is 2^-15 or more from every
// half-integer, rint(y) is quantize_one's code (no tie and no integer boundary between y and
// fl(x/s)), and no clamp is needed. Range: with s = fl(amax * fl(1/127)) over the elements and r
// finite, every |x| <= amax gives |fl(x * r)| <= 127 * (1 + 2^-20) < 127.5 (four roundings, one of
// them of s, which is at least 2^-128 whenever 1/s is finite and so keeps 22 significant bits even
// when subnormal), so rint(y) is already in [-127, 127]. Margin: |y - x/s| <= |x/s| * (2^-23 +
// 2^-48) < 2^-16 and |fl(x/s) - x/s| <= 2^-17 below 128, so |y - fl(x/s)| < 3 * 2^-17. NaN, inf
// and near-tie products set `amb`, and the caller takes quantize_exact (the same code bit for bit).
__device__ __forceinline__ int quantize_code(float x, float r, bool& amb)
{
    const float y = __fmul_rn(x, r);
    const float t = __builtin_rintf(y);
    amb |= !(fabsf(y - t) < 0.5f - 0x1p-15f);
    return (int)t;
}

// quantize_one(x, s) without a division and without branches, for s >= 2^-100 and r = fl(1/s)
// (the correctly rounded reciprocal). q0 = fl(x * r) is within one ulp of x/s, the residual
// x - q0 * s is exact under one FMA, and fl(q0 + residual * r) is then the correctly rounded
// quotient fl(x/s) (Markstein's theorem; the bound on s keeps the residual out of the subnormal
// range wherever the code can be nonzero). Clamped to 127 in magnitude and rounded half away
// from zero as roundf; a NaN quotient (NaN x, or 0 * inf when s is 0) gives 0.
__device__ __forceinline__ int quantize_exact(float x, float s, float r)
{
    const float q0 = __fmul_rn(x, r);
    const float e = __builtin_fmaf(-q0, s, x);
    const float v = __builtin_fmaf(e, r, q0);
    const float a = fminf(fabsf(v), 127.0f);
    float t = __builtin_rintf(a);
    t = (__fsub_rn(a, t) == 0.5f) ? __fadd_rn(t, 1.0f) : t;
    const int c = (int)t;
    return v != v ? 0 : (__builtin_signbit(v) ? -c : c);
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

__device__ __forceinline__ float rms_inv_of(float sum_sq, float inv_f, float eps)
{
    return __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(__fmul_rn(sum_sq, inv_f), eps)));
}

__device__ __forceinline__ int wave_sum_i(int v)
{
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// In-register butterfly levels: v[k] holds part p + stride*k (k < N); after the levels for
// offsets stride*N/2 .. stride, v[0] holds part p of the tree at level `stride`.
template <int N>
__device__ __forceinline__ float tree_levels(float (&v)[N])
{
#pragma unroll
    for (int d = N / 2; d >= 1; d >>= 1)
#pragma unroll
        for (int k = 0; k < d; ++k) v[k] = __fadd_rn(v[k], v[k + d]);
    return v[0];
}


// Lane exchanges of a butterfly with descending offsets: the value of lane l ^ OFF as seen after
// the levels above OFF (by then a lane's value depends only on its lane bits below 2*OFF, so any
// partner with those bits equal to (l mod 2*OFF) ^ OFF carries the same value). OFF = 1, 2:
// quad_perm; OFF = 4, 8: row_ror; OFF = 16, 32: v_permlane16_swap / v_permlane32_swap of two
// copies (inline asm; the two-result builtin returned its first register for both with this
// compiler), which leave the lower row's value in the first register and the upper row's in the
// second in every lane of a pair. bfly() combines own and partner with op, which is commutative
// here (fl(a + b), max, integer +), so both lanes of a pair get the same bits.
template <int CTRL>
__device__ __forceinline__ int tq_dpp(int v)
{
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, false);
}
template <int OFF, class T, class Op>
__device__ __forceinline__ T bfly(T v, Op op)
{
    if constexpr (OFF >= 16)
    {
        int a = __builtin_bit_cast(int, v), b = a;
        if constexpr (OFF == 32)
            asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
        else
            asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
        return op(__builtin_bit_cast(T, a), __builtin_bit_cast(T, b));
    }
    else
    {
        constexpr int ctrl = OFF == 1 ? 0xB1 : OFF == 2 ? 0x4E : OFF == 4 ? 0x124 : 0x128;
        return op(v, __builtin_bit_cast(T, tq_dpp<ctrl>(__builtin_bit_cast(int, v))));
    }
}
// over all 64 lanes, offsets 32, 16, ..., 1 (every lane gets the result)
template <class T, class Op>
__device__ __forceinline__ T wave_bfly(T v, Op op)
{
    v = bfly<32>(v, op);
    v = bfly<16>(v, op);
    v = bfly<8>(v, op);
    v = bfly<4>(v, op);
    v = bfly<2>(v, op);
    return bfly<1>(v, op);
}
struct TqAdd
{
    __device__ float operator()(float a, float b) const { return __fadd_rn(a, b); }
};
struct TqMax
{
    __device__ float operator()(float a, float b) const { return fmaxf(a, b); }
};
struct TqIAdd
{
    __device__ int operator()(int a, int b) const { return a + b; }
};

struct TokArgs
{
    const float* X;
    bool norm;
    float eps, inv_f;
    int K, M, Kp, mode;
    int8_t* xi;
    float* s;
    int32_t* rowsum;
    uint32_t* xq_ref;
    float* fout;
    int xtm;  // one-token kernel: X is token-major (M, K) instead of (K, M)
    Prefetch pf;  // one-token kernels: blocks M .. M + pf.blocks - 1 read these ranges
    // k_token_one gathering its rows: token m is row gids[m] of X (gV rows; NaN for an id outside
    // [0, gV)), also stored as row m of gout (M, K)
    const int32_t* gids;
    int gV;
    float* gout;
};

// Block b of a one-token kernel's prefetch blocks: thread t reads the 16-byte units
// (k * blocks + b) * 512 + t (k < kPfUnitsPerThread) of the concatenated ranges, consecutive
// threads consecutive units. The empty asm keeps the loads (their values are not used).
__device__ __forceinline__ void prefetch_block(const Prefetch& pf, int b)
{
    const uint32_t e0 = pf.n16[0], e1 = e0 + pf.n16[1], e2 = e1 + pf.n16[2], e3 = e2 + pf.n16[3];
    uint32_t acc = 0;
#pragma unroll
    for (int k = 0; k < kPfUnitsPerThread; ++k)
    {
        const uint32_t u = (uint32_t)(k * pf.blocks + b) * kOneThreads + threadIdx.x;
        if (u >= e3) break;
        const uint4* q = u < e0   ? static_cast<const uint4*>(pf.p[0]) + u
                         : u < e1 ? static_cast<const uint4*>(pf.p[1]) + (u - e0)
                         : u < e2 ? static_cast<const uint4*>(pf.p[2]) + (u - e1)
                                  : static_cast<const uint4*>(pf.p[3]) + (u - e2);
        const uint4 v = *q;
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    asm volatile("" ::"v"(acc));
}

// LDS of the one-token kernels
struct OneShared
{
    float red[kParts];
    float wred[kOneThreads / kWave];
    int wsum[kOneThreads / kWave];
    float tok_ri;
};

// The passes of one token (m = blockIdx.x) once thread t holds x[r] = its value at feature
// f = t + 512 r (0 past K): [RMSNorm with gamma: rms_inv from the 512 parts summed in ascending f
// and the tree over them in wave 0, then (x * rms_inv) * gamma], then either the normalized values
// to a.fout (mode 1) or the absmax scale, the codes (fast / exact quantizer pair) into the
// token-major xi, the container a.xq_ref if given, s and the code row sum.
template <int R>
__device__ __forceinline__ void one_token_finish(float (&x)[R], const TokArgs& a, const float* __restrict__ gamma,
                                                 OneShared& sh)
{
    constexpr int NW = kOneThreads / kWave;
    static_assert(kOneThreads == kParts, "one part per thread");
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int m = blockIdx.x;
    if (a.norm)
    {
        float gm[R];
#pragma unroll
        for (int r = 0; r < R; ++r)
        {
            const int f = t + kParts * r;
            gm[r] = f < a.K ? gamma[f] : 0.0f;
        }
        float acc = 0.0f;
#pragma unroll
        for (int r = 0; r < R; ++r) acc = __fadd_rn(acc, __fmul_rn(x[r], x[r]));
        sh.red[t] = acc;
        __syncthreads();
        if (w == 0)
        {
            float v[kParts / kWave];
#pragma unroll
            for (int k = 0; k < kParts / kWave; ++k) v[k] = sh.red[lane + kWave * k];
            const float sum = wave_bfly(tree_levels(v), TqAdd{});
            if (lane == 0) sh.tok_ri = rms_inv_of(sum, a.inv_f, a.eps);
        }
        __syncthreads();
        const float ri = sh.tok_ri;
#pragma unroll
        for (int r = 0; r < R; ++r) x[r] = __fmul_rn(__fmul_rn(x[r], ri), gm[r]);
    }
    if (a.mode == 1)
    {
#pragma unroll
        for (int r = 0; r < R; ++r)
        {
            const int f = t + kParts * r;
            if (f < a.K) a.fout[(size_t)f * a.M + m] = x[r];
        }
        return;
    }
    float mx = 0.0f;
#pragma unroll
    for (int r = 0; r < R; ++r) mx = fmaxf(mx, fabsf(x[r]));
    mx = wave_bfly(mx, TqMax{});
    if (lane == 0) sh.wred[w] = mx;
    __syncthreads();
    float tm = sh.wred[0];
#pragma unroll
    for (int v = 1; v < NW; ++v) tm = fmaxf(tm, sh.wred[v]);
    const float sc = __fmul_rn(tm, 1.0f / 127.0f);
    const float rc = quant_rcp(sc);
    int q[R];
    bool amb = isinf(rc);
#pragma unroll
    for (int r = 0; r < R; ++r) q[r] = quantize_code(x[r], rc, amb);
    if (amb)
    {
        // a flagged element: the thread's codes again through the exact division-free path, on
        // x * xs / (s * xs) with the power-of-two prescale that keeps s * xs >= 2^-100
        const float xs = sc < 0x1p-100f ? 0x1p100f : 1.0f;
        const float se = __fmul_rn(sc, xs), re = quant_rcp(se);
#pragma unroll
        for (int r = 0; r < R; ++r) q[r] = quantize_exact(__fmul_rn(x[r], xs), se, re);
    }
    int tsum = 0;
    const int wpr = (a.M + 3) / 4;
#pragma unroll
    for (int r = 0; r < R; ++r)
    {
        const int f = t + kParts * r;
        tsum += q[r];  // rows past K hold code 0
        if (f < a.Kp) a.xi[(size_t)m * a.Kp + f] = (int8_t)q[r];
        if (a.xq_ref && f < a.K)
            reinterpret_cast<int8_t*>(a.xq_ref)[((size_t)f * wpr + m / 4) * 4 + m % 4] = (int8_t)q[r];
    }
    tsum = wave_bfly(tsum, TqIAdd{});
    if (lane == 0) sh.wsum[w] = tsum;
    __syncthreads();
    if (t == 0)
    {
        int sum = 0;
#pragma unroll
        for (int v = 0; v < NW; ++v) sum += sh.wsum[v];
        a.s[m] = sc;
        a.rowsum[m] = sum;
    }
}

}  // namespace
}  // namespace nnhip
