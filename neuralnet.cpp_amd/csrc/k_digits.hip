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
#include "gemv_tile.hpp"

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

// The same digits for a few long tokens (the split-k path, M <= 4): block (c, m) takes columns
// [c * kChunk, (c + 1) * kChunk) of token m. Each block first reduces the absmax and the
// non-finite flag over the whole token (every chunk of a token sees the same E, so the digits are
// k_digits' bit for bit), then writes its chunk's digit rows and its partial digit sums
// rsp[(m * P + c) * 4 + p] (the combine adds the P partials: integers, exact in any order).
constexpr int kChunk = 4096;
constexpr int kChunkThreads = 256;

__global__ __launch_bounds__(kChunkThreads) void k_digits_chunks(const void* __restrict__ B, bool f16,
                                                                 const float* __restrict__ kscale, int K, int M, int Kp,
                                                                 int8_t* __restrict__ xi, int32_t* __restrict__ rsp,
                                                                 int32_t* __restrict__ ex)
{
    constexpr int NW = kChunkThreads / kWave;
    __shared__ float smax[NW];
    __shared__ int sbad[NW];
    __shared__ int ssum[4][NW];
    const int c = blockIdx.x, m = blockIdx.y, P = gridDim.x;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    constexpr int STEP = kChunkThreads * kDigUnroll;
    float mx = 0.0f;
    int bad = 0;
    for (int k0 = tid; k0 < K; k0 += STEP)
    {
        float v[kDigUnroll];
#pragma unroll
        for (int u = 0; u < kDigUnroll; ++u)
        {
            const int k = k0 + u * kChunkThreads;
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
    const int kend = min(Kp, (c + 1) * kChunk);
    for (int k = c * kChunk + tid; k < kend; k += kChunkThreads)
    {
        const float v = (k < K && !bad) ? load_bk(B, kscale, k, M, m, f16) : 0.0f;
        int X = (int)__builtin_rintf(ldexpf(v, shift));
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
        rsp[((size_t)m * P + c) * 4 + tid] = t;
    }
    if (c == 0 && tid == 0) ex[m] = bad ? kSpecialToken : E;
}

// Code (trit + 2) of row n, column k in the T16K256 layout.
__device__ __forceinline__ int code_at(const uint32_t* rp, int KT, int n, int k)
{
    const int rt = n >> 4, r = n & 15, kt = k >> 8, kk = k & 255;
    const int j = kk >> 6, g = (kk >> 4) & 3, q = (kk >> 2) & 3, b = kk & 3;
    const uint32_t word = rp[((size_t)rt * KT + kt) * 256 + 4 * (16 * g + r) + q];
    return (int)((word >> (8 * b + 2 * j)) & 3u);
}

// Y[n, m] of a token holding a NaN or an infinity: the finite terms cannot change a NaN or an
// infinite total, so only the non-finite ones are evaluated (IEEE products tau_n * trit * x):
// NaN if any is NaN (0 x inf included) or infinities of both signs meet, else that infinity.
__device__ float special_dot(const void* B, bool b16, const float* kscale, const uint32_t* rp, int KT, int K, int M,
                             int n, int m, float tn)
{
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
    return (nan || (pos && neg)) ? __builtin_nanf("") : (pos ? __builtin_inff() : -__builtin_inff());
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
        y = special_dot(B, b16, kscale, rp, KT, K, M, n, m, tn);
    if (y16)
        reinterpret_cast<_Float16*>(Y)[idx] = (_Float16)y;
    else
        reinterpret_cast<float*>(Y)[idx] = y;
}

// k_digit_combine on the split-k path: the digit products come as S int32 slice sums of
// sum(code * d) (part[ks][4m + p][n], k_gemv_part) and P partial digit sums per token; their
// exact total A_p = sum_ks part - 2 sum_c rsp is the integer the unit-scale GEMV would have given,
// so Y is k_digit_combine's bit for bit.
__global__ __launch_bounds__(kDigBlock) void k_digit_combine_parts(const int32_t* __restrict__ part, int S,
                                                                   const int32_t* __restrict__ rsp, int P,
                                                                   const float* __restrict__ tau,
                                                                   const int32_t* __restrict__ ex,
                                                                   const uint32_t* __restrict__ rp, int KT,
                                                                   const void* __restrict__ B, bool b16,
                                                                   const float* __restrict__ kscale, int N, int K, int M,
                                                                   void* __restrict__ Y, bool y16)
{
    const size_t idx = (size_t)blockIdx.x * kDigBlock + threadIdx.x;
    if (idx >= (size_t)N * M) return;
    const int n = (int)(idx % N), m = (int)(idx / N);  // consecutive threads: consecutive n
    const int E = ex[m];
    const float tn = tau ? tau[n] : 1.0f;
    float y;
    if (E != kSpecialToken)
    {
        long long T = 0;
#pragma unroll
        for (int p = 3; p >= 0; --p)
        {
            int a = 0;
            for (int ks = 0; ks < S; ++ks) a += part[((size_t)ks * 4 * M + 4 * m + p) * N + n];
            int r = 0;
            for (int c = 0; c < P; ++c) r += rsp[((size_t)m * P + c) * 4 + p];
            T = (T << 8) + (long long)(a - 2 * r);
        }
        y = tn * ldexpf((float)T, E - 30);
    }
    else
        y = special_dot(B, b16, kscale, rp, KT, K, M, n, m, tn);
    const size_t o = (size_t)n * M + m;
    if (y16)
        reinterpret_cast<_Float16*>(Y)[o] = (_Float16)y;
    else
        reinterpret_cast<float*>(Y)[o] = y;
}

// ---------------------------------------------------------------------------------------
// One-launch float-activation GEMV for decode sizes: M <= 4 f32 tokens, so the 4M digit rows
// fit one 16-column MFMA operand. Each block of 4 waves (one 16-row tile per wave):
//   1. issues the loads of its share of the activations (groups of 4 consecutive k, all M
//      tokens: 4M contiguous floats, and kscale), then every weight stage of its tile. The
//      activation loads are the older ones, so waiting for them leaves the weight stream in
//      flight while step 2 runs;
//   2. makes the digits of the M tokens as k_digits does (per-token absmax and non-finite flag
//      over the block, E, X = rint(x 2^(30 - E)), four balanced base-256 digits) into LDS: digit
//      row t = 4m + p in the deep GEMV's XOR-swizzled 16-byte units, plus the digit row sums;
//   3. runs the MFMAs of its tile against the digit rows;
//   4. lane (g, t = 4m + p) gathers from its lane quad the four digit sums A_q of row 4g + p
//      (DPP broadcasts), forms T = sum_q A_q 256^q in int64 and stores tau * (fl(T) 2^(E - 30)):
//      k_digit_combine's arithmetic, so the result equals the three-launch path's bit for bit.
//      A token with a NaN or an infinity takes the same IEEE evaluation (special_dot).
// Every block repeats step 2 over the whole activation (4MK bytes from L2): small next to its
// tile's weights at these sizes, and it saves two launches and the digit round trip.
constexpr int kDgBlock = 256;
constexpr uint32_t kDgOOB = 0x80000000u;

struct DigitGemvArgs
{
    const u32x4* rp;
    const float* tau;     // per row; null for the transposed product (unit)
    const float* kscale;  // per k (the transposed product's tau) or null
    const float* B;       // (K, M) f32, 16-byte aligned
    void* Y;              // (N, M) f32 or f16
    int N, K, y16;
};

__device__ __forceinline__ float4 ld_x4(__amdgpu_buffer_rsrc_t r, uint32_t off)
{
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

__device__ __forceinline__ float f4c(const float4& v, int c)
{
    return c == 0 ? v.x : c == 1 ? v.y : c == 2 ? v.z : v.w;
}

// lane q of the caller's lane quad, broadcast to the quad
template <int Q>
__device__ __forceinline__ int quad_bcast(int v)
{
    return __builtin_amdgcn_mov_dpp(v, Q * 0x55, 0xF, 0xF, false);
}

// workgroup barrier for LDS data: this wave's LDS operations done, no wait on vector memory
__device__ __forceinline__ void dg_lds_barrier()
{
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt at their maxima
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

template <int KT, int M>
__global__ __launch_bounds__(kDgBlock) void k_gemv_digits(DigitGemvArgs a)
{
    constexpr int NW = kDgBlock / kWave;
    constexpr uint32_t Kp = (uint32_t)KT * kTileK;
    constexpr int GP = (int)(Kp / 4);                   // groups of 4 k, padding included
    constexpr int G = (GP + kDgBlock - 1) / kDgBlock;   // groups per thread
    extern __shared__ __align__(16) uint8_t lds[];      // 4M digit rows of Kp bytes
    __shared__ float s_mx[NW][M];
    __shared__ int s_bad[NW][M];
    __shared__ int s_rs[NW][4 * M];

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int g = lane >> 4, t = lane & 15;
    const int rt = blockIdx.x * NW + wv;
    const bool live = rt < (a.N + 15) >> 4;
    const int groups = a.K >> 2;  // K % 4 == 0
    const bool has_ks = a.kscale != nullptr;

    // 1. activation loads (past K: zeros without traffic), then the tile's weights
    const __amdgpu_buffer_rsrc_t rb = rsrc(a.B, (uint32_t)a.K * M * 4u);
    const __amdgpu_buffer_rsrc_t rk = rsrc(has_ks ? a.kscale : a.B, has_ks ? (uint32_t)a.K * 4u : 0u);
    float4 xv[G][M], ks[G];
#pragma unroll
    for (int i = 0; i < G; ++i)
    {
        const int q = tid + kDgBlock * i;
        const uint32_t off = q < groups ? (uint32_t)q * 16u * M : kDgOOB;
#pragma unroll
        for (int c = 0; c < M; ++c) xv[i][c] = ld_x4(rb, off + 16u * c);
        ks[i] = ld_x4(rk, q < groups ? (uint32_t)q * 16u : kDgOOB);
    }
    const __amdgpu_buffer_rsrc_t rw = rsrc(a.rp + (size_t)(live ? rt : 0) * KT * 64, live ? (uint32_t)KT * 1024u : 0u);
    v4i w[KT];
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) w[kt] = ld16<kNT>(rw, (uint32_t)lane * 16u, (uint32_t)kt * 1024u);
    const int p = t & 3, mt = t >> 2;           // this lane: digit p of token mt
    const int n_out = rt * 16 + 4 * g + p;      // the output row it stores
    const __amdgpu_buffer_rsrc_t rtau = rsrc(a.tau ? a.tau : a.B, a.tau ? (uint32_t)a.N * 4u : 0u);
    const float tau_n = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rtau, (uint32_t)n_out * 4u, 0, 0));
    const float tn = a.tau ? tau_n : 1.0f;

    // value of token m at k = 4q + j of group i: element j M + m of the group, times kscale[k]
    auto val = [&](int i, int j, int m) {
        const int e = j * M + m;
        const float x = f4c(xv[i][e >> 2], e & 3);
        return has_ks ? __fmul_rn(f4c(ks[i], j), x) : x;
    };

    // 2a. per-token absmax and non-finite flag over the block
    float mx[M];
    int bad[M];
#pragma unroll
    for (int m = 0; m < M; ++m)
    {
        mx[m] = 0.0f;
        bad[m] = 0;
#pragma unroll
        for (int i = 0; i < G; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
            {
                const float v = fabsf(val(i, j, m));
                bad[m] |= !(v <= 3.4028234663852886e38f);
                mx[m] = fmaxf(mx[m], v);
            }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1)
        {
            mx[m] = fmaxf(mx[m], __shfl_xor(mx[m], off, kWave));
            bad[m] |= __shfl_xor(bad[m], off, kWave);
        }
        if (lane == 0)
        {
            s_mx[wv][m] = mx[m];
            s_bad[wv][m] = bad[m];
        }
    }
    dg_lds_barrier();
    int E[M];
#pragma unroll
    for (int m = 0; m < M; ++m)
    {
#pragma unroll
        for (int v = 0; v < NW; ++v)
        {
            mx[m] = fmaxf(mx[m], s_mx[v][m]);
            bad[m] |= s_bad[v][m];
        }
        E[m] = 0;
        (void)frexpf(mx[m], &E[m]);  // mx < 2^E (E = 0 for mx = 0)
    }

    // 2b. digit rows into LDS (unit u of row r holds 16-byte column u ^ (r & 7) of its 128-byte
    //     group) and the digit row sums
    int rs[4 * M];
#pragma unroll
    for (int e = 0; e < 4 * M; ++e) rs[e] = 0;
#pragma unroll
    for (int i = 0; i < G; ++i)
    {
        const int q = tid + kDgBlock * i;
        if (q >= GP) continue;
        const uint32_t k0 = 4u * (uint32_t)q;
#pragma unroll
        for (int m = 0; m < M; ++m)
        {
            uint32_t pk[4] = {0u, 0u, 0u, 0u};
#pragma unroll
            for (int j = 0; j < 4; ++j)
            {
                int X = bad[m] ? 0 : (int)__builtin_rintf(ldexpf(val(i, j, m), 30 - E[m]));
#pragma unroll
                for (int d = 0; d < 3; ++d)
                {
                    const int dg = ((X + 128) & 255) - 128;
                    X = (X - dg) >> 8;  // exact: X - dg is a multiple of 256
                    pk[d] |= (uint32_t)(dg & 255) << (8 * j);
                    rs[4 * m + d] += dg;
                }
                pk[3] |= (uint32_t)(X & 255) << (8 * j);
                rs[4 * m + 3] += X;
            }
#pragma unroll
            for (int d = 0; d < 4; ++d)
            {
                const uint32_t r = (uint32_t)(4 * m + d);
                const uint32_t addr = r * Kp + (k0 & ~127u) + ((((k0 >> 4) & 7u) ^ (r & 7u)) << 4) + (k0 & 15u);
                *reinterpret_cast<uint32_t*>(lds + addr) = pk[d];
            }
        }
    }
#pragma unroll
    for (int e = 0; e < 4 * M; ++e)
    {
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) rs[e] += __shfl_xor(rs[e], off, kWave);
        if (lane == 0) s_rs[wv][e] = rs[e];
    }
    dg_lds_barrier();
    int rsum = 0;
    if (t < 4 * M)
#pragma unroll
        for (int v = 0; v < NW; ++v) rsum += s_rs[v][t];

    // 3. MFMAs over the k tiles; columns t >= 4M read digit row 0 (never stored)
    Acc acc[1];
    acc[0].a0 = acc[0].a1 = acc[0].a2 = acc[0].a3 = v4i{0, 0, 0, 0};
    const int tr = t < 4 * M ? t : 0;
    const uint8_t* xrow = lds + (size_t)tr * Kp;
    const int sw0 = 16 * (g ^ (tr & 7)), sw1 = 16 * ((4 + g) ^ (tr & 7));
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
    {
        v4i x[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            x[j] = *reinterpret_cast<const v4i*>(xrow + kt * 256 + (j >> 1) * 128 + ((j & 1) ? sw1 : sw0));
        const v4i w1[1] = {w[kt]};
        compute_stage<1>(w1, x, acc);
    }

    // 4. digit sums of row 4g + p from the quad, int64 combine, tau * (fl(T) 2^(E - 30))
    int A[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) A[i] = acc_sum(acc[0], i) - 2 * rsum;
    auto pick = [&](int v0, int v1, int v2, int v3) { return p == 0 ? v0 : p == 1 ? v1 : p == 2 ? v2 : v3; };
    const long long T = (long long)pick(quad_bcast<0>(A[0]), quad_bcast<0>(A[1]), quad_bcast<0>(A[2]), quad_bcast<0>(A[3])) +
                        ((long long)pick(quad_bcast<1>(A[0]), quad_bcast<1>(A[1]), quad_bcast<1>(A[2]), quad_bcast<1>(A[3])) << 8) +
                        ((long long)pick(quad_bcast<2>(A[0]), quad_bcast<2>(A[1]), quad_bcast<2>(A[2]), quad_bcast<2>(A[3])) << 16) +
                        ((long long)pick(quad_bcast<3>(A[0]), quad_bcast<3>(A[1]), quad_bcast<3>(A[2]), quad_bcast<3>(A[3])) << 24);
    if (!live || n_out >= a.N || mt >= M) return;
    int Em = E[0], badm = bad[0];
#pragma unroll
    for (int m = 1; m < M; ++m)
        if (mt == m)
        {
            Em = E[m];
            badm = bad[m];
        }
    const float y = badm ? special_dot(a.B, false, a.kscale, reinterpret_cast<const uint32_t*>(a.rp), KT, a.K, M, n_out, mt, tn)
                         : tn * ldexpf((float)T, Em - 30);
    const size_t idx = (size_t)n_out * M + mt;
    if (a.y16)
        reinterpret_cast<_Float16*>(a.Y)[idx] = (_Float16)y;
    else
        reinterpret_cast<float*>(a.Y)[idx] = y;
}

template <int KT, int M>
hipError_t launch_dg(hipStream_t st, const DigitGemvArgs& a)
{
    static bool attr = false;
    const uint32_t lds_bytes = 4u * M * (uint32_t)KT * kTileK;
    if (!attr)
    {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemv_digits<KT, M>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_bytes);
        if (e != hipSuccess) return e;
        attr = true;
    }
    const unsigned blocks = (unsigned)ceil_div(ceil_div((size_t)a.N, 16), (size_t)(kDgBlock / kWave));
    hipLaunchKernelGGL((k_gemv_digits<KT, M>), dim3(blocks), dim3(kDgBlock), lds_bytes, st, a);
    return hipGetLastError();
}

template <int KT>
hipError_t launch_dg_m(hipStream_t st, const DigitGemvArgs& a, int M)
{
    switch (M)
    {
    case 1: return launch_dg<KT, 1>(st, a);
    case 2: return launch_dg<KT, 2>(st, a);
    case 3: if constexpr (KT <= 16) return launch_dg<KT, 3>(st, a); else return hipErrorInvalidValue;
    case 4: if constexpr (KT <= 16) return launch_dg<KT, 4>(st, a); else return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

hipError_t launch_digits(hipStream_t st, const void* B, bool b16, const float* kscale, size_t K, size_t M, int8_t* xi,
                         int32_t* rowsum, int32_t* ex)
{
    const size_t Kp = round_up(K, kTileK);
    k_digits<<<dim3((unsigned)M), kDigThreads, 0, st>>>(B, b16, kscale, (int)K, (int)M, (int)Kp, xi, rowsum, ex);
    return hipGetLastError();
}

size_t digit_chunks(size_t K) { return ceil_div(round_up(K, kTileK), (size_t)kChunk); }

hipError_t launch_digits_chunks(hipStream_t st, const void* B, bool b16, const float* kscale, size_t K, size_t M,
                                int8_t* xi, int32_t* rsp, int32_t* ex)
{
    const size_t Kp = round_up(K, kTileK);
    k_digits_chunks<<<dim3((unsigned)digit_chunks(K), (unsigned)M), kChunkThreads, 0, st>>>(B, b16, kscale, (int)K, (int)M,
                                                                                           (int)Kp, xi, rsp, ex);
    return hipGetLastError();
}

hipError_t launch_digit_combine_parts(hipStream_t st, const int32_t* part, int S, const int32_t* rsp, size_t P,
                                      const float* tau, const int32_t* ex, const uint32_t* rp, const void* B, bool b16,
                                      const float* kscale, size_t N, size_t K, size_t M, void* Y, bool y16)
{
    const size_t n = N * M;
    k_digit_combine_parts<<<dim3((unsigned)ceil_div(n, kDigBlock)), kDigBlock, 0, st>>>(
        part, S, rsp, (int)P, tau, ex, rp, (int)ceil_div(K, kTileK), B, b16, kscale, (int)N, (int)K, (int)M, Y, y16);
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

// (K, M) pairs the one-launch kernel is built for: the weight stages (4 KT VGPRs) and the
// activation share (16 G M VGPRs, G = ceil(KT / 4)) held together stay within ~200 registers
bool digit_gemv_ok(size_t N, size_t K, size_t M, bool b16, const void* B)
{
    if (b16 || M < 1 || M > 4 || K % 4 != 0 || N == 0 || (reinterpret_cast<uintptr_t>(B) & 15u) != 0) return false;
    const size_t KT = ceil_div(K, kTileK);
    if (KT == 4 || KT == 10 || KT == 16) return true;
    if (KT == 27) return M <= 2;
    if (KT == 32) return M == 1;
    return false;
}

hipError_t launch_digit_gemv(hipStream_t st, const void* rp, const float* tau, const float* kscale, const float* B,
                             size_t N, size_t K, size_t M, void* Y, bool y16)
{
    DigitGemvArgs a{};
    a.rp = static_cast<const u32x4*>(rp);
    a.tau = tau;
    a.kscale = kscale;
    a.B = B;
    a.Y = Y;
    a.N = (int)N;
    a.K = (int)K;
    a.y16 = y16 ? 1 : 0;
    switch (ceil_div(K, kTileK))
    {
    case 4: return launch_dg_m<4>(st, a, (int)M);
    case 10: return launch_dg_m<10>(st, a, (int)M);
    case 16: return launch_dg_m<16>(st, a, (int)M);
    case 27: return launch_dg_m<27>(st, a, (int)M);
    case 32: return M == 1 ? launch_dg<32, 1>(st, a) : hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
    }
}

}  // namespace nnhip
