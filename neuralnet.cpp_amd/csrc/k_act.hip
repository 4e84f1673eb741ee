// k_act.hip — activation-side kernels: fused [RMSNorm ->] per-token absmax -> int8
// quantization into the token-major layout the ternary GEMV/GEMM read, RMSNorm alone,
// and conversions between that layout and the reference int8 container.
//
// Every kernel here evaluates the per-token sum of squares in one fixed order, the same as
// the oracle: 512 strided parts (feature f in part f % 512), each summed in ascending f, then
// the xor butterfly over 256,128,...,1. So the normalized values, the scale and the int8 codes
// are bit-identical to the unfused reference sequence whichever kernel runs.
//
// Kernels by shape:
//   k_token_regs   M > 64, K up to 512 * 22: 8 tokens per 16-wave block (M <= 8192 and
//                  K <= 5120, or K <= 7168 without RMSNorm), else 4 per 8-wave block. Each
//                  thread loads its rows (16 B = 4 tokens per row) once and keeps them in
//                  registers through the passes (sum of squares, absmax, quantize), so X is read
//                  from HBM exactly once. With RMSNorm a thread's rows are the features of its
//                  sum-of-squares part; without it each wave of an 8-token block reads one
//                  contiguous band of rows. Codes leave through a 4x4 byte transpose in lane
//                  quads as dword stores.
//   k_token_one    M <= 64, K up to 512 * 22: one token per block, 512 threads, thread t owns
//                  part t and holds one element per row (decode sizes: the per-token VALU work
//                  of the 4-token kernel on one CU was its limit).
//   k_token_wave   larger K, M <= 32: one wave per token, lane l owns parts l + 64q (q = 0..7).
//   k_token_lanes  larger K, M > 32: 64 tokens per block, re-reads X per pass.
#include "common.hpp"
#include "token_quant.hpp"

#include <cmath>

namespace nnhip
{
namespace
{

constexpr int kBlock = 256;
// Cache-policy operand of the register quantizer's xi stores. The 8-token blocks (M <= 8192: a
// grid of one or a few resident rounds) write the codes through the L2 (kPolicySys) as they are
// produced: at M = 2048, K = 4096 12.1 -> 10.9 us, RMSNorm 2560 9.35 -> 9.0 us, K = 6912 21.1 ->
// 20.9 us. The 4-token blocks (larger M, many rounds) keep the default policy, 1-2 % faster
// there (2560 x 32768: 157.6-159.2 against 160.4-161.0 us).
template <int TPB>
constexpr int kXiPolicy = TPB >= 8 ? kPolicySys : 0;
#ifndef NNHIP_ONE_TOK_MAX_M
#define NNHIP_ONE_TOK_MAX_M 64  // largest M for k_token_one (K=6912, M=64: 6.8 us per call, the
                                // 4-token kernel 11.0; equal at K=2560)
#endif

__device__ __forceinline__ uint32_t pack4(int q0, int q1, int q2, int q3)
{
    // low bytes of q0..q3 -> bytes 0..3
    return __builtin_amdgcn_perm(__builtin_amdgcn_perm((uint32_t)q3, (uint32_t)q2, 0x0c0c0400u),
                                 __builtin_amdgcn_perm((uint32_t)q1, (uint32_t)q0, 0x0c0c0400u), 0x05040100u);
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

// Value of lane l ^ OFF as seen after the butterfly levels above OFF (descending offsets):
// by then a lane's value depends only on its lane bits below 2*OFF, so any partner with those
// bits equal to (l mod 2*OFF) ^ OFF carries the same value. OFF = 1, 2: quad_perm [1,0,3,2] /
// [2,3,0,1]; OFF = 4, 8: row_ror (l - OFF mod 16 agrees with l ^ OFF below 2*OFF); larger OFF:
// ds_bpermute.
template <int OFF>
__device__ __forceinline__ int lane_xor(int v)
{
    if constexpr (OFF == 1) return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);
    else if constexpr (OFF == 2) return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);
    else if constexpr (OFF == 4) return __builtin_amdgcn_mov_dpp(v, 0x124, 0xF, 0xF, false);
    else if constexpr (OFF == 8) return __builtin_amdgcn_mov_dpp(v, 0x128, 0xF, 0xF, false);
    else return __shfl_xor(v, OFF, kWave);
}
template <int OFF>
__device__ __forceinline__ float lane_xor(float v)
{
    return __builtin_bit_cast(float, lane_xor<OFF>(__builtin_bit_cast(int, v)));
}

// Butterfly over lane bits below 2*OFF (offsets OFF, OFF/2, ..., 1), four values at a time so
// the lane exchanges of one level overlap. Sum: fl(own + partner), the fixed order of the
// oracle's tree; max ignores NaN as `a > b ? a : b` does; integer sum is exact.
template <int OFF>
__device__ __forceinline__ void bfly_fsum(float (&v)[4])
{
    float o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = lane_xor<OFF>(v[i]);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = __fadd_rn(v[i], o[i]);
    if constexpr (OFF > 1) bfly_fsum<OFF / 2>(v);
}
// Max over the same lanes of values that are never NaN and never negative (absolute values,
// +0 included): their bit patterns order as unsigned integers, so one integer max per level
// replaces a float compare and select.
template <int OFF>
__device__ __forceinline__ void bfly_umax(uint32_t (&v)[4])
{
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = (uint32_t)lane_xor<OFF>((int)v[i]);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = o[i] > v[i] ? o[i] : v[i];
    if constexpr (OFF > 1) bfly_umax<OFF / 2>(v);
}
template <int OFF>
__device__ __forceinline__ void bfly_isum(int (&v)[4])
{
    int o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = lane_xor<OFF>(v[i]);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] += o[i];
    if constexpr (OFF > 1) bfly_isum<OFF / 2>(v);
}

__device__ __forceinline__ int lane_j(int fl) { return fl & 3; }

// Integer sum over lane bits LO..log2(2*OFF)-1 (offsets OFF down to LO).
template <int OFF, int LO>
__device__ __forceinline__ int bfly_isum1(int v)
{
    v += lane_xor<OFF>(v);
    if constexpr (OFF > LO) return bfly_isum1<OFF / 2, LO>(v);
    else return v;
}

// 4x4 byte transpose inside each quad of lanes: lane j (= lane & 3) holds bytes B_j[0..3] and
// ends with B_0[j], B_1[j], B_2[j], B_3[j]. Two exchanges, 16-bit halves with lane j^2, then
// bytes with lane j^1 (v_perm: bytes 0..3 are the second operand, 4..7 the first).
__device__ __forceinline__ uint32_t quad_transpose(uint32_t v, int j)
{
    const uint32_t p2 = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false);
    const uint32_t a = __builtin_amdgcn_perm(p2, v, (j & 2) ? 0x03020706u : 0x05040100u);
    const uint32_t p1 = (uint32_t)__builtin_amdgcn_mov_dpp((int)a, 0xB1, 0xF, 0xF, false);
    return __builtin_amdgcn_perm(p1, a, (j & 1) ? 0x03070105u : 0x06020400u);
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
        // parts lane + 64q; the butterfly levels 256, 128, 64 stay in the lane
        float pq[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) pq[q] = 0.0f;
        for (size_t f0 = 0; f0 < K; f0 += kParts)
#pragma unroll
            for (int q = 0; q < 8; ++q)
            {
                const size_t f = f0 + 64 * q + (size_t)lane;
                if (f < K)
                {
                    const float x = X[f * M + m];
                    pq[q] = __fadd_rn(pq[q], __fmul_rn(x, x));
                }
            }
        float part = tree_levels(pq);
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) part = __fadd_rn(part, __shfl_xor(part, off, kWave));
        ri = rms_inv_of(part, inv_f, eps);
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
// Large K fallback: 64 tokens per block (lane = token, coalesced rows of the (K, M) layout),
// 8 waves; wave w owns features f = 64*b + 8*w + j (j = 0..7), i.e. parts 64(b%8) + 8w + j.
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
        // parts 64q + 8w + j (q = b % 8); the butterfly levels 256, 128, 64 combine q in the lane
        float acc[8][8];
#pragma unroll
        for (int q = 0; q < 8; ++q)
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[q][j] = 0.0f;
        if (active)
            for (size_t b = 0; b < nb; b += 8)
            {
#pragma unroll
                for (int q = 0; q < 8; ++q)
#pragma unroll
                    for (int j = 0; j < 8; ++j)
                    {
                        const size_t f = 64 * (b + q) + 8 * w + j;
                        if (f < K)
                        {
                            const float x = X[f * M + m];
                            acc[q][j] = __fadd_rn(acc[q][j], __fmul_rn(x, x));
                        }
                    }
            }
#pragma unroll
        for (int j = 0; j < 8; ++j)
        {
            float v[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) v[q] = acc[q][j];
            part[8 * w + j][lane] = tree_levels(v);
        }
        __syncthreads();
        // the levels 32..1 on the lower halves: v[p] = v[p] + v[p + off] for p < off
        float v[64];
#pragma unroll
        for (int p = 0; p < 64; ++p) v[p] = part[p][lane];
        ri = rms_inv_of(tree_levels(v), inv_f, eps);
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

// ---------------------------------------------------------------------------------------
// Large M: TPB tokens per block (4 or 8) and 2*TPB waves, X read from HBM exactly once.
// A thread holds 4 tokens of one row per round (16 B, a float4 when M % 4 == 0); LPR = TPB/4
// lanes share a row (a 16- or 32-byte segment), so a wave covers RPW = 64/LPR rows and a round
// RR = reg_waves*RPW = 512 rows. Thread (wave w, lane RPW*h + fl) loads rows f = RR*r + RPW*w + fl
// (r < R), tokens 4h..4h+3, keeps them in registers, and owns sum-of-squares part f % 512 of its
// four tokens. The butterfly levels down to offset RPW go through LDS, the rest are lane
// shuffles.
template <int TPB>
constexpr int reg_waves = 2 * TPB;

// Everything a block needs to load and finish token groups (uniform across the block).
template <int TPB>
struct TokShared
{
    float red[kParts][TPB];  // sum-of-squares parts
    float wred[reg_waves<TPB>][TPB];
    int wsum[reg_waves<TPB>][TPB];
    float tok_ri[TPB];
    float tok_sc[TPB], tok_rc[TPB];  // per-token scale and its reciprocal
    float4 tok_ex[TPB];              // exact path: prescale xs, s * xs, fl(1 / (s * xs))
};

// Rows of a thread: base + step * r for round r < R. Strided (the default): row RR * r + ro, so
// thread ro owns sum-of-squares part ro (the fixed order of the RMSNorm sum). Contiguous (no
// RMSNorm: the absmax and the code sums do not depend on the order): wave w reads the band of
// R * RPW rows from R * RPW * w, RPW rows per round, so its loads stay within a few MiB of X.
template <int R, int TPB, bool kContig>
__device__ __forceinline__ int row_base(int ro)
{
    constexpr int RPW = kWave / (TPB / 4);
    return kContig ? (ro / RPW) * (R * RPW) + ro % RPW : ro;
}
template <int R, int TPB, bool kContig>
constexpr int row_step = kContig ? kWave / (TPB / 4) : reg_waves<TPB> * (kWave / (TPB / 4));

// Issue the loads of group g into x (vector path: one buffer resource over X, K*M*4 < 2^31
// checked at launch, so rows past K and tokens past M read 0 without a branch).
template <int R, bool kVec, int TPB, bool kContig = false>
__device__ __forceinline__ void load_group(float (&x)[R][4], const TokArgs& a, int g, int ro, int h)
{
    const int mt = g * TPB + 4 * h;
    const int base = row_base<R, TPB, kContig>(ro);
    constexpr int step = row_step<R, TPB, kContig>;
    if (kVec)
    {
        typedef float v4f __attribute__((ext_vector_type(4)));
        const __amdgpu_buffer_rsrc_t rx =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(a.X), (short)0, a.K * a.M * 4, 0x00020000);
        const uint32_t moff = mt < a.M ? (uint32_t)mt * 4u : 0x80000000u;
#pragma unroll
        for (int r = 0; r < R; ++r)
        {
            const v4f v = __builtin_bit_cast(
                v4f, __builtin_amdgcn_raw_buffer_load_b128(rx, moff + (uint32_t)(base + step * r) * (uint32_t)a.M * 4u, 0, 0));
            x[r][0] = v[0];
            x[r][1] = v[1];
            x[r][2] = v[2];
            x[r][3] = v[3];
        }
    }
    else
    {
#pragma unroll
        for (int r = 0; r < R; ++r)
        {
            const int f = base + step * r;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                x[r][i] = (f < a.K && mt + i < a.M) ? a.X[(size_t)f * a.M + mt + i] : 0.0f;
        }
    }
}

// The three passes over one group held in registers: sum of squares -> rms_inv (RMSNorm),
// per-token absmax -> scale, quantize -> xi / s / rowsum (and the reference container).
template <int R, bool kVec, int TPB, bool kNormOK, bool kContig = false>
__device__ __forceinline__ void finish_group(float (&x)[R][4], const float (&gm)[R], const TokArgs& a,
                                             TokShared<TPB>& sh, int g, int w, int fl, int h, int ro)
{
    static_assert(!(kContig && kNormOK), "the contiguous row bands only serve quantization without RMSNorm");
    constexpr int LPR = TPB / 4;          // lanes per row
    constexpr int RPW = kWave / LPR;      // rows per wave per round
    constexpr int RW = reg_waves<TPB>;    // waves per block
    constexpr int RR = RW * RPW;          // rows per round
    constexpr int NP = kParts / RR;       // parts per thread (1 or 2)
    const int mt = g * TPB + 4 * h;       // first of this thread's four tokens

    // ---- pass 1: sum of squares -> rms_inv, then normalize in place
    if (kNormOK && a.norm)
    {
        float acc[NP][4];
#pragma unroll
        for (int q = 0; q < NP; ++q)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[q][i] = 0.0f;
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[r % NP][i] = __fadd_rn(acc[r % NP][i], __fmul_rn(x[r][i], x[r][i]));
#pragma unroll
        for (int q = 0; q < NP; ++q)
#pragma unroll
            for (int i = 0; i < 4; ++i) sh.red[ro + RR * q][4 * h + i] = acc[q][i];
        __syncthreads();
        if (w == 0)
        {
            float sum[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
            {
                float v[kParts / RPW];
#pragma unroll
                for (int k = 0; k < kParts / RPW; ++k) v[k] = sh.red[fl + RPW * k][4 * h + i];
                sum[i] = tree_levels(v);
            }
            bfly_fsum<RPW / 2>(sum);
            if (fl == 0)
#pragma unroll
                for (int i = 0; i < 4; ++i) sh.tok_ri[4 * h + i] = rms_inv_of(sum[i], a.inv_f, a.eps);
        }
        __syncthreads();
        float ri[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) ri[i] = sh.tok_ri[4 * h + i];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int i = 0; i < 4; ++i) x[r][i] = __fmul_rn(__fmul_rn(x[r][i], ri[i]), gm[r]);
    }

    const int base = row_base<R, TPB, kContig>(ro);
    constexpr int step = row_step<R, TPB, kContig>;
    if (a.mode == 1)
    {
#pragma unroll
        for (int r = 0; r < R; ++r)
        {
            const int f = base + step * r;
            if (f >= a.K) continue;
            if (kVec)
            {
                if (mt < a.M)
                    *reinterpret_cast<float4*>(a.fout + (size_t)f * a.M + mt) = make_float4(x[r][0], x[r][1], x[r][2], x[r][3]);
            }
            else
            {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (mt + i < a.M) a.fout[(size_t)f * a.M + mt + i] = x[r][i];
            }
        }
        return;
    }

    // ---- pass 2: per-token absmax -> scale (fmaxf ignores NaN, as `a > m ? a : m` from 0 does).
    // The waves' maxima meet in LDS; TPB lanes of wave 0 reduce them, one token each, and post
    // the scale and its reciprocal for the block.
    uint32_t mx[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
    {
        float m = 0.0f;
#pragma unroll
        for (int r = 0; r < R; ++r) m = fmaxf(m, fabsf(x[r][i]));
        mx[i] = __builtin_bit_cast(uint32_t, m);
    }
    bfly_umax<RPW / 2>(mx);
    if (fl == 0)
#pragma unroll
        for (int i = 0; i < 4; ++i) sh.wred[w][4 * h + i] = __builtin_bit_cast(float, mx[i]);
    __syncthreads();
    if (threadIdx.x < TPB)
    {
        float t = sh.wred[0][threadIdx.x];
#pragma unroll
        for (int v = 1; v < RW; ++v) t = fmaxf(t, sh.wred[v][threadIdx.x]);
        const float scv = __fmul_rn(t, 1.0f / 127.0f);
        sh.tok_sc[threadIdx.x] = scv;
        sh.tok_rc[threadIdx.x] = quant_rcp(scv);
        const float xs = scv < 0x1p-100f ? 0x1p100f : 1.0f;
        const float se = __fmul_rn(scv, xs);
        sh.tok_ex[threadIdx.x] = make_float4(xs, se, quant_rcp(se), 0.0f);
    }
    __syncthreads();
    float sc[4], rc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
    {
        sc[i] = sh.tok_sc[4 * h + i];
        rc[i] = sh.tok_rc[4 * h + i];
    }

    // ---- pass 3: quantize; codes on the fast path with one flag per round. Rows past K hold
    // x = 0 (or NaN when rms_inv is infinite), which every path turns into code 0. A round with a
    // flagged element (a product near a tie, NaN or inf, or any product of a token whose
    // reciprocal overflowed) is recomputed by the exact division-free code for its four elements,
    // on x * xs / (s * xs) with the token's power-of-two prescale xs (2^100 below s = 2^-100, else
    // 1): the same quotient, with s * xs in quantize_exact's range.
    uint32_t pk[R];
    uint32_t amb = 0;  // bit r: round r holds a flagged element
#pragma unroll
    for (int r = 0; r < R; ++r)
    {
        bool f = false;
        int qv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) qv[i] = quantize_code(x[r][i], rc[i], f);
        pk[r] = pack4(qv[0], qv[1], qv[2], qv[3]);
        amb |= f ? 1u << r : 0u;
    }
    if (amb)
    {
        float4 ex[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) ex[i] = sh.tok_ex[4 * h + i];
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (amb >> r & 1u)
            {
                int qv[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) qv[i] = quantize_exact(__fmul_rn(x[r][i], ex[i].x), ex[i].y, ex[i].z);
                pk[r] = pack4(qv[0], qv[1], qv[2], qv[3]);
            }
    }
    // xi: after a quad transpose lane (quad q, position j) holds token 4h+j for the four rows
    // 4q..4q+3 of its wave's slice, one dword store each; dot4 against 1s sums those codes.
    // Stores go through one buffer resource over xi (M * Kp < 2^31 at launch) from one offset per
    // thread; a token past M gets an offset past the range, which the buffer store drops. Rows
    // past Kp (the next token's bytes otherwise) are never stored: rounds below Kp / RR are whole,
    // the round at Kp / RR holds rows below Kp in the threads whose first row of a round is below
    // Kp % RR (Kp % 256 == 0, so a thread's four rows are all in or all out), later rounds none.
    const int wpr = (a.M + 3) / 4;
    const int j = lane_j(fl);
    const int q0 = base - (fl & 3);  // first of the thread's four rows in round 0
    const __amdgpu_buffer_rsrc_t rxi =
        __builtin_amdgcn_make_buffer_rsrc(a.xi, (short)0, a.M * a.Kp, 0x00020000);
    const uint32_t xoff = mt + j < a.M ? (uint32_t)((mt + j) * a.Kp + q0) : 0x80000000u;
    const uint32_t xpart = q0 < a.Kp % RR ? xoff : 0x80000000u;
    const int whole = a.Kp / RR;
    if (a.xq_ref && g * LPR + h < wpr)
#pragma unroll
        for (int r = 0; r < R; ++r)
        {
            const int f = base + step * r;
            if (f < a.K) a.xq_ref[(size_t)f * wpr + g * LPR + h] = pk[r];
        }
    int tsum = 0;
#pragma unroll
    for (int r = 0; r < R; ++r)
    {
        const uint32_t col = quad_transpose(pk[r], j);
        tsum = __builtin_amdgcn_sdot4((int)col, 0x01010101, tsum, false);
        if constexpr (kContig)
        {
            // a band's rounds end at Kp in any round (rows past Kp read 0 and are never stored)
            const uint32_t o = q0 + step * r < a.Kp ? xoff + (uint32_t)(step * r) : 0x80000000u;
            __builtin_amdgcn_raw_buffer_store_b32(col, rxi, o, 0, kXiPolicy<TPB>);
        }
        else if (r < whole)
            __builtin_amdgcn_raw_buffer_store_b32(col, rxi, xoff + (uint32_t)(RR * r), 0, kXiPolicy<TPB>);
        else if (r == whole)
            __builtin_amdgcn_raw_buffer_store_b32(col, rxi, xpart + (uint32_t)(RR * r), 0, kXiPolicy<TPB>);
    }
    tsum = bfly_isum1<RPW / 2, 4>(tsum);  // over the quads of the wave's slice
    if (fl < 4) sh.wsum[w][4 * h + j] = tsum;
    __syncthreads();
    if (w == 0 && fl == 0)
    {
#pragma unroll
        for (int i = 0; i < 4; ++i)
        {
            int t = 0;
#pragma unroll
            for (int v = 0; v < RW; ++v) t += sh.wsum[v][4 * h + i];
            if (mt + i < a.M)
            {
                a.s[mt + i] = sc[i];
                a.rowsum[mt + i] = t;
            }
        }
    }
}

// One block per token group; block b takes group slot(b), XCD-aware when the group count is a
// multiple of 8, so the blocks of one XCD take consecutive groups and the groups sharing a
// 128-byte row segment of X meet in one L2.
// (R = 12 and 14 with 4-token blocks: at least 3 waves per SIMD, 168 registers; left to itself the
// compiler took 171 for R = 14, i.e. 2 waves per SIMD, too few loads in flight at prefill sizes)
template <int R, bool kVec, int TPB, bool kNormOK, bool kContig = false>
__global__ __launch_bounds__(reg_waves<TPB> * kWave, ((R == 12 || R == 14) && TPB == 4) ? 3 : 1) void k_token_regs(TokArgs a, const float* __restrict__ gamma,
                                                                  int n_groups)
{
    constexpr int RPW = kWave / (TPB / 4);
    constexpr int RR = reg_waves<TPB> * RPW;
    static_assert(TPB == 4 || TPB == 8, "tokens per block");
    __shared__ TokShared<TPB> sh;

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int fl = lane % RPW, h = lane / RPW;  // row within the wave's slice, token quad
    const int ro = RPW * w + fl;
    const int b = blockIdx.x;
    const int g = n_groups % 8 == 0 ? (b & 7) * (n_groups >> 3) + (b >> 3) : b;

    float x[R][4];
    load_group<R, kVec, TPB, kContig>(x, a, g, ro, h);
    float gm[R];
    if (kNormOK && a.norm)
    {
        const __amdgpu_buffer_rsrc_t rg =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(gamma), (short)0, a.K * 4, 0x00020000);
#pragma unroll
        for (int r = 0; r < R; ++r)
            gm[r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rg, (uint32_t)(RR * r + ro) * 4u, 0, 0));
    }
    finish_group<R, kVec, TPB, kNormOK, kContig>(x, gm, a, sh, g, w, fl, h, ro);
}

// Decode-sized M (up to 64 tokens): one token per block, 512 threads. Thread t owns sum-of-squares
// part t (rows f = t + 512 r, r < R) of token m = blockIdx.x and holds one element per row, so a
// token's VALU work (the three passes) is spread over M CUs rather than M/4, which is what bounds
// the 4-token kernel at these sizes (one CU per 4 tokens, ~20 VALU ops per element). Same passes,
// orders and codes as finish_group (one_token_finish, token_quant.hpp).
template <int R>
__global__ __launch_bounds__(kOneThreads) void k_token_one(TokArgs a, const float* __restrict__ gamma)
{
    __shared__ OneShared sh;
    if ((int)blockIdx.x >= a.M)
    {
        prefetch_block(a.pf, (int)blockIdx.x - a.M);
        return;
    }
    const int t = threadIdx.x, m = blockIdx.x;
    float x[R];
    if (a.gids)
    {
        const int id = a.gids[m];
        const bool ok = id >= 0 && id < a.gV;
#pragma unroll
        for (int r = 0; r < R; ++r)
        {
            const int f = t + kParts * r;
            x[r] = f < a.K ? (ok ? a.X[(size_t)id * a.K + f] : __builtin_nanf("")) : 0.0f;
            if (f < a.K) a.gout[(size_t)m * a.K + f] = x[r];
        }
    }
    else
    {
#pragma unroll
        for (int r = 0; r < R; ++r)
        {
            const int f = t + kParts * r;
            x[r] = f < a.K ? a.X[a.xtm ? (size_t)m * a.K + f : (size_t)f * a.M + m] : 0.0f;
        }
    }
    one_token_finish<R>(x, a, gamma, sh);
}

// The same passes after the epilogue of a split-k GEMV (k_gemv_part) and the decoder's residual
// add: x = (tau[f] * s_in[m]) * float(sum over slices of part[.][m][f] - 2 rowsum_in[m]) [+ bias[f]]
// [+ res[f][m]], the deep GEMV's epilogue operation for operation (the slice sums add up exactly),
// stored to xout (the residual stream, may alias res) and quantized for the next BitLinear.
template <int R, int kEpiMaxSlices>
__global__ __launch_bounds__(kOneThreads) void k_token_epi(TokArgs a, EpiArgs e, const float* __restrict__ gamma)
{
    __shared__ OneShared sh;
    if ((int)blockIdx.x >= a.M)
    {
        prefetch_block(a.pf, (int)blockIdx.x - a.M);
        return;
    }
    const int t = threadIdx.x, m = blockIdx.x, N = a.K, M = a.M;
    const float sv = e.s_in[m];
    const int rs2 = 2 * e.rowsum_in[m];
    // every load of the thread is issued before the first use: the slice sums through one buffer
    // resource over part (slices past S and features past N read 0), tau and the residual
    const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int32_t*>(e.part), (short)0, (int)((size_t)e.S * M * N * 4), 0x00020000);
    int ps[R][kEpiMaxSlices];
    float tv[R], rv[R];
#pragma unroll
    for (int r = 0; r < R; ++r)
    {
        const int f = t + kParts * r;
#pragma unroll
        for (int k = 0; k < kEpiMaxSlices; ++k)
        {
            const uint32_t off = (k < e.S && f < N) ? (uint32_t)(((size_t)k * M + m) * N + f) * 4u : 0x80000000u;
            ps[r][k] = __builtin_bit_cast(int, __builtin_amdgcn_raw_buffer_load_b32(rp, off, 0, 0));
        }
        tv[r] = f < N ? e.tau[f] : 0.0f;
        rv[r] = (f < N && e.res) ? e.res[e.tm ? (size_t)m * N + f : (size_t)f * M + m] : 0.0f;
    }
    float x[R];
#pragma unroll
    for (int r = 0; r < R; ++r)
    {
        const int f = t + kParts * r;
        x[r] = 0.0f;
        if (f < N)
        {
            int acc = 0;
#pragma unroll
            for (int k = 0; k < kEpiMaxSlices; ++k) acc += ps[r][k];
            float y = (tv[r] * sv) * (float)(acc - rs2);
            if (e.bias) y = y + e.bias[f];
            if (e.res) y = y + rv[r];
            e.xout[e.tm ? (size_t)m * N + f : (size_t)f * M + m] = y;
            x[r] = y;
        }
    }
    one_token_finish<R>(x, a, gamma, sh);
}

// slices are loaded up to a compiled maximum (4 or 8; those past S read 0)
template <int R>
void launch_epi_r(hipStream_t st, const TokArgs& a, const EpiArgs& e, const float* gamma)
{
    if (e.S <= 4)
        hipLaunchKernelGGL((k_token_epi<R, 4>), dim3((unsigned)(a.M + a.pf.blocks)), dim3(kOneThreads), 0, st, a, e,
                           gamma);
    else
        hipLaunchKernelGGL((k_token_epi<R, 8>), dim3((unsigned)(a.M + a.pf.blocks)), dim3(kOneThreads), 0, st, a, e,
                           gamma);
}

template <int... Rs>
bool launch_epi_pick(int rounds, hipStream_t st, const TokArgs& a, const EpiArgs& e, const float* gamma)
{
    bool done = false;
    ((done = done || (Rs >= rounds && (launch_epi_r<Rs>(st, a, e, gamma), true))), ...);
    return done;
}

template <int R>
void launch_one_r(hipStream_t st, const TokArgs& a, const float* gamma)
{
    hipLaunchKernelGGL(k_token_one<R>, dim3((unsigned)(a.M + a.pf.blocks)), dim3(kOneThreads), 0, st, a, gamma);
}

template <int... Rs>
bool launch_one_pick(int rounds, hipStream_t st, const TokArgs& a, const float* gamma)
{
    bool done = false;
    ((done = done || (Rs >= rounds && (launch_one_r<Rs>(st, a, gamma), true))), ...);
    return done;
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

#ifndef NNHIP_TOK8_MAX_ROUNDS
#define NNHIP_TOK8_MAX_ROUNDS 10  // largest K/512 rounds for the 8-token register kernel
#endif
constexpr size_t kSmallM = 32;
constexpr size_t kOneTokMaxM = NNHIP_ONE_TOK_MAX_M;

template <int TPB, int R, bool kNormOK = true, bool kContig = false>
void launch_regs_r(bool vec, hipStream_t st, int n_groups, const TokArgs& a, const float* gamma)
{
    auto kern = vec ? k_token_regs<R, true, TPB, kNormOK, kContig> : k_token_regs<R, false, TPB, kNormOK, kContig>;
    hipLaunchKernelGGL(kern, dim3((unsigned)n_groups), dim3(reg_waves<TPB> * kWave), 0, st, a, gamma, n_groups);
}

// Launch the instantiation with the smallest R >= rounds from the ascending list Rs; false if
// none is large enough.
template <int TPB, int... Rs>
bool launch_regs_pick(int rounds, bool vec, hipStream_t st, int n_groups, const TokArgs& a, const float* gamma)
{
    bool done = false;
    ((done = done || (Rs >= rounds && (launch_regs_r<TPB, Rs>(vec, st, n_groups, a, gamma), true))), ...);
    return done;
}

// the same without the RMSNorm passes, rows in contiguous bands per wave
template <int TPB, int... Rs>
bool launch_regs_pick_contig(int rounds, bool vec, hipStream_t st, int n_groups, const TokArgs& a)
{
    bool done = false;
    ((done = done || (Rs >= rounds && (launch_regs_r<TPB, Rs, false, true>(vec, st, n_groups, a, nullptr), true))),
     ...);
    return done;
}

}  // namespace

static hipError_t launch_token_kernel(hipStream_t st, const float* X, const float* gamma, bool norm,
                                      float eps, size_t K, size_t M, int mode, int8_t* xi, float* s,
                                      int32_t* rowsum, uint32_t* xq_ref, float* fout, const Prefetch* pf = nullptr)
{
    if (M == 0) return hipSuccess;
    const float inv_f = 1.0f / (float)K;
    const size_t Kp = round_up(K, kTileK);
    const int rounds = (int)ceil_div(K, (size_t)512);
    // the register kernel addresses X through one 31-bit buffer range, including the padding
    // rows of its last round (at most 4096 rows past K). It serves every larger M up to 22
    // rounds (K <= 11264).
    // decode sizes: one token per block (more CUs share each token group's VALU work)
    if (M <= kOneTokMaxM && rounds <= 22)
    {
        TokArgs a{X, norm, eps, inv_f, (int)K, (int)M, (int)Kp, mode, xi, s, rowsum, xq_ref, fout};
        if (pf) a.pf = *pf;
        if (launch_one_pick<1, 2, 3, 4, 5, 6, 8, 10, 12, 14, 16, 18, 20, 22>(rounds, st, a, gamma))
            return hipGetLastError();
    }
    if (rounds <= 22 && (K + 4096) * M * 4 < 0x7FFFFFFFull)
    {
        // rows are read as float4 when every row start is 16-byte aligned
        const bool vec = M % 4 == 0 && reinterpret_cast<uintptr_t>(X) % 16 == 0 &&
                         (fout == nullptr || reinterpret_cast<uintptr_t>(fout) % 16 == 0);
        // 8 tokens per block (32-byte row segments, 16 waves) while a thread's rows fit the
        // 128 registers of a 1024-thread block and the grid is at most a few rounds (K=4096,
        // M=2048: 14.2 against 15.7 us; 2560 x 32768, where the smaller blocks keep more waves
        // resident: 193 against 159 us); 4 tokens (16-byte segments, 8 waves) otherwise
        TokArgs a{X, norm, eps, inv_f, (int)K, (int)M, (int)Kp, mode, xi, s, rowsum, xq_ref, fout};
        // Without RMSNorm the 8-token layout also serves 11 to 14 rounds (K <= 7168: the FFN
        // width 6912): those instantiations leave the norm passes out, which keeps them within
        // the 128 registers (K=6912, M=2048: 16-byte segments read the 56 MB at ~4 TB/s).
        const bool tok8 = vec && M <= 8192 && (rounds <= NNHIP_TOK8_MAX_ROUNDS || (!norm && mode == 0 && rounds <= 14));
        const int n_groups = (int)ceil_div(M, (size_t)(tok8 ? 8 : 4));
        // Without RMSNorm (mode 0) the 8-token blocks read each wave's rows as one contiguous band
        // (the absmax and the code sums do not depend on the order): K=4096, M=2048 11.1 -> 10.3 us,
        // K=6912 21.6-22.1 -> 19.8-20.1 us, the same codes (A/B of two builds on one box).
        bool launched;
        if (tok8 && !norm && mode == 0)
            launched = launch_regs_pick_contig<8, 1, 2, 3, 4, 5, 6, 8, 10, 12, 14>(rounds, vec, st, n_groups, a);
        else
            launched = tok8 ? launch_regs_pick<8, 1, 2, 3, 4, 5, 6, 8, 10>(rounds, vec, st, n_groups, a, gamma)
                            : launch_regs_pick<4, 1, 2, 3, 4, 5, 6, 8, 10, 12, 14, 16, 18, 20, 22>(rounds, vec, st,
                                                                                                n_groups, a, gamma);
        if (launched) return hipGetLastError();
    }
    if (M <= kSmallM)
    {
        const unsigned grid = (unsigned)ceil_div(M, kBlock / kWave);
        hipLaunchKernelGGL(k_token_wave, dim3(grid), dim3(kBlock), 0, st, X, gamma, norm, eps, inv_f,
                           K, M, Kp, mode, xi, s, rowsum, xq_ref, fout);
        return hipGetLastError();
    }
    const unsigned grid = (unsigned)ceil_div(M, kWave);
    hipLaunchKernelGGL(k_token_lanes, dim3(grid), dim3(kTW * kWave), 0, st, X, gamma, norm, eps,
                       inv_f, K, M, Kp, mode, xi, s, rowsum, xq_ref, fout);
    return hipGetLastError();
}

bool token_quant_tm_ok(size_t K, size_t M)
{
    return M >= 1 && M <= kOneTokMaxM && K >= 1 && ceil_div(K, (size_t)512) <= 22;
}

hipError_t launch_token_quant_tm(hipStream_t st, const float* X, const float* gamma, float eps, size_t K, size_t M,
                                 int8_t* xi, float* s, int32_t* rowsum, const Prefetch* pf)
{
    if (!token_quant_tm_ok(K, M)) return hipErrorInvalidValue;
    const int rounds = (int)ceil_div(K, (size_t)512);
    TokArgs a{X, gamma != nullptr, eps, 1.0f / (float)K, (int)K, (int)M, (int)round_up(K, kTileK), 0, xi, s, rowsum,
              nullptr, nullptr, 1};
    if (pf) a.pf = *pf;
    if (!launch_one_pick<1, 2, 3, 4, 5, 6, 8, 10, 12, 14, 16, 18, 20, 22>(rounds, st, a, gamma))
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_embed_token_quant(hipStream_t st, const float* table, const int32_t* ids, size_t V, const float* gamma,
                                   float eps, size_t K, size_t M, float* xout, int8_t* xi, float* s, int32_t* rowsum,
                                   const Prefetch* pf)
{
    if (!token_quant_tm_ok(K, M)) return hipErrorInvalidValue;
    const int rounds = (int)ceil_div(K, (size_t)512);
    TokArgs a{table, gamma != nullptr, eps, 1.0f / (float)K, (int)K, (int)M, (int)round_up(K, kTileK), 0, xi, s, rowsum,
              nullptr, nullptr, 1};
    if (pf) a.pf = *pf;
    a.gids = ids;
    a.gV = (int)V;
    a.gout = xout;
    if (!launch_one_pick<1, 2, 3, 4, 5, 6, 8, 10, 12, 14, 16, 18, 20, 22>(rounds, st, a, gamma))
        return hipErrorInvalidValue;
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
                            uint32_t* xq_ref, const Prefetch* pf)
{
    if (xq_ref && M % 4 != 0)
    {
        // tail bytes of the last word of each row must read 0: clear the container first
        const hipError_t e = launch_fill_u32(st, xq_ref, 0u, K * ceil_div(M, 4));
        if (e != hipSuccess) return e;
    }
    return launch_token_kernel(st, X, gamma, norm, eps, K, M, 0, xi, s, rowsum, xq_ref, nullptr, pf);
}

bool epilogue_quant_ok(size_t N, size_t M)
{
    return M >= 1 && M <= kOneTokMaxM && ceil_div(N, (size_t)kParts) <= 22;
}

hipError_t launch_epilogue_quant(hipStream_t st, const EpiArgs& e, const float* gamma, bool norm, float eps, size_t N,
                                 size_t M, int8_t* xi, float* s, int32_t* rowsum, const Prefetch* pf)
{
    if (M == 0) return hipSuccess;
    if (!epilogue_quant_ok(N, M)) return hipErrorInvalidValue;
    TokArgs a{nullptr, norm, eps, 1.0f / (float)N, (int)N, (int)M, (int)round_up(N, kTileK), 0, xi, s, rowsum,
              nullptr, nullptr};
    if (pf) a.pf = *pf;
    const int rounds = (int)ceil_div(N, (size_t)kParts);
    if (!launch_epi_pick<1, 2, 3, 4, 5, 6, 8, 10, 12, 14, 16, 18, 20, 22>(rounds, st, a, e, gamma))
        return hipErrorInvalidValue;
    return hipGetLastError();
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
