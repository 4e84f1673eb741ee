// k_prefill.hip — batched prefill of the decoder's attention: T new tokens for each of B
// sequences at positions pos0 .. pos0 + T - 1 in one pass, instead of T decode steps.
//
// Reference: GPTModel::generate fills the KV cache by calling forward_step once per context
// token (include/neuralnet.cpp/compute_layer_gpt.hpp:774-794); each call rotates the new key
// at its position, appends key and value to the caches and attends over positions [0, pos]
// (AttentionBase::forward_step, compute_layer_attention.hpp:1003-1091). The same results for
// all T tokens at once:
//   * k_kv_fill writes the T rotated keys and values of every sequence into cache rows
//     pos0 .. pos0 + T - 1 (RoPE as the decode append: two rounded products and a rounded sum);
//   * k_attn_prefill gives token t the softmax attention over cache rows [0, pos0 + t] (causal),
//     query head h reading KV head h / (H / Hkv).
//
// Layouts (device, f32): q (H*dk, M), k / v (Hkv*dk, M) and out (H*dk, M) feature-major with
// token column m = b*T + t (the BitLinear outputs of the B*T tokens); caches (B, max_len,
// Hkv*dk) as the decode step's; cos / sin (max_len, dk/2).
//
// k_attn_prefill: work-group = (32 queries, KV head g, sequence b) with one wave per query head
// of the group (R = H / Hkv waves), so each 32-key tile of K and V is staged in LDS once for all
// R heads. Per 32-key tile a wave computes S^T = K . Q^T (32 keys x 32 queries) on the fp32 MFMA
// v_mfma_f32_32x32x2_f32, folds it into an online softmax (running max and sum per query), and
// accumulates O^T += V^T . P^T. With S^T (not S) in the accumulators, lane l holds query l % 32
// and keys 8(v/4) + 4(l/32) + v%4 of its 16 elements v, which is exactly the B operand of the
// P . V products (lane l, k = l/32) when the keys of product s are taken in that order; the
// A operand of product s is then V[key][dimension] of that key for the lane's dimension. The sum
// over the head dimension in S^T takes product s = 4c + e over dimensions 8c + e and 8c + 4 + e
// (the two lane halves), which a lane reads as one 16-byte chunk of its K row. K and V rows are
// padded to dk + 4 floats in LDS, so the 16-byte reads of 8 consecutive rows cover all banks.
// Work-groups are issued heaviest first (the last query blocks attend over the most keys).
// f32 throughout; the accumulation order differs from a sequential dot product (results within
// 2e-6 relative of a float64 evaluation on the test data). Caches of f16 elements (compute = F16)
// are widened exactly when a tile is staged; the fill rounds the rotated keys and the values to
// the nearest f16 (ties to even), as the decode append does.
#include "common.hpp"

#include <cmath>

namespace nnhip
{
namespace
{

typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kPQ = 32;   // queries per work-group
constexpr int kPK = 32;   // keys per tile

__device__ __forceinline__ __amdgpu_buffer_rsrc_t pf_rsrc(const void* base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ float ld_f(__amdgpu_buffer_rsrc_t r, uint32_t off)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}

__device__ __forceinline__ float4 ld_f4(__amdgpu_buffer_rsrc_t r, uint32_t off)
{
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// Four cache elements at byte offset off as floats (f32, or f16 widened exactly)
template <typename CT>
__device__ __forceinline__ float4 ld_c4(__amdgpu_buffer_rsrc_t r, uint32_t off)
{
    if constexpr (sizeof(CT) == 4) return ld_f4(r, off);
    else
    {
        typedef _Float16 h4 __attribute__((ext_vector_type(4)));
        const h4 h = __builtin_bit_cast(h4, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
        return make_float4((float)h[0], (float)h[1], (float)h[2], (float)h[3]);
    }
}

// (x0, x1) = (x[j], x[j + dk/2]) -> x*cos + rotate_half(x)*sin: two rounded products and a
// rounded sum per output, as the decode append does.
__device__ __forceinline__ void pf_rope(float x0, float x1, float cs, float sn, float& y0, float& y1)
{
    y0 = __fadd_rn(__fmul_rn(x0, cs), __fmul_rn(-x1, sn));
    y1 = __fadd_rn(__fmul_rn(x1, cs), __fmul_rn(x0, sn));
}

// ------------------------------------------------------------------ cache fill

// Block = (32 tokens, KV head g): the head's dk feature rows of k and v for the 32 tokens are
// read along tokens (coalesced), transposed through LDS and written as cache rows (coalesced
// along features), the keys rotated at their positions.
template <int DK, typename CT>
__global__ __launch_bounds__(256) void k_kv_fill(const float* __restrict__ k, const float* __restrict__ v, int B, int T,
                                                 int Hkv, int pos0, const float* __restrict__ cosT,
                                                 const float* __restrict__ sinT, CT* __restrict__ kc,
                                                 CT* __restrict__ vc, int max_len)
{
    constexpr int HALF = DK / 2;
    __shared__ float sk[DK][kPQ + 1];
    __shared__ float sv[DK][kPQ + 1];
    const int M = B * T;
    const int g = blockIdx.y;
    const int m0 = blockIdx.x * kPQ;
    const int tid = threadIdx.x;
    const int row = Hkv * DK;
    for (int idx = tid; idx < DK * kPQ; idx += 256)
    {
        const int i = idx / kPQ, c = idx % kPQ;
        const int m = m0 + c;
        const size_t src = (size_t)(g * DK + i) * (size_t)M + (size_t)m;
        sk[i][c] = m < M ? k[src] : 0.0f;
        sv[i][c] = m < M ? v[src] : 0.0f;
    }
    __syncthreads();
    for (int idx = tid; idx < kPQ * HALF; idx += 256)
    {
        const int c = idx / HALF, j = idx % HALF;
        const int m = m0 + c;
        if (m >= M) continue;
        const int b = m / T, t = m % T;
        const int p = pos0 + t;
        CT* kr = kc + ((size_t)b * (size_t)max_len + (size_t)p) * (size_t)row + (size_t)g * DK;
        CT* vr = vc + ((size_t)b * (size_t)max_len + (size_t)p) * (size_t)row + (size_t)g * DK;
        float y0 = sk[j][c], y1 = sk[j + HALF][c];
        if (cosT) pf_rope(sk[j][c], sk[j + HALF][c], cosT[(size_t)p * HALF + j], sinT[(size_t)p * HALF + j], y0, y1);
        kr[j] = (CT)y0;
        kr[j + HALF] = (CT)y1;
        vr[j] = (CT)sv[j][c];
        vr[j + HALF] = (CT)sv[j + HALF][c];
    }
}

// ------------------------------------------------------------------ causal attention

struct PrefillArgs
{
    const float* q;
    const void* kc;  // caches of CT elements
    const void* vc;
    const float* cosT;
    const float* sinT;
    float* out;
    int B, T, H, Hkv, R, pos0, max_len, nqb;
    float scale;
};

template <int DK>
struct PrefillTile
{
    static constexpr int KROW = DK + 4;  // padded K / V row (floats)
    static constexpr int kFloats = 2 * kPK * KROW;
    static constexpr int kBytes = 2 * kFloats * 4;  // double-buffered
};

template <int DK, typename CT>
__global__ __launch_bounds__(512) void k_attn_prefill(PrefillArgs a)
{
    constexpr int HALF = DK / 2;
    constexpr int NC = DK / 8;    // 16-byte chunks of a lane half's K row (S products in groups of 4)
    constexpr int ND = DK / 32;   // 32-row blocks of O^T
    constexpr int KROW = PrefillTile<DK>::KROW;
    constexpr int TILE = PrefillTile<DK>::kFloats;
    extern __shared__ __align__(16) float smem[];

    const int nthreads = a.R * 64;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, h = lane >> 5, l32 = lane & 31;
    // heaviest items first: query block from the last one down
    const int per_qb = a.B * a.Hkv;
    const int qb = a.nqb - 1 - (int)blockIdx.x / per_qb;
    const int bg = (int)blockIdx.x % per_qb;
    const int b = bg / a.Hkv, g = bg % a.Hkv;
    const int head = g * a.R + wave;
    const int M = a.B * a.T;
    const int t0 = qb * kPQ;
    const int qt = t0 + l32;                  // this lane's query token (valid if < T)
    const int qpos = a.pos0 + qt;             // its position
    const int row = a.Hkv * DK;
    const int valid = a.pos0 + a.T;           // cache rows [0, valid) hold keys / values

    // ---- the lane's rotated query values: qv[4c + e] = rot(q)[8c + 4h + e]
    float qv[DK / 2];
    {
        const __amdgpu_buffer_rsrc_t rq = pf_rsrc(a.q, (uint32_t)((size_t)a.H * DK * (size_t)M * 4u));
        const int m = b * a.T + qt;
        const bool qok = qt < a.T;
        float x[DK / 2];
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int e = 0; e < 4; ++e)
            {
                const int i = 8 * c + 4 * h + e;
                const uint32_t off = qok ? (uint32_t)(((size_t)(head * DK + i) * (size_t)M + (size_t)m) * 4u) : 0x80000000u;
                x[4 * c + e] = ld_f(rq, off);
            }
        if (a.cosT)
        {
            const __amdgpu_buffer_rsrc_t rc = pf_rsrc(a.cosT, (uint32_t)((size_t)a.max_len * HALF * 4u));
            const __amdgpu_buffer_rsrc_t rs = pf_rsrc(a.sinT, (uint32_t)((size_t)a.max_len * HALF * 4u));
            // dimension i < HALF pairs with i + HALF: chunk c pairs with c + NC/2 in the same lane
#pragma unroll
            for (int c = 0; c < NC / 2; ++c)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                {
                    const int j = 8 * c + 4 * h + e;
                    const uint32_t off = qok ? (uint32_t)(((size_t)qpos * HALF + (size_t)j) * 4u) : 0x80000000u;
                    const float cs = ld_f(rc, off), sn = ld_f(rs, off);
                    pf_rope(x[4 * c + e], x[4 * (c + NC / 2) + e], cs, sn, qv[4 * c + e], qv[4 * (c + NC / 2) + e]);
                }
        }
        else
        {
#pragma unroll
            for (int i = 0; i < DK / 2; ++i) qv[i] = x[i];
        }
    }

    // ---- key tiles: keys [0, last] with last = min(qpos of the block's last query, valid - 1)
    const int last_key = min(a.pos0 + min(t0 + kPQ, a.T) - 1, valid - 1);
    const int nkb = last_key / kPK + 1;
    const size_t seq_off = (size_t)b * (size_t)a.max_len * (size_t)row;
    // rows at or past `valid` (and past max_len) read as zeros: their scores are masked and their
    // zero values keep 0 * v finite
    const uint32_t seq_bytes = (uint32_t)((size_t)min(valid, a.max_len) * (size_t)row * sizeof(CT));
    const __amdgpu_buffer_rsrc_t rk = pf_rsrc(static_cast<const CT*>(a.kc) + seq_off, seq_bytes);
    const __amdgpu_buffer_rsrc_t rv = pf_rsrc(static_cast<const CT*>(a.vc) + seq_off, seq_bytes);

    // staging: float4 units of a 32 x DK tile, spread over the work-group's threads
    constexpr int kUnits = kPK * DK / 4;
    auto stage_tile = [&](int kb, float* tile) {
        float* ks = tile;
        float* vs = tile + kPK * KROW;
        for (int u = tid; u < kUnits; u += nthreads)
        {
            const int key = u / (DK / 4), c4 = u % (DK / 4);
            const uint32_t off =
                (uint32_t)(((size_t)(kb * kPK + key) * (size_t)row + (size_t)g * DK + 4 * c4) * sizeof(CT));
            const float4 kk = ld_c4<CT>(rk, off);
            const float4 vv = ld_c4<CT>(rv, off);
            *reinterpret_cast<float4*>(ks + key * KROW + 4 * c4) = kk;
            *reinterpret_cast<float4*>(vs + key * KROW + 4 * c4) = vv;
        }
    };

    v16f o[ND];
#pragma unroll
    for (int d = 0; d < ND; ++d) o[d] = v16f{};
    float m_run = -__builtin_inff(), l_run = 0.0f;

    stage_tile(0, smem);
    __syncthreads();
    for (int kb = 0; kb < nkb; ++kb)
    {
        const float* tile = smem + (kb & 1) * TILE;
        const float* ks = tile;
        const float* vs = tile + kPK * KROW;
        // S^T = K . Q^T over the head dimension
        v16f s = v16f{};
#pragma unroll
        for (int c = 0; c < NC; ++c)
        {
            const float4 kk = *reinterpret_cast<const float4*>(ks + l32 * KROW + 8 * c + 4 * h);
            s = __builtin_amdgcn_mfma_f32_32x32x2f32(kk.x, qv[4 * c + 0], s, 0, 0, 0);
            s = __builtin_amdgcn_mfma_f32_32x32x2f32(kk.y, qv[4 * c + 1], s, 0, 0, 0);
            s = __builtin_amdgcn_mfma_f32_32x32x2f32(kk.z, qv[4 * c + 2], s, 0, 0, 0);
            s = __builtin_amdgcn_mfma_f32_32x32x2f32(kk.w, qv[4 * c + 3], s, 0, 0, 0);
        }
        // the next tile's loads overlap this tile's softmax and products
        if (kb + 1 < nkb) stage_tile(kb + 1, smem + ((kb + 1) & 1) * TILE);
        // online softmax over this tile's keys (element v: key 32kb + 8(v/4) + 4h + v%4); the
        // causal mask only where the tile reaches past the wave's first query
        float sc[16];
        float mx = -__builtin_inff();
        if (kb * kPK + kPK - 1 <= a.pos0 + t0)
        {
#pragma unroll
            for (int v = 0; v < 16; ++v)
            {
                sc[v] = s[v] * a.scale;
                mx = fmaxf(mx, sc[v]);
            }
        }
        else
        {
#pragma unroll
            for (int v = 0; v < 16; ++v)
            {
                const int key = kb * kPK + 8 * (v >> 2) + 4 * h + (v & 3);
                const float x = s[v] * a.scale;
                sc[v] = key <= qpos ? x : -__builtin_inff();
                mx = fmaxf(mx, sc[v]);
            }
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_new = fmaxf(m_run, mx);
        const bool any = m_new != -__builtin_inff();
        const float corr = any ? expf(m_run - m_new) : 1.0f;
        float ls = 0.0f;
#pragma unroll
        for (int v = 0; v < 16; ++v)
        {
            sc[v] = any ? expf(sc[v] - m_new) : 0.0f;
            ls += sc[v];
        }
        ls += __shfl_xor(ls, 32);
        l_run = l_run * corr + ls;
        m_run = m_new;
        // corr is exactly 1 where the running maximum did not move: skip the rescale when that
        // holds for every lane (multiplying by 1 would change no bit)
        if (__builtin_amdgcn_ballot_w64(corr != 1.0f) != 0)
        {
#pragma unroll
            for (int d = 0; d < ND; ++d)
#pragma unroll
                for (int v = 0; v < 16; ++v) o[d][v] *= corr;
        }
        // O^T += V^T . P^T: product s takes key 8(s/4) + 4h + s%4 (the lane's score element s)
#pragma unroll
        for (int d = 0; d < ND; ++d)
#pragma unroll
            for (int sp = 0; sp < 16; ++sp)
            {
                const int key = 8 * (sp >> 2) + 4 * h + (sp & 3);
                o[d] = __builtin_amdgcn_mfma_f32_32x32x2f32(vs[key * KROW + 32 * d + l32], sc[sp], o[d], 0, 0, 0);
            }
        __syncthreads();  // every wave is done with this tile; the next one is in LDS
    }

    // ---- out[head*dk + i][m] = O^T[i][query] / l for the block's valid queries
    if (qt < a.T)
    {
        const int m = b * a.T + qt;
#pragma unroll
        for (int d = 0; d < ND; ++d)
#pragma unroll
            for (int v = 0; v < 16; ++v)
            {
                const int i = 32 * d + 8 * (v >> 2) + 4 * h + (v & 3);
                a.out[(size_t)(head * DK + i) * (size_t)M + (size_t)m] = o[d][v] / l_run;
            }
    }
}

template <int DK, typename CT>
hipError_t launch_prefill_dk(hipStream_t st, const PrefillArgs& a)
{
    static bool attr_set = false;
    if (!attr_set)
    {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_attn_prefill<DK, CT>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, PrefillTile<DK>::kBytes);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    const unsigned blocks = (unsigned)(a.nqb * a.B * a.Hkv);
    hipLaunchKernelGGL((k_attn_prefill<DK, CT>), dim3(blocks), dim3(a.R * 64), PrefillTile<DK>::kBytes, st, a);
    return hipGetLastError();
}

}  // namespace

bool prefill_dk_supported(size_t dk) { return dk == 64 || dk == 128; }

template <typename CT>
hipError_t launch_kv_fill_ct(hipStream_t st, const float* k, const float* v, size_t B, size_t T, size_t Hkv, size_t dk,
                             size_t pos0, const float* cosT, const float* sinT, CT* kc, CT* vc, size_t max_len)
{
    const dim3 grid((unsigned)ceil_div(B * T, kPQ), (unsigned)Hkv);
    if (dk == 64)
        hipLaunchKernelGGL((k_kv_fill<64, CT>), grid, dim3(256), 0, st, k, v, (int)B, (int)T, (int)Hkv, (int)pos0, cosT,
                           sinT, kc, vc, (int)max_len);
    else if (dk == 128)
        hipLaunchKernelGGL((k_kv_fill<128, CT>), grid, dim3(256), 0, st, k, v, (int)B, (int)T, (int)Hkv, (int)pos0, cosT,
                           sinT, kc, vc, (int)max_len);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_kv_fill(hipStream_t st, const float* k, const float* v, size_t B, size_t T, size_t Hkv, size_t dk,
                          size_t pos0, const float* cosT, const float* sinT, void* kc, void* vc, bool cache_f16,
                          size_t max_len)
{
    if (B * T == 0) return hipSuccess;
    if (cache_f16)
        return launch_kv_fill_ct(st, k, v, B, T, Hkv, dk, pos0, cosT, sinT, static_cast<_Float16*>(kc),
                                 static_cast<_Float16*>(vc), max_len);
    return launch_kv_fill_ct(st, k, v, B, T, Hkv, dk, pos0, cosT, sinT, static_cast<float*>(kc),
                             static_cast<float*>(vc), max_len);
}

hipError_t launch_attn_prefill(hipStream_t st, const float* q, const void* kc, const void* vc, bool cache_f16,
                               size_t B, size_t T, size_t H, size_t Hkv, size_t dk, size_t pos0, const float* cosT,
                               const float* sinT, size_t max_len, float scale, float* out)
{
    if (B * T == 0) return hipSuccess;
    PrefillArgs a{q, kc, vc, cosT, sinT, out, (int)B, (int)T, (int)H, (int)Hkv, (int)(H / Hkv), (int)pos0,
                  (int)max_len, (int)ceil_div(T, kPQ), scale};
    if (cache_f16)
    {
        if (dk == 64) return launch_prefill_dk<64, _Float16>(st, a);
        if (dk == 128) return launch_prefill_dk<128, _Float16>(st, a);
        return hipErrorInvalidValue;
    }
    if (dk == 64) return launch_prefill_dk<64, float>(st, a);
    if (dk == 128) return launch_prefill_dk<128, float>(st, a);
    return hipErrorInvalidValue;
}

}  // namespace nnhip
