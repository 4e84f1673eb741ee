// k_decode.hip — the kernels of a batched decode step around the BitLinear path: attention of
// one new token per sequence over its KV cache (grouped-query heads, RoPE, the cache append
// fused in), the token-embedding gather, the residual add and the greedy argmax.
//
// Reference: AttentionBase::forward_step (include/neuralnet.cpp/compute_layer_attention.hpp:
// 1003-1091) advances ONE sequence by one token: q/k/v projections, RoPE at position cur_len
// (compute_position_encoding.hpp:150-166), append to the (max_len, H*dk) caches, scores =
// (q . K^T) * scale per head, softmax, V^T . attn. Here B sequences advance one token each in
// one launch, each at its own position, and the caches keep the Hkv KV heads un-expanded
// (the reference's gather_rows expansion only duplicates rows: query head h reads KV head
// h / (H / Hkv), compute_layer_attention.hpp:444-449).
//
// Layouts (device, f32):
//   q      (H*dk, B)      feature-major, one column per sequence (the q projection's output)
//   k, v   (Hkv*dk, B)    the new token's key / value
//   caches (B, max_len, Hkv*dk)   row t of sequence b = the key (value) at position t
//   out    (H*dk, B)
//   pos    (B) int32      position of sequence b's new token (= its cache length before the call)
//   cos/sin (max_len, dk/2) RoPE tables (the reference's cat(freqs, freqs) halves, stored once)
//
// Work split (flash-decoding): work-group (chunk c, KV head g, sequence b) covers cache
// positions [128c, 128c + 128) for the R = H/Hkv query heads that share KV head g, so every
// key/value row is read from HBM once for all of them. The grid is persistent (as many
// work-groups as are resident at once, looping over the items). The scores of a chunk stay in
// LDS; the chunk writes (acc[R][dk], max, sum) to scratch and a second kernel merges the chunks
// of each (sequence, KV head). (Merging in the last chunk to finish, found with a counter, needs
// an agent-scope fence in every work-group; with one L2 per XCD that fence cost far more than the
// second launch.) With a single chunk (every sequence shorter than 129) the work-group writes the
// output itself.
// The work-group whose chunk holds position pos[b] writes the rotated key and the value into the
// cache and uses them from LDS; no other work-group reads that row in the same launch.
#include "common.hpp"

#include <cmath>

namespace nnhip
{
namespace
{

constexpr int kAttnT = 128;        // cache positions per work-group
constexpr int kAttnThreads = 256;  // 4 waves
#ifndef NNHIP_ATTN_MINW
#define NNHIP_ATTN_MINW 5          // waves per SIMD the chunk kernel is compiled for (<= 96 VGPRs)
#endif
#ifndef NNHIP_ATTN_MINW_H
#define NNHIP_ATTN_MINW_H 5        // over f16 caches. 6 (80 VGPRs, no spills) takes C5's 1360 items
                                   // in one round: the lone call 28.7-29.1 against 31.2-31.3 us, but
                                   // the decode step 2.045 against 2.031 ms (A/B, same ids)
#endif
#ifndef NNHIP_ATTN_PB
#define NNHIP_ATTN_PB 2            // score passes (32 positions each) whose loads are in flight together
                                   // (2: 136.0 us at 16 x 8192 positions, 4: 141.6; equal at 2112)
#endif
#ifndef NNHIP_ATTN_PB_H
#define NNHIP_ATTN_PB_H 4          // the same over f16 caches (rows held packed: every pass at once;
                                   // C5 30.9-31.3 us with the merge against 31.5-32.0 at 2 passes)
#endif
constexpr int kRecPad = 16;        // record tail: max[8], sum[8]

struct AttnArgs
{
    const float* q;
    const float* k;
    const float* v;
    const int32_t* pos;
    const float* cosT;
    const float* sinT;
    void* kc;  // caches of CT elements (float, or _Float16 under compute = F16)
    void* vc;
    float* part;
    float* out;
    int B, H, Hkv, R, max_len, len_bound, nchunk;
    float scale;
    int out_tm;  // out is token-major (B, H*dk) instead of (H*dk, B)
    int in_tm;   // q, k, v are token-major (B, H*dk), (B, Hkv*dk) instead of (H*dk, B), (Hkv*dk, B)
};

// Index of element i of head h, sequence b in the attention output
__device__ __forceinline__ size_t attn_out_at(const AttnArgs& a, int h, int DKv, int i, int b)
{
    return a.out_tm ? ((size_t)b * a.H + h) * DKv + i : (size_t)(h * DKv + i) * a.B + b;
}

__device__ __forceinline__ float sum8(float v)
{
    // sum over the 8 lanes {8i .. 8i+7}: quad permutes (xor 1, xor 2), then xor 4
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
    v += __shfl_xor(v, 4, kWave);
    return v;
}

// RoPE on one (x0, x1) = (q[j], q[j + dk/2]) pair, as the reference's
// q*cos + rotate_half(q)*sin with rotate_half(q)[j] = -q[j + dk/2], [j + dk/2] = q[j]:
// two rounded products and a rounded sum per output (no fused multiply-add).
__device__ __forceinline__ void rope_pair(float x0, float x1, float cs, float sn, float& y0, float& y1)
{
    y0 = __fadd_rn(__fmul_rn(x0, cs), __fmul_rn(-x1, sn));
    y1 = __fadd_rn(__fmul_rn(x1, cs), __fmul_rn(x0, sn));
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t attn_rsrc(const void* base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// 16 bytes at byte offset voff + soff of the resource (0 when out of range). The cached keys and
// values are read once per call: non-temporal loads ("nt" on gfx950) keep them from displacing
// the rest of L2.
#ifndef NNHIP_ATTN_LOAD_AUX
#define NNHIP_ATTN_LOAD_AUX 2
#endif
__device__ __forceinline__ float4 ld_f4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff)
{
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, voff + soff, 0, NNHIP_ATTN_LOAD_AUX));
}

// x as the cache stores it: itself in an f32 cache, the nearest f16 (ties to even) in an f16 one
template <typename CT>
__device__ __forceinline__ float cache_round(float x)
{
    if constexpr (sizeof(CT) == 4) return x;
    else return (float)(_Float16)x;
}

// Four cache elements as they are held between their load and their use: a float4 from an f32
// cache, or the four halves of an f16 one packed in two registers (half the registers, so twice
// the rows can be in flight), widened by widen4 where they are used.
template <typename CT>
struct CacheQuad
{
    using type = float4;
};
template <>
struct CacheQuad<_Float16>
{
    typedef uint32_t type __attribute__((ext_vector_type(2)));
};

template <typename CT>
__device__ __forceinline__ typename CacheQuad<CT>::type ld_q4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff)
{
    if constexpr (sizeof(CT) == 4) return ld_f4(r, voff, soff);
    else
        return __builtin_bit_cast(typename CacheQuad<CT>::type,
                                  __builtin_amdgcn_raw_buffer_load_b64(r, voff + soff, 0, NNHIP_ATTN_LOAD_AUX));
}

template <typename CT>
__device__ __forceinline__ float4 widen4(typename CacheQuad<CT>::type v)
{
    if constexpr (sizeof(CT) == 4) return v;
    else
    {
        typedef _Float16 h4 __attribute__((ext_vector_type(4)));
        const h4 h = __builtin_bit_cast(h4, v);
        return make_float4((float)h[0], (float)h[1], (float)h[2], (float)h[3]);
    }
}

// 4 bytes at byte offset off of the resource (0 when out of range), default cache policy
__device__ __forceinline__ float ld_f1(__amdgpu_buffer_rsrc_t r, uint32_t off)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}

// Workgroup barrier for LDS data only: waits for this wave's LDS operations (lgkmcnt(0); the
// gfx950 s_barrier does not wait for them by itself), then s_barrier. There is no vmcnt wait, so
// global loads in flight stay in flight. The empty asm statements keep the compiler from moving
// memory accesses across it.
__device__ __forceinline__ void lds_only_barrier()
{
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // vmcnt and expcnt at their maxima, lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

template <int DK, int RT, bool kFinal, typename CT>
__global__ __launch_bounds__(kAttnThreads, (DK <= 128 && RT <= 4) ? (sizeof(CT) == 2 ? NNHIP_ATTN_MINW_H : NNHIP_ATTN_MINW) : 1) void k_attn_chunk(AttnArgs a)
{
    constexpr int HALF = DK / 2;
    constexpr int Q4 = DK / 4;         // float4 per row
    constexpr int F4 = DK / 32;        // float4 per lane in the score phase (8 lanes per position)
    constexpr bool kH = sizeof(CT) == 2;  // f16 cache rows, held packed until use
    constexpr int PB = DK <= 128 ? (kH ? NNHIP_ATTN_PB_H : NNHIP_ATTN_PB) : 2;  // passes whose loads go together
    using Quad = typename CacheQuad<CT>::type;
    constexpr int VL = DK / 4;         // lanes per row in the value phase
    constexpr int NG = kAttnThreads / VL;  // rows per value step
    constexpr int QI = (RT * HALF + kAttnThreads - 1) / kAttnThreads;  // query pairs per thread
    static_assert(DK <= kAttnThreads, "one thread per element of the new key / value");
    __shared__ float4 q_s[RT * Q4];
    __shared__ float4 kn_s[Q4], vn_s[Q4];
    __shared__ float S[RT][kAttnT];
    __shared__ float ml[2][RT];
    __shared__ float4 red[4][RT * Q4];

    const int tid0 = threadIdx.x;
    const int R = a.R;  // query heads per KV head (<= RT, the register / LDS sizing)
    const int total = a.nchunk * a.Hkv * a.B;
    // persistent: work-group items. The chunks before each (sequence, KV head)'s last come first
    // (chunk fastest, then KV head, then sequence), then the last chunks: those are partial
    // (positions past the last multiple of 128), so when the items outnumber the resident
    // work-groups by a little, the second round is made of short items.
    const int nfull = (a.nchunk - 1) * a.Hkv * a.B;
    for (int item = blockIdx.x; item < total; item += gridDim.x)
    {
        int tid = tid0;
        // opaque per item: the compiler keeps no thread-index arithmetic live across items (hoisted
        // out of the loop, those values took ~28 VGPRs and pushed the kernel into spills)
        asm volatile("" : "+v"(tid));
        const int w = tid >> 6, lane = tid & 63;
        int c, pr;
        if (item < nfull)
        {
            c = item % (a.nchunk - 1);
            pr = item / (a.nchunk - 1);
        }
        else
        {
            c = a.nchunk - 1;
            pr = item - nfull;
        }
        const int g = pr % a.Hkv;
        const int b = pr / a.Hkv;
        const int p = a.pos[b];
        const int t0 = c * kAttnT;
        if (p < 0 || p >= a.len_bound)
        {
            // out-of-range position: NaN output for this sequence's heads, cache untouched
            if (c == 0)
                for (int e = tid; e < R * DK; e += kAttnThreads)
                    a.out[attn_out_at(a, g * R + e / DK, DK, e % DK, b)] = __builtin_nanf("");
            continue;
        }
        const int len = p + 1;
        if (t0 >= len) continue;
        const int n = min(kAttnT, len - t0);
        const bool has_new = p < t0 + kAttnT;
        const size_t rstride = (size_t)a.Hkv * DK;
        const size_t seq_off = (size_t)b * a.max_len * rstride + (size_t)g * DK;

        // ---- loads first, in this order: the query pairs (and, in the chunk holding p, the new
        //      key/value), then the first PB passes of cached key rows. The queries' RoPE and
        //      LDS staging wait only for the query loads, so the key rows stream in meanwhile.
        // (buffer-resource loads: 32-bit offsets keep the address registers few)
        // bytes between features of one token: 4 in token-major rows, B * 4 down a column
        const uint32_t qkv_rows = a.in_tm ? 4u : (uint32_t)a.B * 4u;
        const __amdgpu_buffer_rsrc_t rq =
            attn_rsrc(a.in_tm ? a.q + (size_t)b * a.H * DK : a.q + b, (uint32_t)a.H * DK * qkv_rows);
        const __amdgpu_buffer_rsrc_t rkn =
            attn_rsrc(a.in_tm ? a.k + (size_t)b * a.Hkv * DK : a.k + b, (uint32_t)a.Hkv * DK * qkv_rows);
        const __amdgpu_buffer_rsrc_t rvn =
            attn_rsrc(a.in_tm ? a.v + (size_t)b * a.Hkv * DK : a.v + b, (uint32_t)a.Hkv * DK * qkv_rows);
        // the RoPE table rows of position p (unused without tables)
        const __amdgpu_buffer_rsrc_t rcs = attn_rsrc(a.cosT ? a.cosT + (size_t)p * HALF : a.q, HALF * 4u);
        const __amdgpu_buffer_rsrc_t rsn = attn_rsrc(a.sinT ? a.sinT + (size_t)p * HALF : a.q, HALF * 4u);
        float qx0[QI], qx1[QI], qcs[QI], qsn[QI];
#pragma unroll
        for (int u = 0; u < QI; ++u)
        {
            const int e = tid + u * kAttnThreads;
            const int r = e / HALF, j = e - r * HALF;
            // lanes past R heads read zeros (offset beyond the resource)
            const uint32_t qo = e < R * HALF ? (uint32_t)((g * R + r) * DK + j) * qkv_rows : 0x80000000u;
            qx0[u] = ld_f1(rq, qo);
            qx1[u] = ld_f1(rq, qo + HALF * qkv_rows);
            qcs[u] = a.cosT ? ld_f1(rcs, 4u * j) : 1.f;
            qsn[u] = a.cosT ? ld_f1(rsn, 4u * j) : 0.f;
        }
        float kx0 = 0.f, kx1 = 0.f, kcs = 1.f, ksn = 0.f, vx = 0.f;
        if (has_new)
        {
            const uint32_t ko = tid < HALF ? (uint32_t)(g * DK + tid) * qkv_rows : 0x80000000u;
            kx0 = ld_f1(rkn, ko);
            kx1 = ld_f1(rkn, ko + HALF * qkv_rows);
            if (a.cosT)
            {
                kcs = ld_f1(rcs, 4u * (tid & (HALF - 1)));
                ksn = ld_f1(rsn, 4u * (tid & (HALF - 1)));
            }
            vx = ld_f1(rvn, tid < DK ? (uint32_t)(g * DK + tid) * qkv_rows : 0x80000000u);
        }

        // key rows: 8 lanes per position, lane j8 holds float4 columns j8 + 8i of the row.
        // Cached rows come through one buffer resource per (sequence, KV head): lanes past the
        // chunk or on the new position read zeros without a branch, so every load of a pass
        // group is in flight at once; the new position's key is selected from LDS afterwards.
        const int pg = tid >> 3, j8 = tid & 7;
        constexpr uint32_t ES = sizeof(CT);  // bytes per cache element
        const __amdgpu_buffer_rsrc_t rk =
            attn_rsrc(static_cast<const CT*>(a.kc) + seq_off, (uint32_t)((size_t)a.max_len * rstride * ES));
        Quad kv[PB][F4];
        auto load_keys = [&](int pass0) {
#pragma unroll
            for (int u = 0; u < PB; ++u)
            {
                const int tl = (pass0 + u) * 32 + pg;
                const int t = t0 + tl;
                const uint32_t row = (tl < n && t < p) ? (uint32_t)t * (uint32_t)rstride * ES : 0x80000000u;
#pragma unroll
                for (int i = 0; i < F4; ++i) kv[u][i] = ld_q4<CT>(rk, row, 4u * ES * (j8 + 8 * i));
            }
        };
        load_keys(0);

        // value-row geometry: VL lanes per row (one quad each), NG rows per step, VR rows per thread
        constexpr int VR = kAttnT / NG;
        const int vg = tid / VL, vi = tid % VL;
        Quad vv[VR];
        const __amdgpu_buffer_rsrc_t rv =
            attn_rsrc(static_cast<const CT*>(a.vc) + seq_off, (uint32_t)((size_t)a.max_len * rstride * ES));
        auto load_values = [&]() {
#pragma unroll
            for (int u = 0; u < VR; ++u)
            {
                const int tl = vg + u * NG;
                const int t = t0 + tl;
                const uint32_t row = (tl < n && t < p) ? (uint32_t)t * (uint32_t)rstride * ES : 0x80000000u;
                vv[u] = ld_q4<CT>(rv, row, 4u * ES * vi);
            }
        };

        // ---- stage the rotated queries (R heads) and, in the chunk holding p, the new key/value
        float* qf = reinterpret_cast<float*>(q_s);
#pragma unroll
        for (int u = 0; u < QI; ++u)
        {
            const int e = tid + u * kAttnThreads;
            if (e < R * HALF)
            {
                const int r = e / HALF, j = e - r * HALF;
                float y0 = qx0[u], y1 = qx1[u];
                if (a.cosT) rope_pair(qx0[u], qx1[u], qcs[u], qsn[u], y0, y1);
                qf[r * DK + j] = y0;
                qf[r * DK + j + HALF] = y1;
            }
        }
        if (has_new)
        {
            float* kf = reinterpret_cast<float*>(kn_s);
            float* vf = reinterpret_cast<float*>(vn_s);
            if (tid < HALF)
            {
                float y0 = kx0, y1 = kx1;
                if (a.cosT) rope_pair(kx0, kx1, kcs, ksn, y0, y1);
                kf[tid] = cache_round<CT>(y0);
                kf[tid + HALF] = cache_round<CT>(y1);
            }
            if (tid < DK) vf[tid] = cache_round<CT>(vx);
        }
        // LDS-only barrier: a workgroup fence (__syncthreads) would also wait for the key loads
        lds_only_barrier();
        if (has_new)
        {
            CT* krow = static_cast<CT*>(a.kc) + seq_off + (size_t)p * rstride;
            CT* vrow = static_cast<CT*>(a.vc) + seq_off + (size_t)p * rstride;
            for (int i = tid; i < Q4; i += kAttnThreads)
            {
                if constexpr (sizeof(CT) == 4)
                {
                    reinterpret_cast<float4*>(krow)[i] = kn_s[i];
                    reinterpret_cast<float4*>(vrow)[i] = vn_s[i];
                }
                else
                {
                    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
                    const float4 kq = kn_s[i], vq = vn_s[i];
                    reinterpret_cast<h4*>(krow)[i] = h4{(_Float16)kq.x, (_Float16)kq.y, (_Float16)kq.z, (_Float16)kq.w};
                    reinterpret_cast<h4*>(vrow)[i] = h4{(_Float16)vq.x, (_Float16)vq.y, (_Float16)vq.z, (_Float16)vq.w};
                }
            }
        }

        // ---- scores of the chunk, PB passes of 32 positions at a time
#pragma unroll
        for (int pass0 = 0; pass0 < kAttnT / 32; pass0 += PB)
        {
            if (pass0 > 0) load_keys(pass0);
#pragma unroll
            for (int u = 0; u < PB; ++u)
            {
                const int tl = (pass0 + u) * 32 + pg;
                // the row widened; the new position's key comes from LDS (in place over f32)
                float4 kk[F4];
                if constexpr (kH)
                {
#pragma unroll
                    for (int i = 0; i < F4; ++i) kk[i] = widen4<CT>(kv[u][i]);
                    if (t0 + tl == p)
                    {
#pragma unroll
                        for (int i = 0; i < F4; ++i) kk[i] = kn_s[j8 + 8 * i];
                    }
                }
                else
                {
                    if (t0 + tl == p)
                    {
#pragma unroll
                        for (int i = 0; i < F4; ++i) kv[u][i] = kn_s[j8 + 8 * i];
                    }
#pragma unroll
                    for (int i = 0; i < F4; ++i) kk[i] = kv[u][i];
                }
                float d[RT];
#pragma unroll
                for (int r = 0; r < RT; ++r)
                {
                    d[r] = 0.f;
                    if (r < R)
                    {
#pragma unroll
                        for (int i = 0; i < F4; ++i)
                        {
                            const float4 qq = q_s[r * Q4 + j8 + 8 * i];
                            d[r] = __builtin_fmaf(kk[i].x, qq.x, d[r]);
                            d[r] = __builtin_fmaf(kk[i].y, qq.y, d[r]);
                            d[r] = __builtin_fmaf(kk[i].z, qq.z, d[r]);
                            d[r] = __builtin_fmaf(kk[i].w, qq.w, d[r]);
                        }
                        d[r] = sum8(d[r]);
                    }
                }
                if (tl < n)
                {
#pragma unroll
                    for (int r = 0; r < RT; ++r)
                        if (r < R && j8 == r) S[r][tl] = __fmul_rn(d[r], a.scale);
                }
            }
        }
        __syncthreads();

        // ---- value rows of the whole chunk: issued before the softmax so its latency hides
        //      behind them (with the first key rows instead, over f16 caches: 8 VGPRs of spills
        //      at 96, 38.7 against 31.1 us)
        load_values();

        // ---- chunk softmax statistics: one wave per head
        for (int r = w; r < R; r += 4)
        {
            float m = -__builtin_inff();
            for (int i = lane; i < n; i += kWave) m = fmaxf(m, S[r][i]);
            for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, kWave));
            float l = 0.f;
            for (int i = lane; i < n; i += kWave)
            {
                const float e = expf(S[r][i] - m);
                S[r][i] = e;
                l += e;
            }
            for (int off = 32; off >= 1; off >>= 1) l += __shfl_xor(l, off, kWave);
            if (lane == 0)
            {
                ml[0][r] = m;
                ml[1][r] = l;
            }
        }
        __syncthreads();

        // ---- weighted values (the new position's value from LDS)
        if constexpr (!kH)
        {
#pragma unroll
            for (int u = 0; u < VR; ++u)
                if (t0 + vg + u * NG == p) vv[u] = vn_s[vi];
        }
        float4 acc[RT];
#pragma unroll
        for (int r = 0; r < RT; ++r) acc[r] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int u = 0; u < VR; ++u)
        {
            const int tl = vg + u * NG;
            if (tl < n)
            {
                float4 vf = widen4<CT>(vv[u]);
                if constexpr (kH)
                    if (t0 + tl == p) vf = vn_s[vi];
#pragma unroll
                for (int r = 0; r < RT; ++r)
                    if (r < R)
                    {
                        const float pr = S[r][tl];
                        acc[r].x = __builtin_fmaf(pr, vf.x, acc[r].x);
                        acc[r].y = __builtin_fmaf(pr, vf.y, acc[r].y);
                        acc[r].z = __builtin_fmaf(pr, vf.z, acc[r].z);
                        acc[r].w = __builtin_fmaf(pr, vf.w, acc[r].w);
                    }
            }
        }
        // rows of one wave -> lanes [0, VL), then the 4 waves through LDS in a fixed order
#pragma unroll
        for (int r = 0; r < RT; ++r)
            if (r < R)
                for (int off = VL; off < kWave; off <<= 1)
                {
                    acc[r].x += __shfl_xor(acc[r].x, off, kWave);
                    acc[r].y += __shfl_xor(acc[r].y, off, kWave);
                    acc[r].z += __shfl_xor(acc[r].z, off, kWave);
                    acc[r].w += __shfl_xor(acc[r].w, off, kWave);
                }
        if (lane < VL)
        {
#pragma unroll
            for (int r = 0; r < RT; ++r)
                if (r < R) red[w][r * Q4 + vi] = acc[r];
        }
        __syncthreads();
        const size_t stride = (size_t)(R * DK + kRecPad);
        float* rec0 = a.part + (size_t)(b * a.Hkv + g) * a.nchunk * stride;
        float* rec = rec0 + (size_t)c * stride;
        for (int e = tid; e < R * Q4; e += kAttnThreads)
        {
            float4 s4 = red[0][e];
#pragma unroll
            for (int ww = 1; ww < 4; ++ww)
            {
                s4.x += red[ww][e].x;
                s4.y += red[ww][e].y;
                s4.z += red[ww][e].z;
                s4.w += red[ww][e].w;
            }
            if constexpr (kFinal)
            {
                const int r = e / Q4, i = 4 * (e - r * Q4);
                const float l = ml[1][r];
                const size_t st = a.out_tm ? 1 : (size_t)a.B;
                float* o = a.out + attn_out_at(a, g * R + r, DK, i, b);
                o[0] = s4.x / l;
                o[st] = s4.y / l;
                o[2 * st] = s4.z / l;
                o[3 * st] = s4.w / l;
            }
            else
            {
                reinterpret_cast<float4*>(rec)[e] = s4;
            }
        }
        if constexpr (!kFinal)
        {
            if (tid < R)
            {
                rec[R * DK + tid] = ml[0][tid];
                rec[R * DK + 8 + tid] = ml[1][tid];
            }
        }
        __syncthreads();  // LDS is reused by the next item
    }
}

// Merge of the chunk records (acc[R][DK], then max[8], sum[8]) of one (sequence, head):
// out = sum_c e_c acc_c / sum_c e_c l_c, e_c = exp(max_c - max), in ascending batches of 16
// chunks whose loads are all issued before use (an online maximum rescales earlier batches).
constexpr int kMergeBatch = 16;

template <int DK>
__global__ __launch_bounds__(DK) void k_attn_merge(AttnArgs a)
{
    const int b = blockIdx.x / a.H, h = blockIdx.x % a.H;
    const int g = h / a.R, r = h % a.R;
    const int i = threadIdx.x;
    const int p = a.pos[b];
    if (p < 0 || p >= a.len_bound) return;  // the chunk kernel wrote NaN
    const int nch = (p + kAttnT) / kAttnT;
    const size_t stride = (size_t)(a.R * DK + kRecPad);
    const float* rec0 = a.part + (size_t)(b * a.Hkv + g) * a.nchunk * stride;
    float M = -__builtin_inff(), num = 0.f, den = 0.f;
    // the loads of two batches are issued together (one round trip for up to 32 chunks); the
    // arithmetic stays per batch of kMergeBatch
    for (int c00 = 0; c00 < nch; c00 += 2 * kMergeBatch)
    {
        float mv[2][kMergeBatch], lv[2][kMergeBatch], av[2][kMergeBatch];
#pragma unroll
        for (int hb = 0; hb < 2; ++hb)
#pragma unroll
            for (int j = 0; j < kMergeBatch; ++j)
            {
                const int c = c00 + hb * kMergeBatch + j;
                const bool ok = c < nch;
                const float* rc = rec0 + (size_t)(ok ? c : c00) * stride;
                mv[hb][j] = ok ? rc[a.R * DK + r] : -__builtin_inff();
                lv[hb][j] = ok ? rc[a.R * DK + 8 + r] : 0.f;
                av[hb][j] = ok ? rc[r * DK + i] : 0.f;
            }
#pragma unroll
        for (int hb = 0; hb < 2; ++hb)
        {
            const int c0 = c00 + hb * kMergeBatch;
            if (c0 >= nch) break;
            float Mb = M;
#pragma unroll
            for (int j = 0; j < kMergeBatch; ++j) Mb = fmaxf(Mb, mv[hb][j]);
            const float resc = expf(M - Mb);  // 0 on the first batch (M = -inf)
            num = c0 == 0 ? 0.f : num * resc;
            den = c0 == 0 ? 0.f : den * resc;
#pragma unroll
            for (int j = 0; j < kMergeBatch; ++j)
            {
                const float e = c0 + j < nch ? expf(mv[hb][j] - Mb) : 0.f;
                num = __builtin_fmaf(e, av[hb][j], num);
                den = __builtin_fmaf(e, lv[hb][j], den);
            }
            M = Mb;
        }
    }
    a.out[attn_out_at(a, h, DK, i, b)] = num / den;
}

// Persistent grid: as many work-groups as fit the device at once (at most one per item).
template <int DK, int RT, bool kFinal, typename CT>
hipError_t launch_attn_variant(hipStream_t st, const AttnArgs& a, int num_cus)
{
    static int per_cu = 0;
    if (per_cu == 0)
    {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k_attn_chunk<DK, RT, kFinal, CT>, kAttnThreads, 0) !=
                hipSuccess ||
            n < 1)
            n = 1;
        per_cu = n;
    }
    const long total = (long)a.nchunk * a.Hkv * a.B;
    const long cap = (long)per_cu * (num_cus > 0 ? num_cus : 256);
    const unsigned grid = (unsigned)(total < cap ? total : cap);
    k_attn_chunk<DK, RT, kFinal, CT><<<dim3(grid), kAttnThreads, 0, st>>>(a);
    return hipGetLastError();
}

// query heads per KV head: 1, 2, 4 or 8 at compile time (3, 5, 6, 7 run as the next power of two
// with the extra heads masked)
template <int DK, bool kFinal, typename CT>
hipError_t launch_attn_r(hipStream_t st, const AttnArgs& a, int num_cus)
{
    if (a.R == 1) return launch_attn_variant<DK, 1, kFinal, CT>(st, a, num_cus);
    if (a.R == 2) return launch_attn_variant<DK, 2, kFinal, CT>(st, a, num_cus);
    if (a.R <= 4) return launch_attn_variant<DK, 4, kFinal, CT>(st, a, num_cus);
    return launch_attn_variant<DK, 8, kFinal, CT>(st, a, num_cus);
}

template <int DK, typename CT>
hipError_t launch_attn_dk(hipStream_t st, const AttnArgs& a, int num_cus)
{
    if (a.nchunk == 1) return launch_attn_r<DK, true, CT>(st, a, num_cus);
    const hipError_t e = launch_attn_r<DK, false, CT>(st, a, num_cus);
    if (e != hipSuccess) return e;
    k_attn_merge<DK><<<dim3(a.B * a.H), DK, 0, st>>>(a);
    return hipGetLastError();
}

// ---- small kernels of the decode step

constexpr int kSmallBlock = 256;

__global__ __launch_bounds__(kSmallBlock) void k_add(const float* __restrict__ x, const float* __restrict__ y,
                                                     size_t n, float* out)
{
    const size_t i = (size_t)blockIdx.x * kSmallBlock + threadIdx.x;
    if (i < n) out[i] = __fadd_rn(x[i], y[i]);
}

// dst (rows, n): column j = column col0 + j * stride of src (rows, src_cols)
__global__ __launch_bounds__(kSmallBlock) void k_copy_cols(const float* __restrict__ src, size_t rows, size_t src_cols,
                                                           size_t col0, size_t stride, size_t n, float* __restrict__ dst)
{
    const size_t i = (size_t)blockIdx.x * kSmallBlock + threadIdx.x;
    if (i >= rows * n) return;
    const size_t r = i / n, j = i % n;
    dst[i] = src[r * src_cols + col0 + j * stride];
}

// out (d, B), or token-major (B, d) when tm: column (row) b = row ids[b] of the (V, d) table
// (NaN for an id outside [0, V))
__global__ __launch_bounds__(kSmallBlock) void k_embed(const float* __restrict__ table, const int32_t* __restrict__ ids,
                                                       int V, int d, int B, int tm, float* __restrict__ out)
{
    const int b = blockIdx.y;
    const int i = blockIdx.x * kSmallBlock + threadIdx.x;
    if (i >= d) return;
    const int id = ids[b];
    out[tm ? (size_t)b * d + i : (size_t)i * B + b] = (id >= 0 && id < V) ? table[(size_t)id * d + i] : __builtin_nanf("");
}

// ids[b] = the reference greedy rule over column b of logits (V, B): best = l[0], then every
// l[v] > best replaces it (first index of the largest value; NaN entries never win, a NaN at
// v = 0 keeps index 0).
constexpr int kArgThreads = 1024;
constexpr int kArgBatch = 16;  // loads in flight per thread (V <= 16384 in one batch)

// kRows: logits are token-major (B, V), row b contiguous; otherwise column b of (V, B). pos, when
// given, is advanced by one for every sequence after its choice (the next decode position).
template <bool kRows>
__global__ __launch_bounds__(kArgThreads) void k_argmax(const float* __restrict__ L, int V, int B, int32_t* ids,
                                                        int32_t* pos)
{
    __shared__ float sv[kArgThreads / kWave];
    __shared__ int si[kArgThreads / kWave];
    const int b = blockIdx.x, tid = threadIdx.x;
    float bv = -__builtin_inff();
    int bi = -1;
    // each thread scans v = tid + kArgThreads j in ascending order (strict > keeps the first of
    // equal values; NaN never wins), a batch of loads at a time
    for (int v0 = tid; v0 < V; v0 += kArgThreads * kArgBatch)
    {
        float x[kArgBatch];
#pragma unroll
        for (int u = 0; u < kArgBatch; ++u)
        {
            const int v = v0 + u * kArgThreads;
            x[u] = v < V ? L[kRows ? (size_t)b * V + v : (size_t)v * B + b] : __builtin_nanf("");
        }
#pragma unroll
        for (int u = 0; u < kArgBatch; ++u)
            if (x[u] == x[u] && (bi < 0 || x[u] > bv))
            {
                bv = x[u];
                bi = v0 + u * kArgThreads;
            }
    }
    for (int off = 32; off >= 1; off >>= 1)
    {
        const float ov = __shfl_xor(bv, off, kWave);
        const int oi = __shfl_xor(bi, off, kWave);
        if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi < bi)))
        {
            bv = ov;
            bi = oi;
        }
    }
    if ((tid & 63) == 0)
    {
        sv[tid >> 6] = bv;
        si[tid >> 6] = bi;
    }
    __syncthreads();
    if (tid == 0)
    {
        for (int w = 1; w < kArgThreads / kWave; ++w)
            if (si[w] >= 0 && (bi < 0 || sv[w] > bv || (sv[w] == bv && si[w] < bi)))
            {
                bv = sv[w];
                bi = si[w];
            }
        // the reference's loop starts from l[0]: a NaN there is never replaced
        const float l0 = L[kRows ? (size_t)b * V : (size_t)b];
        ids[b] = (l0 != l0 || bi < 0) ? 0 : bi;
        if (pos) pos[b] = pos[b] + 1;
    }
}

}  // namespace

size_t attn_chunks(size_t len_bound) { return ceil_div(len_bound, kAttnT); }

size_t attn_workspace_bytes(size_t B, size_t H, size_t Hkv, size_t dk, size_t len_bound)
{
    if (attn_chunks(len_bound) <= 1) return 0;
    return B * Hkv * attn_chunks(len_bound) * ((H / Hkv) * dk + kRecPad) * sizeof(float);
}

hipError_t launch_attn_decode(hipStream_t st, const float* q, const float* k, const float* v, size_t B, size_t H,
                              size_t Hkv, size_t dk, const int32_t* pos, size_t len_bound, const float* cosT,
                              const float* sinT, void* kc, void* vc, bool cache_f16, size_t max_len, float scale,
                              float* part, float* out, int num_cus, bool out_tm)
{
    AttnArgs a{q, k, v, pos, cosT, sinT, kc, vc, part, out, (int)B, (int)H, (int)Hkv, (int)(H / Hkv),
               (int)max_len, (int)len_bound, (int)attn_chunks(len_bound), scale, out_tm ? 1 : 0, out_tm ? 1 : 0};
    if (cache_f16)
    {
        switch (dk)
        {
        case 64: return launch_attn_dk<64, _Float16>(st, a, num_cus);
        case 128: return launch_attn_dk<128, _Float16>(st, a, num_cus);
        case 256: return launch_attn_dk<256, _Float16>(st, a, num_cus);
        default: return hipErrorInvalidValue;
        }
    }
    switch (dk)
    {
    case 64: return launch_attn_dk<64, float>(st, a, num_cus);
    case 128: return launch_attn_dk<128, float>(st, a, num_cus);
    case 256: return launch_attn_dk<256, float>(st, a, num_cus);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_add(hipStream_t st, const float* x, const float* y, size_t n, float* out)
{
    k_add<<<dim3((unsigned)ceil_div(n, kSmallBlock)), kSmallBlock, 0, st>>>(x, y, n, out);
    return hipGetLastError();
}

hipError_t launch_copy_cols(hipStream_t st, const float* src, size_t rows, size_t src_cols, size_t col0, size_t stride,
                            size_t n, float* dst)
{
    if (rows * n == 0) return hipSuccess;
    k_copy_cols<<<dim3((unsigned)ceil_div(rows * n, kSmallBlock)), kSmallBlock, 0, st>>>(src, rows, src_cols, col0,
                                                                                       stride, n, dst);
    return hipGetLastError();
}

hipError_t launch_embed(hipStream_t st, const float* table, const int32_t* ids, size_t V, size_t d, size_t B, bool tm,
                        float* out)
{
    k_embed<<<dim3((unsigned)ceil_div(d, kSmallBlock), (unsigned)B), kSmallBlock, 0, st>>>(table, ids, (int)V, (int)d,
                                                                                         (int)B, tm ? 1 : 0, out);
    return hipGetLastError();
}

hipError_t launch_argmax(hipStream_t st, const float* L, size_t V, size_t B, int32_t* ids, bool rows, int32_t* pos)
{
    if (rows)
        k_argmax<true><<<dim3((unsigned)B), kArgThreads, 0, st>>>(L, (int)V, (int)B, ids, pos);
    else
        k_argmax<false><<<dim3((unsigned)B), kArgThreads, 0, st>>>(L, (int)V, (int)B, ids, pos);
    return hipGetLastError();
}

}  // namespace nnhip
