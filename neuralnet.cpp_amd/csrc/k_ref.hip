// k_ref.hip — kernels for the reference-layout primitives of nn::ComputeEngine
// (trit_pack, absmean tau, col_reduce_max, abs, scale_inplace, quantize_i8, unpack_i8,
// bias add). These are O(N*K) or O(K*M) elementwise/reduction passes: HBM-bound, one
// coalesced pass each. Every fp32 multiply/add that the reference rounds separately is
// written with __fmul_rn/__fadd_rn so the compiler cannot contract it into an FMA.
#include "common.hpp"

#include <cmath>

namespace nnhip
{
namespace
{

constexpr int kBlock = 256;

inline unsigned grid_for(size_t n, int per_block = kBlock)
{
    size_t g = ceil_div(n, (size_t)per_block);
    if (g < 1) g = 1;
    if (g > (1u << 20)) g = 1u << 20;  // grid-stride loops cover the rest
    return (unsigned)g;
}

// f32 -> IEEE binary16, round to nearest even (overflow -> inf, NaN stays NaN), and back (exact)
__global__ void k_f32_to_f16(const float* __restrict__ src, size_t n, uint16_t* __restrict__ dst)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        dst[i] = __builtin_bit_cast(uint16_t, (_Float16)src[i]);
}

__global__ void k_f16_to_f32(const uint16_t* __restrict__ src, size_t n, float* __restrict__ dst)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        dst[i] = (float)__builtin_bit_cast(_Float16, src[i]);
}

__global__ void k_fill_u32(uint32_t* __restrict__ dst, uint32_t value, size_t words)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < words;
         i += (size_t)gridDim.x * blockDim.x)
        dst[i] = value;
}

// One wave per row: lane l sums fl(|w| * fl(1/K)) for k = l, l+64, ... in ascending order,
// then a xor butterfly over 32,16,8,4,2,1 (commutative pairs, so every lane ends with the
// same value). Matches orc_row_absmean bit for bit.
__global__ __launch_bounds__(kBlock) void k_row_absmean(const float* __restrict__ W, size_t N,
                                                        size_t K, float inv_k, float* __restrict__ tau)
{
    const int lane = threadIdx.x & 63;
    const size_t row = (size_t)blockIdx.x * (kBlock / kWave) + (threadIdx.x >> 6);
    if (row >= N) return;
    const float* w = W + row * K;
    float acc = 0.0f;
    for (size_t k = (size_t)lane; k < K; k += kWave)
        acc = __fadd_rn(acc, __fmul_rn(fabsf(w[k]), inv_k));
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) acc = __fadd_rn(acc, __shfl_xor(acc, off, kWave));
    if (lane == 0) tau[row] = acc;
}

// One thread per output word: 16 weights -> 16 two-bit codes, LSB first.
__global__ __launch_bounds__(kBlock) void k_trit_pack(const float* __restrict__ W,
                                                      const float* __restrict__ tau, size_t N,
                                                      size_t K, size_t wpr, bool vec4,
                                                      uint32_t* __restrict__ wq)
{
    const size_t total = N * wpr;
    for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (size_t)gridDim.x * blockDim.x)
    {
        const size_t n = idx / wpr, wi = idx - n * wpr;
        const float h = 0.5f * tau[n];
        const float* row = W + n * K;
        const size_t k0 = wi * 16;
        uint32_t word = 0;
        if (vec4 && k0 + 16 <= K)
        {
            const float4* p = reinterpret_cast<const float4*>(row + k0);
#pragma unroll
            for (int v = 0; v < 4; ++v)
            {
                const float4 f = p[v];
                const float e[4] = {f.x, f.y, f.z, f.w};
#pragma unroll
                for (int c = 0; c < 4; ++c)
                {
                    const uint32_t code = e[c] > h ? 3u : (e[c] < -h ? 1u : 2u);
                    word |= code << (2 * (4 * v + c));
                }
            }
        }
        else
        {
            for (int j = 0; j < 16; ++j)
            {
                const size_t k = k0 + j;
                uint32_t code = 2u;
                if (k < K)
                {
                    const float e = row[k];
                    code = e > h ? 3u : (e < -h ? 1u : 2u);
                }
                word |= code << (2 * j);
            }
        }
        wq[idx] = word;
    }
}

// Column max over rows of a (rows, cols) row-major matrix. Block = 64 columns x 4 waves;
// wave w scans rows w, w+4, ...; partials combine in LDS. Max is order-free. NaN never
// compares greater, so it is ignored (as std::max(mx, v) in src/int8_act_test.cpp:95-101).
__global__ __launch_bounds__(kBlock) void k_col_reduce_max(const float* __restrict__ x, size_t rows,
                                                           size_t cols, bool absval,
                                                           float post_scale, bool do_scale,
                                                           float* __restrict__ out)
{
    __shared__ float part[4][kWave];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const size_t c = (size_t)blockIdx.x * kWave + lane;
    float m = absval ? 0.0f : -INFINITY;
    if (c < cols)
        for (size_t r = (size_t)w; r < rows; r += 4)
        {
            float v = x[r * cols + c];
            if (absval) v = fabsf(v);
            m = v > m ? v : m;
        }
    part[w][lane] = m;
    __syncthreads();
    if (w == 0 && c < cols)
    {
        float r = part[0][lane];
#pragma unroll
        for (int i = 1; i < 4; ++i) r = part[i][lane] > r ? part[i][lane] : r;
        out[c] = do_scale ? __fmul_rn(r, post_scale) : r;
    }
}

__global__ void k_abs(const float* __restrict__ x, size_t n, float* __restrict__ out)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        out[i] = fabsf(x[i]);
}

__global__ void k_scale(float* __restrict__ x, size_t n, float alpha)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        x[i] = __fmul_rn(x[i], alpha);
}

__device__ __forceinline__ int quantize_one(float x, float s)
{
    if (s == 0.0f || isnan(x)) return 0;
    float v = __fdiv_rn(x, s);
    if (isnan(v)) return 0;
    v = fminf(fmaxf(v, -127.0f), 127.0f);
    return (int)roundf(v);  // round half away from zero
}

// One thread per output word of the (rows, ceil(cols/4)) int8 container.
__global__ __launch_bounds__(kBlock) void k_quantize_i8(const float* __restrict__ x,
                                                        const float* __restrict__ scale, size_t rows,
                                                        size_t cols, size_t wpr, bool col_scale,
                                                        uint32_t* __restrict__ out)
{
    const size_t total = rows * wpr;
    for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (size_t)gridDim.x * blockDim.x)
    {
        const size_t r = idx / wpr, wi = idx - r * wpr;
        uint32_t word = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b)
        {
            const size_t c = wi * 4 + b;
            if (c < cols)
            {
                const float s = col_scale ? scale[c] : scale[r];
                const int q = quantize_one(x[r * cols + c], s);
                word |= (uint32_t)(q & 0xFF) << (8 * b);
            }
        }
        out[idx] = word;
    }
}

__global__ __launch_bounds__(kBlock) void k_unpack_i8(const uint32_t* __restrict__ packed,
                                                      size_t rows, size_t cols, size_t wpr,
                                                      float* __restrict__ out)
{
    const size_t total = rows * cols;
    for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (size_t)gridDim.x * blockDim.x)
    {
        const size_t r = idx / cols, c = idx - r * cols;
        const uint32_t w = packed[r * wpr + c / 4];
        out[idx] = (float)(int8_t)(uint8_t)((w >> (8 * (c % 4))) & 0xFFu);
    }
}

__global__ void k_add_row_broadcast(float* __restrict__ Y, const float* __restrict__ b, size_t N,
                                    size_t M)
{
    const size_t total = N * M;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x)
        Y[i] = __fadd_rn(Y[i], b[i / M]);
}

// XOR of all words of a buffer, in one streaming pass: every thread keeps kReadUnroll
// non-temporal 16-byte loads in flight per step, then a wave / block xor reduction to one
// partial per block; k_xor_fold xors the partials into *out. (One device-scope atomic per
// block instead costs ~4 % at 1024 blocks: they serialize on one address across the XCDs.)
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kReadUnroll = 4;

__global__ __launch_bounds__(kBlock) void k_stream_xor(const u32x4* __restrict__ p, size_t n16,
                                                       const uint32_t* __restrict__ tail, int ntail,
                                                       uint32_t* __restrict__ part)
{
    __shared__ uint32_t sred[kBlock / kWave];
    uint32_t acc = 0;
    const size_t stride = (size_t)gridDim.x * kBlock * kReadUnroll;
    size_t i = (size_t)blockIdx.x * kBlock * kReadUnroll + threadIdx.x;
    for (; i + (size_t)kBlock * (kReadUnroll - 1) < n16; i += stride)
    {
        u32x4 v[kReadUnroll];
#pragma unroll
        for (int u = 0; u < kReadUnroll; ++u) v[u] = __builtin_nontemporal_load(p + i + (size_t)kBlock * u);
#pragma unroll
        for (int u = 0; u < kReadUnroll; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    // the groups after the last whole one start past n16, so one partial group remains
#pragma unroll
    for (int u = 0; u < kReadUnroll; ++u)
    {
        const size_t j = i + (size_t)kBlock * u;
        if (j < n16)
        {
            const u32x4 v = __builtin_nontemporal_load(p + j);
            acc ^= v.x ^ v.y ^ v.z ^ v.w;
        }
    }
    if (blockIdx.x == 0 && (int)threadIdx.x < ntail) acc ^= tail[threadIdx.x];
    for (int off = 32; off >= 1; off >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, off, kWave);
    if ((threadIdx.x & 63) == 0) sred[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0)
    {
        uint32_t t = 0;
        for (int w = 0; w < kBlock / kWave; ++w) t ^= sred[w];
        part[blockIdx.x] = t;
    }
}

__global__ __launch_bounds__(kBlock) void k_xor_fold(const uint32_t* __restrict__ part, int n,
                                                     uint32_t* __restrict__ out)
{
    __shared__ uint32_t sred[kBlock / kWave];
    uint32_t acc = 0;
    for (int i = threadIdx.x; i < n; i += kBlock) acc ^= part[i];
    for (int off = 32; off >= 1; off >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, off, kWave);
    if ((threadIdx.x & 63) == 0) sred[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0)
    {
        uint32_t t = *out;
        for (int w = 0; w < kBlock / kWave; ++w) t ^= sred[w];
        *out = t;
    }
}

}  // namespace

size_t stream_xor_blocks(size_t bytes, int num_cus)
{
    const size_t n16 = bytes / 16;
    const size_t g = ceil_div(n16 > 0 ? n16 : 1, (size_t)kBlock * kReadUnroll);
    const size_t cap = (size_t)(num_cus > 0 ? num_cus : 256) * 4;
    return g < cap ? g : cap;
}

hipError_t launch_stream_xor(hipStream_t st, const void* src, size_t bytes, uint32_t* part, uint32_t* out,
                             int num_cus)
{
    const size_t n16 = bytes / 16;
    const int ntail = (int)((bytes % 16) / 4);
    const size_t g = stream_xor_blocks(bytes, num_cus);
    hipLaunchKernelGGL(k_stream_xor, dim3((unsigned)g), dim3(kBlock), 0, st, static_cast<const u32x4*>(src), n16,
                       static_cast<const uint32_t*>(src) + n16 * 4, ntail, part);
    hipLaunchKernelGGL(k_xor_fold, dim3(1), dim3(kBlock), 0, st, part, (int)g, out);
    return hipGetLastError();
}

hipError_t launch_f32_to_f16(hipStream_t st, const float* src, size_t n, uint16_t* dst)
{
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_f32_to_f16, dim3(grid_for(n)), dim3(kBlock), 0, st, src, n, dst);
    return hipGetLastError();
}

hipError_t launch_f16_to_f32(hipStream_t st, const uint16_t* src, size_t n, float* dst)
{
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_f16_to_f32, dim3(grid_for(n)), dim3(kBlock), 0, st, src, n, dst);
    return hipGetLastError();
}

hipError_t launch_fill_u32(hipStream_t st, uint32_t* dst, uint32_t value, size_t words)
{
    if (words == 0) return hipSuccess;
    hipLaunchKernelGGL(k_fill_u32, dim3(grid_for(words)), dim3(kBlock), 0, st, dst, value, words);
    return hipGetLastError();
}

hipError_t launch_row_absmean(hipStream_t st, const float* W, size_t N, size_t K, float* tau)
{
    if (N == 0) return hipSuccess;
    const float inv_k = 1.0f / (float)K;
    const unsigned grid = (unsigned)ceil_div(N, kBlock / kWave);
    hipLaunchKernelGGL(k_row_absmean, dim3(grid), dim3(kBlock), 0, st, W, N, K, inv_k, tau);
    return hipGetLastError();
}

hipError_t launch_trit_pack(hipStream_t st, const float* W, const float* tau, size_t N, size_t K,
                            uint32_t* wq)
{
    const size_t wpr = ceil_div(K, 16);
    if (N == 0 || wpr == 0) return hipSuccess;
    const bool vec4 = (K % 4 == 0) && ((reinterpret_cast<uintptr_t>(W) & 15) == 0);
    hipLaunchKernelGGL(k_trit_pack, dim3(grid_for(N * wpr)), dim3(kBlock), 0, st, W, tau, N, K, wpr,
                       vec4, wq);
    return hipGetLastError();
}

hipError_t launch_col_reduce_max(hipStream_t st, const float* x, size_t rows, size_t cols,
                                 float* out, bool absval, float post_scale)
{
    if (cols == 0) return hipSuccess;
    const bool do_scale = post_scale != 1.0f;
    hipLaunchKernelGGL(k_col_reduce_max, dim3((unsigned)ceil_div(cols, kWave)), dim3(kBlock), 0, st,
                       x, rows, cols, absval, post_scale, do_scale, out);
    return hipGetLastError();
}

hipError_t launch_abs(hipStream_t st, const float* x, size_t n, float* out)
{
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_abs, dim3(grid_for(n)), dim3(kBlock), 0, st, x, n, out);
    return hipGetLastError();
}

hipError_t launch_scale(hipStream_t st, float* x, size_t n, float alpha)
{
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_scale, dim3(grid_for(n)), dim3(kBlock), 0, st, x, n, alpha);
    return hipGetLastError();
}

hipError_t launch_quantize_i8(hipStream_t st, const float* x, const float* scale, size_t rows,
                              size_t cols, bool col_scale, uint32_t* out)
{
    const size_t wpr = ceil_div(cols, 4);
    if (rows == 0 || wpr == 0) return hipSuccess;
    hipLaunchKernelGGL(k_quantize_i8, dim3(grid_for(rows * wpr)), dim3(kBlock), 0, st, x, scale,
                       rows, cols, wpr, col_scale, out);
    return hipGetLastError();
}

hipError_t launch_unpack_i8(hipStream_t st, const uint32_t* packed, size_t rows, size_t cols,
                            float* out)
{
    if (rows == 0 || cols == 0) return hipSuccess;
    hipLaunchKernelGGL(k_unpack_i8, dim3(grid_for(rows * cols)), dim3(kBlock), 0, st, packed, rows,
                       cols, ceil_div(cols, 4), out);
    return hipGetLastError();
}

hipError_t launch_add_row_broadcast(hipStream_t st, float* Y, const float* b, size_t N, size_t M)
{
    if (N == 0 || M == 0) return hipSuccess;
    hipLaunchKernelGGL(k_add_row_broadcast, dim3(grid_for(N * M)), dim3(kBlock), 0, st, Y, b, N, M);
    return hipGetLastError();
}

}  // namespace nnhip
