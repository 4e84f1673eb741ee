// gemv_tile.hpp — the pieces of a ternary x int8 MFMA GEMV tile shared by the decode GEMV
// kernels (k_gemv.hip) and the one-launch float-activation GEMV (k_digits.hip): buffer
// resources and loads, the v_mfma_i32_16x16x64_i8 step on four accumulators per 16-row tile.
//
// A T16K256 weight tile (16 rows x 256 k, 1 KiB) is one 16-byte load per lane; bits 8b + 2j of
// lane word q are codes (trit + 2) of four MFMAs j = 0..3. Four accumulators with scaled codes
// make the unpack 5 VALU ops per weight word instead of 7:
//   j=0: w & 0x03030303 (codes)          -> a0      j=1: w & 0x0C0C0C0C (4 * codes)  -> a1
//   j=2: w & 0x30303030 (16 * codes)     -> a2      j=3: (w >> 6) & 0x03030303       -> a3
//   acc = a0 + a3 + (a1 >> 2) + (a2 >> 4) - 2 * rowsum       (shifts divide exact multiples)
// Output layout of the 16x16 MFMA: lane l = 16 g + t holds rows 4g + i (i = 0..3) of column
// (token) t. The A and B operands share one lane layout (lane l: row / column l % 16, k block
// l / 16), so passing the activations as A and the codes as B (kT) computes the transposed
// tile from the same registers: lane 16 g + r then holds tokens 4g + i of row r, four
// consecutive floats of a feature-major (N, M) output.
#pragma once

#include "common.hpp"

namespace nnhip
{
namespace
{

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr uint32_t kM3 = 0x03030303u;
constexpr uint32_t kOOB = 0x80000000u;
constexpr int kRsrcFlags = 0x00020000;      // gfx9-family buffer resource word 3 (raw, dword)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kRsrcFlags);
}

// kAux is the cache-policy operand: 0 = default; kNT = non-temporal ("nt" on gfx950), for the
// weight stream, which is read once per launch (measured on MI355X: a streaming read reaches
// about 7.0 TB/s with nt loads and about 6.1 TB/s without).
constexpr int kNT = 2;
template <int kAux = 0>
__device__ __forceinline__ v4i ld16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff)
{
    return __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, kAux));
}

__device__ __forceinline__ v4i mfma16(v4i a, v4i b, v4i c)
{
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

struct Acc
{
    v4i a0, a1, a2, a3;
};

template <bool kT>
__device__ __forceinline__ v4i mfma_wx(v4i w, v4i x, v4i c)
{
    return kT ? mfma16(x, w, c) : mfma16(w, x, c);
}

template <int kRTW, bool kT = false>
__device__ __forceinline__ void compute_stage(const v4i (&w4)[kRTW], const v4i (&x)[4], Acc (&acc)[kRTW])
{
#pragma unroll
    for (int r = 0; r < kRTW; ++r)
    {
        const v4i w = w4[r];
        acc[r].a0 = mfma_wx<kT>(w & (int)kM3, x[0], acc[r].a0);
        acc[r].a1 = mfma_wx<kT>(w & (int)(kM3 << 2), x[1], acc[r].a1);
        acc[r].a2 = mfma_wx<kT>(w & (int)(kM3 << 4), x[2], acc[r].a2);
        acc[r].a3 = mfma_wx<kT>((v4i)((__builtin_bit_cast(u32x4, w) >> 6) & kM3), x[3], acc[r].a3);
    }
}

// the four accumulators of one row tile combined: the int32 sum of code * x over k
__device__ __forceinline__ int acc_sum(const Acc& a, int i)
{
    return a.a0[i] + a.a3[i] + (a.a1[i] >> 2) + (a.a2[i] >> 4);
}

}  // namespace
}  // namespace nnhip
