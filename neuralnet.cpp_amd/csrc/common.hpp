// common.hpp — shared declarations of libnn-hip.so (gfx950 only).
//
// Kernel launchers are host functions that enqueue on a given stream and return the
// hipError_t of the launch; the C ABI (runtime.hip) validates arguments before calling them.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "nnhip.h"

namespace nnhip
{

constexpr int kWave = 64;

// Cache-policy operands of buffer loads and stores (gfx950 bits: sc0 = 1, nt = 2, sc1 = 16).
// A store with sc0 sc1 (system scope) is written through the L2 as it is issued; with the default
// policy a large output sits dirty in the L2 and is written back at the end of the kernel, after
// the last wave, where nothing overlaps it.
constexpr int kPolicyNT = 2;
constexpr int kPolicySys = 17;

// T16K256 repacked-weight geometry (see include/nnhip.h and oracle/nn_oracle.c).
constexpr int kTileRows = 16;
constexpr int kTileK = 256;
constexpr int kTileWords = 256;  // 1 KiB per tile

__host__ __device__ inline size_t round_up(size_t v, size_t m) { return (v + m - 1) / m * m; }
__host__ __device__ inline size_t ceil_div(size_t v, size_t m) { return (v + m - 1) / m; }

// 16-byte vector of u32 (a native clang vector, usable with the nontemporal builtins)
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Largest M handled by the weight-streaming decode GEMV (one 16-token MFMA column block).
constexpr int kGemvMaxM = 16;
// Decode GEMV geometry shared by the kernels and the host schedule. Two variants:
//  * LDS: the group's activations are staged in LDS (they fit kGemvLdsBudget), one 16-row
//    tile per wave item, 3 k-tile stages in flight, 16 waves per CU (M = 1 decode);
//  * register: activations are loaded with the weights, 8 row tiles per item share them,
//    3 stages (larger M). The kernel takes 481 VGPRs (accumulators, stages and epilogue
//    operands of 8 row tiles), so one wave per SIMD is resident: the grid is 4 waves per CU
//    (sized for 8, the launch ran as two rounds: 5018 against 5117 GB/s on the M = 16 sweep).
//    At M = 16 the sweep measured 4505 GB/s with 4 tiles and 4 stages, 4635 with 4 tiles at
//    two waves per SIMD (256 VGPRs), 5117 with 8 and 3.
// Tuned on MI355X with the 30-layer BitNet-2B sweep (M = 1 and M = 16).
#ifndef NNHIP_GEMV_LDS_DEPTH
#define NNHIP_GEMV_LDS_DEPTH 3
#endif
#ifndef NNHIP_GEMV_LDS_WAVES
#define NNHIP_GEMV_LDS_WAVES 16
#endif
#ifndef NNHIP_GEMV_REG_RTW
#define NNHIP_GEMV_REG_RTW 8
#endif
#ifndef NNHIP_GEMV_REG_DEPTH
#define NNHIP_GEMV_REG_DEPTH 3
#endif
#ifndef NNHIP_GEMV_REG_WAVES
#define NNHIP_GEMV_REG_WAVES 4
#endif
#ifndef NNHIP_GEMV_BIG_DEPTH
#define NNHIP_GEMV_BIG_DEPTH 2
#endif
constexpr int kLdsRTW = 1, kLdsDepth = NNHIP_GEMV_LDS_DEPTH, kLdsWavesPerCu = NNHIP_GEMV_LDS_WAVES;
// The 16-wave blocks (one per CU, activation sets beyond 48 KiB) keep 2 stages in flight: with
// 16 waves per CU that holds as many bytes in flight, and the M = 16 sweep measured 102.6-102.7
// against 103.6-104.5 us at 3 stages (97.9-98.8 against 101.2-101.8 us with write-through stores).
constexpr int kBigDepth = NNHIP_GEMV_BIG_DEPTH;
constexpr int kRegRTW = NNHIP_GEMV_REG_RTW, kRegDepth = NNHIP_GEMV_REG_DEPTH, kRegWavesPerCu = NNHIP_GEMV_REG_WAVES;

struct GemvVariant
{
    int row_tiles;
    int waves_per_cu;
};
inline GemvVariant gemv_variant(bool lds)
{
    return lds ? GemvVariant{kLdsRTW, kLdsWavesPerCu} : GemvVariant{kRegRTW, kRegWavesPerCu};
}

struct GemvProblem
{
    const u32x4* rp;
    const float* tau;
    const int8_t* xi;
    const float* s;
    const int32_t* rowsum;
    const float* bias;
    float* y;
    int32_t N, K, M, KT;  // KT = Kp / 256
    int32_t xlds;         // byte offset of this problem's activations in LDS, or -1
    int32_t glu;          // prefill GEMM epilogue: 0 plain Y, else gated activation act = glu - 1
                          // (0 SwiGLU, 1 ReLU^2-GLU) of interleaved gate/up rows into y (glu_F, M)
    int32_t glu_F;        // features of the gated output (rows of y when glu != 0)
    int32_t ytm;          // deep decode GEMV with glu: h token-major (M, glu_F) instead of (glu_F, M)
    const float* res;     // deep decode GEMV: residual (N, M) added after the epilogue (may alias y), or null
};

// ---- gated activations (shared by k_glu.hip and the GEMM epilogue)
// exp(x) from IEEE-rounded operations in a fixed order (no fused multiply-add): Cody-Waite
// reduction x = k ln2 + r with ln2 split as 22713/32768 + fl(ln2 - 22713/32768) (the first
// product is exact for |k| < 256, the first difference exact by Sterbenz), then the Taylor
// series of e^r to r^7 (|r| <= 0.347: truncation < 6e-9 relative) and ldexp. x > 100 -> inf,
// x < -87 -> 0 (no subnormal results), NaN propagates. Within 2 ulp of exp.
__device__ __forceinline__ float glu_exp(float x)
{
    if (x != x) return x;
    if (x > 100.0f) return __builtin_inff();
    if (x < -87.0f) return 0.0f;
    const float k = __builtin_rintf(x * 0x1.715476p+0f);
    const float r = (x - k * 0x1.62e4p-1f) - k * 0x1.7f7d1cp-20f;
    float p = 0x1.a01a02p-13f;
    p = p * r + 0x1.6c16c2p-10f;
    p = p * r + 0x1.111112p-7f;
    p = p * r + 0x1.555556p-5f;
    p = p * r + 0x1.555556p-3f;
    p = p * r + 0.5f;
    p = p * r + 1.0f;
    p = p * r + 1.0f;
    return __builtin_ldexpf(p, (int)k);
}

// act 1: ReLU^2-GLU (r * r) * u with r = g > 0 ? g : 0; otherwise SwiGLU (g * (1/(1+exp(-g)))) * u
__device__ __forceinline__ float glu_one(float g, float u, int act)
{
    if (act == 1)
    {
        const float r = g > 0.0f ? g : 0.0f;
        return (r * r) * u;
    }
    const float sig = 1.0f / (1.0f + glu_exp(-g));
    return (g * sig) * u;
}

// One activation block the decode GEMV stages in LDS at block start (M * Kp bytes).
struct XStage
{
    const int8_t* src;
    uint32_t bytes;   // multiple of 256
    uint32_t lds_off;
    uint32_t row;     // bytes of one token row (Kp): the 16-byte units of row t are staged XOR-swizzled
};

// LDS budget per block for staged activations (3 blocks of 4 waves fit one CU).
constexpr uint32_t kGemvLdsBudget = 48 * 1024;
// A single activation block up to this size is staged by 1024-thread blocks (16 waves sharing
// it, one block per CU); larger ones go to the register variant.
constexpr uint32_t kGemvLdsBigBudget = 152 * 1024;

// ---- reference-layout kernels (k_ref.hip)
hipError_t launch_fill_u32(hipStream_t st, uint32_t* dst, uint32_t value, size_t words);
hipError_t launch_f32_to_f16(hipStream_t st, const float* src, size_t n, uint16_t* dst);
hipError_t launch_f16_to_f32(hipStream_t st, const uint16_t* src, size_t n, float* dst);
hipError_t launch_row_absmean(hipStream_t st, const float* W, size_t N, size_t K, float* tau);
hipError_t launch_trit_pack(hipStream_t st, const float* W, const float* tau, size_t N, size_t K,
                            uint32_t* wq);
hipError_t launch_col_reduce_max(hipStream_t st, const float* x, size_t rows, size_t cols,
                                 float* out, bool absval, float post_scale);
hipError_t launch_abs(hipStream_t st, const float* x, size_t n, float* out);
hipError_t launch_scale(hipStream_t st, float* x, size_t n, float alpha);
hipError_t launch_quantize_i8(hipStream_t st, const float* x, const float* scale, size_t rows,
                              size_t cols, bool col_scale, uint32_t* out);
hipError_t launch_unpack_i8(hipStream_t st, const uint32_t* packed, size_t rows, size_t cols,
                            float* out);
hipError_t launch_add_row_broadcast(hipStream_t st, float* Y, const float* b, size_t N, size_t M);
// Float-activation products (k_matq.hip): the plan splits the reduction into chunks whose
// partial sums (part_bytes of scratch, 0 for one chunk) a second kernel adds in fixed order.
struct MatqPlan
{
    int n_chunks;
    int chunk;          // packed words of the reduction per chunk
    size_t part_bytes;  // scratch: [transposed container (at_bytes)] + partial sums
    size_t at_bytes;    // matmul_q_t only
};
MatqPlan plan_matmul_q(size_t N, size_t K, size_t M);
MatqPlan plan_matmul_q_t(size_t K, size_t M, size_t N);
hipError_t launch_matmul_q(hipStream_t st, const uint32_t* wq, const float* tau, const void* B, bool b16, size_t N,
                           size_t K, size_t M, void* Y, bool y16, const MatqPlan& plan, float* part);
hipError_t launch_matmul_q_t(hipStream_t st, const uint32_t* A, const float* tau, const void* B, bool b16, size_t K,
                             size_t M, size_t N, void* Y, bool y16, const MatqPlan& plan, float* scratch);

// ---- activation kernels (k_act.hip)
// Extra blocks of the one-token kernels (k_token_one, k_token_epi) that read up to kPfRanges
// device ranges in whole 16-byte units with the default cache policy while the kernel's tokens
// are processed, so that the next kernel, which reads the same bytes, finds them in the
// memory-side cache (256 MB) instead of HBM. Outputs do not depend on it.
constexpr int kPfRanges = 4;
constexpr int kOneThreadsHost = 512;                  // threads of a one-token block
// loads per prefetch thread: 4 and 2 measured alike in the decode step, 1 (more blocks to
// dispatch) and 16 (prefetch blocks outlasting the quantizer) slower
constexpr int kPfUnitsPerThread = 4;
constexpr uint64_t kPfMaxUnits = (64ull << 20) / 16;  // at most 64 MiB per kernel
struct Prefetch
{
    const void* p[kPfRanges];
    uint32_t n16[kPfRanges];  // 16-byte units per range
    int blocks;               // extra blocks of 512 threads (0: none)
};
hipError_t launch_rmsnorm(hipStream_t st, const float* X, const float* gamma, float eps, size_t F,
                          size_t M, float* out);
hipError_t launch_layernorm(hipStream_t st, const float* X, const float* gamma, const float* beta, float eps,
                            size_t F, size_t M, float* out);
// Epilogue of a split-k GEMV (part[S][M][N] slice sums) + residual, then [RMSNorm ->] absmax
// int8 quantization, one token per block (epilogue_quant_ok: M <= 64, N <= 11264).
struct EpiArgs
{
    const int32_t* part;
    int S;
    const float* tau;          // (N)
    const float* s_in;         // (M) scales of the GEMV's input tokens
    const int32_t* rowsum_in;  // (M) code sums of the GEMV's input tokens
    const float* bias;         // (N) or null
    const float* res;          // (N, M) residual or null
    float* xout;               // (N, M) epilogue + residual (may alias res)
    int tm;                    // res and xout are token-major (M, N)
};
bool epilogue_quant_ok(size_t N, size_t M);
hipError_t launch_epilogue_quant(hipStream_t st, const EpiArgs& e, const float* gamma, bool norm, float eps, size_t N,
                                 size_t M, int8_t* xi, float* s, int32_t* rowsum, const Prefetch* pf = nullptr);
// The one-token [RMSNorm (gamma) ->] absmax -> int8 pass on a token-major X (M, K), decode sizes
// (token_quant_tm_ok: M <= 64, K <= 11264); same bits as launch_act_quant on X transposed.
bool token_quant_tm_ok(size_t K, size_t M);
hipError_t launch_token_quant_tm(hipStream_t st, const float* X, const float* gamma, float eps, size_t K, size_t M,
                                 int8_t* xi, float* s, int32_t* rowsum, const Prefetch* pf = nullptr);
hipError_t launch_embed_token_quant(hipStream_t st, const float* table, const int32_t* ids, size_t V, const float* gamma,
                                   float eps, size_t K, size_t M, float* xout, int8_t* xi, float* s, int32_t* rowsum,
                                   const Prefetch* pf);
hipError_t launch_act_quant(hipStream_t st, const float* X, const float* gamma, bool norm, float eps,
                            size_t K, size_t M, int8_t* xi, float* s, int32_t* rowsum,
                            uint32_t* xq_ref, const Prefetch* pf = nullptr);
hipError_t launch_act_from_container(hipStream_t st, const uint32_t* xq, size_t K, size_t M,
                                     int8_t* xi, int32_t* rowsum);
hipError_t launch_act_to_container(hipStream_t st, const int8_t* xi, size_t K, size_t M,
                                   uint32_t* xq);

// ---- ternary kernels (k_ternary.hip, k_gemv.hip)
hipError_t launch_repack(hipStream_t st, const uint32_t* wq, size_t N, size_t K, uint32_t* rp);
hipError_t launch_unrepack(hipStream_t st, const uint32_t* rp, size_t N, size_t K, uint32_t* wq);
hipError_t launch_gemv(hipStream_t st, const GemvProblem& p, int num_cus);
// Deep single-problem decode GEMV (all k stages in flight per wave, activations staged in LDS;
// p.glu selects the gated epilogue into p.y = h). Applies when gemv_deep_ok: KT in {4, 10, 16, 27},
// round_up(M * Kp, 1 KiB) <= kGemvDeepLds and at most kGemvDeepMaxTilesPerCu row tiles per CU.
constexpr uint32_t kGemvDeepLds = 160 * 1024;
constexpr int kGemvDeepMaxTilesPerCu = 4;
bool gemv_deep_ok(const GemvProblem& p, int num_cus);
hipError_t launch_gemv_deep(hipStream_t st, const GemvProblem& p);
// Up to kGemvDeepMulti problems that share K, M and the activations (xi, s, rowsum) in one deep
// launch; gemv_deep_multi_ok checks the shared shape and the total row tiles.
constexpr int kGemvDeepMulti = 4;
bool gemv_deep_multi_ok(const GemvProblem* ps, int count, int num_cus);
hipError_t launch_gemv_deep_multi(hipStream_t st, const GemvProblem* ps, int count);
// Split-k partial sums (no epilogue): part[ks][t][n] int32, S slices of ceil(KT / S) k tiles
// (each slice non-empty and at most 14 tiles long, S <= 32, M <= 16); the epilogue runs in the
// kernel that follows (the decoder's per-token kernel takes S <= 8).
bool gemv_part_ok(const GemvProblem& p, int S);
hipError_t launch_gemv_part(hipStream_t st, const GemvProblem& p, int S, int32_t* part);
// Grouped GEMV over a precomputed per-wave schedule: wave w runs the items
// d_wave_items[d_wave_start[w] .. d_wave_start[w+1]) (item = problem << 20 | row tile).
// If n_xstage > 0, the listed activation blocks (lds_bytes in total) are staged in LDS at
// block start and every problem reads its activations at its xlds offset.
hipError_t launch_gemv_grouped(hipStream_t st, const GemvProblem* d_probs, const uint32_t* d_wave_start,
                               const uint32_t* d_wave_items, size_t n_waves, const XStage* d_xstage,
                               int n_xstage, uint32_t lds_bytes);
size_t gemv_grid_waves(size_t n_items, int num_cus, bool lds);
// Prefill GEMM; tile is one of NNHIP_GEMM_TILE_* (AUTO: gemm_tile_choice).
hipError_t launch_gemm(hipStream_t st, const GemvProblem& p, int num_cus, int tile);
int gemm_tile_choice(const GemvProblem& p, int num_cus);
// Time of one round of 128 x 128 / 64 x 64 blocks relative to one round of 256 x 128 blocks,
// measured over M = 128..4096, K = 2560..6912, N = 2560..13824 (with these the automatic choice
// picked the fastest tile on every measured shape).
constexpr double kGemmRelB = 0.6, kGemmRelC = 0.45;
// The automatic choice may split the rows: 256 x 128 blocks over the longest row prefix that
// fills whole rounds of the CUs, then the remaining rows in a second launch (tail_tile), when the
// estimate (rounds, plus kGemmSplitCost of a 256 x 128 round for the second launch) is lower
// than every single-launch tile's. rows = 0: one launch of tile.
struct GemmSplit
{
    int tile, rows, tail_tile;
};
constexpr double kGemmSplitCost = 0.1;
GemmSplit gemm_split_choice(const GemvProblem& p, int num_cus);

// ---- gated activations (k_glu.hip)
hipError_t launch_glu(hipStream_t st, const float* Y1, size_t F, size_t M, int act, bool interleaved, float* h);
hipError_t launch_glu_interleave(hipStream_t st, const uint32_t* wq, const float* tau, const float* bias, size_t F,
                                 size_t K, uint32_t* wq_out, float* tau_out, float* bias_out);

// ---- ternary x float products on the MFMA path (k_digits.hip): digit split of the activations
// (4 int8 digit tokens per token, row sums, per-token exponents) and the int64 combine
// kscale (nullable, per k) multiplies the activations first (the transposed product's tau);
// tau (nullable) is the per-row output factor.
hipError_t launch_digits(hipStream_t st, const void* B, bool b16, const float* kscale, size_t K, size_t M, int8_t* xi,
                         int32_t* rowsum, int32_t* ex);
hipError_t launch_digit_combine(hipStream_t st, const float* Yp, const float* tau, const int32_t* ex,
                                const uint32_t* rp, const void* B, bool b16, const float* kscale, size_t N, size_t K,
                                size_t M, void* Y, bool y16);
// split-k form for a few long tokens (M <= 4): digits in chunks of 4096 columns (P =
// digit_chunks(K) partial digit sums per token), the slice sums of k_gemv_part, and a combine
// that adds both exactly (bit-identical to the unit-scale GEMV path)
size_t digit_chunks(size_t K);
hipError_t launch_digits_chunks(hipStream_t st, const void* B, bool b16, const float* kscale, size_t K, size_t M,
                                int8_t* xi, int32_t* rsp, int32_t* ex);
hipError_t launch_digit_combine_parts(hipStream_t st, const int32_t* part, int S, const int32_t* rsp, size_t P,
                                      const float* tau, const int32_t* ex, const uint32_t* rp, const void* B, bool b16,
                                      const float* kscale, size_t N, size_t K, size_t M, void* Y, bool y16);
// the same product in one launch at decode sizes (f32 activations, M <= 4, K % 4 == 0, 16-byte
// aligned B, the compiled k-tile counts): digits in LDS per block, int64 combine in the
// epilogue; bit-identical to the three launches
bool digit_gemv_ok(size_t N, size_t K, size_t M, bool b16, const void* B);
hipError_t launch_digit_gemv(hipStream_t st, const void* rp, const float* tau, const float* kscale, const float* B,
                             size_t N, size_t K, size_t M, void* Y, bool y16);
// *out ^= xor of the bytes / 4 words at src, one streaming pass into stream_xor_blocks()
// per-block partials, then a one-block fold (k_ref.hip)
size_t stream_xor_blocks(size_t bytes, int num_cus);
hipError_t launch_stream_xor(hipStream_t st, const void* src, size_t bytes, uint32_t* part, uint32_t* out,
                             int num_cus);
// Bit transpose of a packed container: A (K, ceil(M/16)) -> At (M, ceil(K/16)) (k_matq.hip)
hipError_t launch_trit_transpose(hipStream_t st, const uint32_t* A, size_t K, size_t M, uint32_t* At);

// ---- batched decode step (k_decode.hip)
size_t attn_chunks(size_t len_bound);
size_t attn_workspace_bytes(size_t B, size_t H, size_t Hkv, size_t dk, size_t len_bound);
// caches of f32, or of f16 elements when cache_f16 (compute = F16); tm: q, k, v and out token-major
hipError_t launch_attn_decode(hipStream_t st, const float* q, const float* k, const float* v, size_t B, size_t H,
                              size_t Hkv, size_t dk, const int32_t* pos, size_t len_bound, const float* cosT,
                              const float* sinT, void* kc, void* vc, bool cache_f16, size_t max_len, float scale,
                              float* part, float* out, int num_cus, bool tm = false);
hipError_t launch_add(hipStream_t st, const float* x, const float* y, size_t n, float* out);
// dst (rows, n) column j = src (rows, src_cols) column col0 + j * stride (k_decode.hip)
hipError_t launch_copy_cols(hipStream_t st, const float* src, size_t rows, size_t src_cols, size_t col0, size_t stride,
                            size_t n, float* dst);

// ---- batched prefill (k_prefill.hip): T tokens of each of B sequences at positions pos0 + t
bool prefill_dk_supported(size_t dk);
hipError_t launch_kv_fill(hipStream_t st, const float* k, const float* v, size_t B, size_t T, size_t Hkv, size_t dk,
                          size_t pos0, const float* cosT, const float* sinT, void* kc, void* vc, bool cache_f16,
                          size_t max_len);
hipError_t launch_attn_prefill(hipStream_t st, const float* q, const void* kc, const void* vc, bool cache_f16,
                               size_t B, size_t T, size_t H, size_t Hkv, size_t dk, size_t pos0, const float* cosT,
                               const float* sinT, size_t max_len, float scale, float* out);
hipError_t launch_embed(hipStream_t st, const float* table, const int32_t* ids, size_t V, size_t d, size_t B, bool tm,
                        float* out);
hipError_t launch_argmax(hipStream_t st, const float* L, size_t V, size_t B, int32_t* ids, bool rows = false,
                         int32_t* pos = nullptr);

}  // namespace nnhip
