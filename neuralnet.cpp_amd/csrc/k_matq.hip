// k_matq.hip — ternary x float products on the reference packed container (f32 or f16
// activations, f32 accumulation): the reference's default BitLinear branch and its dX path.
//
//   matmul_q   Y (N, M)  = (tau o trit(wq)) . B,        wq (N, ceil(K/16)), B (K, M)
//   matmul_q_t Y (M, N)  = (tau o trit(A))^T . B,       A  (K, ceil(M/16)), B (K, N), tau per
//                                                        stored row k
//
// matmul_q streams the packed words from HBM once per token block (0.25 B per weight) with
// coalesced 4-byte loads (64 lanes read 256 contiguous bytes of one row): one wave owns 16
// rows and a window of 64 words (1024 k) per step; lane l takes word l of the window, holds
// its 16 x MT activations in registers, walks the 16 rows, and the 16 x MT partial sums are
// combined across the 64 lanes by a halving transpose-reduce (lane l ends with row l/4).
// Large reductions are split over waves into chunks whose partial sums a second kernel adds
// in ascending chunk order, so results do not depend on scheduling.
// matmul_q_t runs the same kernel on a bit-transposed copy of the container (made in scratch
// by k_trit_transpose) with tau folded into the activations: fl(tau_k * b) * trit equals
// fl(tau_k * trit) * b exactly, since trit is -1, 0 or 1.
// Trits are decoded exactly through an fp8 byte table (trits4); products are accumulated with
// fmaf. The reference pins only a tolerance, 1e-4 x max(1, max|Y|) in f32 and 4e-3 with f16
// operands (src/ternary_gemm_test.cpp:503-516).
#include "common.hpp"

namespace nnhip
{
namespace
{

constexpr int kMqBlock = 256;      // 4 waves
constexpr int kWinWords = 64;      // words per window (one per lane)

__device__ __forceinline__ float load_act(const void* B, size_t idx, bool f16)
{
    return f16 ? (float)reinterpret_cast<const _Float16*>(B)[idx] : reinterpret_cast<const float*>(B)[idx];
}

__device__ __forceinline__ void store_out(void* Y, size_t idx, float v, bool f16)
{
    if (f16) reinterpret_cast<_Float16*>(Y)[idx] = (_Float16)v;
    else reinterpret_cast<float*>(Y)[idx] = v;
}

typedef float v2f __attribute__((ext_vector_type(2)));

// Four trits as floats from c4 = (word >> 2j) & 0x03030303 (byte bb = code of k = 4bb + j):
// v_perm looks the codes up in a byte table of fp8 (E4M3) encodings {-, -1.0, 0.0, +1.0}
// and v_cvt_pk_f32_fp8 widens two bytes at a time; the values are exact.
constexpr uint32_t kFp8Trits = 0x3800B800u;  // byte 1: 0xB8 = -1.0, byte 2: 0x00, byte 3: 0x38 = +1.0
__device__ __forceinline__ void trits4(uint32_t c4, float (&t)[4])
{
    const uint32_t f8 = __builtin_amdgcn_perm(0u, kFp8Trits, c4);
    const v2f lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)f8, false);
    const v2f hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)f8, true);
    t[0] = lo[0];
    t[1] = lo[1];
    t[2] = hi[0];
    t[3] = hi[1];
}

// ---------------------------------------------------------------- matmul_q

// Wave item = (16-row tile, chunk of words). part == nullptr: one chunk, write tau * sum to Y.
// kscale (nullable): per-k factor applied to the activations, b = fl(kscale[k] * B[k][m]) (the
// transposed product's tau); tau (nullable): per-row output factor.
template <int MT>
__global__ __launch_bounds__(kMqBlock) void k_matmul_q(const uint32_t* __restrict__ wq, const float* __restrict__ tau,
                                                       const float* __restrict__ kscale, const void* __restrict__ B,
                                                       bool b16, int N, int K, int M, int n_chunks, int chunk_words,
                                                       float* __restrict__ part, void* __restrict__ Y, bool y16)
{
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(blockIdx.x * (kMqBlock / kWave) + (threadIdx.x >> 6));
    const int n_tiles = (N + 15) / 16;
    if (wv >= n_tiles * n_chunks) return;
    const int t = wv / n_chunks, c = wv % n_chunks;
    const int m0 = blockIdx.y * MT;
    const int wpr = (K + 15) / 16;
    const int cbeg = c * chunk_words, cend = min(cbeg + chunk_words, wpr);

    float acc[16][MT];
#pragma unroll
    for (int r = 0; r < 16; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[r][m] = 0.0f;

    for (int w0 = cbeg; w0 < cend; w0 += kWinWords)
    {
        // activations of this lane's two words (16 k each) for the MT tokens
        float b[1][16][MT];
#pragma unroll
        for (int u = 0; u < 1; ++u)
        {
            const int w = w0 + lane + 64 * u;
#pragma unroll
            for (int i = 0; i < 16; ++i)
            {
                const int k = 16 * w + i;
#pragma unroll
                for (int m = 0; m < MT; ++m)
                {
                    const bool ok = w < cend && k < K && m0 + m < M;
                    const float v = ok ? load_act(B, (size_t)k * M + m0 + m, b16) : 0.0f;
                    b[u][i][m] = (kscale && ok) ? kscale[k] * v : v;
                }
            }
        }
        // the window's 16 words per lane (one per row) are all loaded before the math
        uint32_t wds[16][1];
#pragma unroll
        for (int r = 0; r < 16; ++r)
#pragma unroll
            for (int u = 0; u < 1; ++u)
            {
                const int n = 16 * t + r, w = w0 + lane + 64 * u;  // rows past N read as trit 0
                wds[r][u] = (w < cend && n < N) ? wq[(size_t)n * wpr + w] : 0xAAAAAAAAu;  // code 2 = trit 0
            }
#pragma unroll
        for (int r = 0; r < 16; ++r)
        {
            const uint32_t* wd = wds[r];
#pragma unroll
            for (int u = 0; u < 1; ++u)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                {
                    float tf[4];
                    trits4((wd[u] >> (2 * j)) & 0x03030303u, tf);  // tf[bb]: trit of k = 4bb + j
#pragma unroll
                    for (int bb = 0; bb < 4; ++bb)
#pragma unroll
                        for (int m = 0; m < MT; ++m)
                            acc[r][m] = __builtin_fmaf(tf[bb], b[u][4 * bb + j][m], acc[r][m]);
                }
        }
    }

    // transpose-reduce: after the offsets 32, 16, 8, 4 lane l holds row l / 4 summed over the 16
    // lanes that share l % 4; the offsets 2, 1 finish the sum over all 64 lanes.
#pragma unroll
    for (int s = 0; s < 4; ++s)
    {
        const int off = 32 >> s, half = 8 >> s;
        const bool upper = (lane & off) != 0;
#pragma unroll
        for (int r = 0; r < half; ++r)
#pragma unroll
            for (int m = 0; m < MT; ++m)
            {
                const float keep = upper ? acc[r + half][m] : acc[r][m];
                const float send = upper ? acc[r][m] : acc[r + half][m];
                acc[r][m] = keep + __shfl_xor(send, off, kWave);
            }
    }
#pragma unroll
    for (int m = 0; m < MT; ++m)
    {
        acc[0][m] += __shfl_xor(acc[0][m], 2, kWave);
        acc[0][m] += __shfl_xor(acc[0][m], 1, kWave);
    }
    const int n = 16 * t + (lane >> 2);
    if ((lane & 3) == 0 && n < N)
    {
#pragma unroll
        for (int m = 0; m < MT; ++m)
        {
            if (m0 + m >= M) break;
            if (part) part[((size_t)c * N + n) * M + m0 + m] = acc[0][m];
            else store_out(Y, (size_t)n * M + m0 + m, tau ? tau[n] * acc[0][m] : acc[0][m], y16);
        }
    }
}

// Y[n][m] = tau[n] * sum_c part[c][n][m], c ascending (tau == nullptr: no scale).
__global__ __launch_bounds__(256) void k_sum_parts(const float* __restrict__ part, int n_chunks, size_t rows,
                                                   size_t cols, const float* __restrict__ tau, void* __restrict__ Y,
                                                   bool y16)
{
    const size_t total = rows * cols;
    for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (size_t)gridDim.x * blockDim.x)
    {
        float s = 0.0f;
        for (int c = 0; c < n_chunks; ++c) s += part[(size_t)c * total + idx];
        store_out(Y, idx, tau ? tau[idx / cols] * s : s, y16);
    }
}

// ---------------------------------------------------------------- matmul_q_t

// Bit transpose of a packed container: A (K, ceil(M/16)) -> At (M, ceil(K/16)), trit (m, k) of
// At = trit (k, m) of A; codes for k >= K are 2 (trit 0). A block moves a tile of 64 stored
// rows x 64 words (1024 m): coalesced loads into LDS, then each output word (one m, 16 rows)
// is gathered from LDS and the 4 words of an m are stored contiguously.
constexpr int kTpRows = 64, kTpWords = 64;
__global__ __launch_bounds__(256) void k_trit_transpose(const uint32_t* __restrict__ A, int K, int M,
                                                        uint32_t* __restrict__ At)
{
    __shared__ uint32_t tile[kTpRows][kTpWords + 1];
    const int wpa = (M + 15) / 16, wpk = (K + 15) / 16;
    const int k0 = blockIdx.y * kTpRows, c0 = blockIdx.x * kTpWords;
    for (int e = threadIdx.x; e < kTpRows * kTpWords; e += 256)
    {
        const int r = e / kTpWords, c = e % kTpWords;
        const int k = k0 + r, col = c0 + c;
        tile[r][c] = (k < K && col < wpa) ? A[(size_t)k * wpa + col] : 0xAAAAAAAAu;
    }
    __syncthreads();
    // output words: m = 16 * c0 + mm (1024 values), kw = k0 / 16 + q (4 values)
    for (int e = threadIdx.x; e < 16 * kTpWords * (kTpRows / 16); e += 256)
    {
        const int q = e % (kTpRows / 16), mm = e / (kTpRows / 16);
        const int m = 16 * c0 + mm, kw = k0 / 16 + q;
        if (m >= M || kw >= wpk) continue;
        const int c = mm / 16, sh = 2 * (mm % 16);
        uint32_t word = 0;
#pragma unroll
        for (int i = 0; i < 16; ++i) word |= ((tile[16 * q + i][c] >> sh) & 3u) << (2 * i);
        At[(size_t)m * wpk + kw] = word;
    }
}

unsigned grid_for(size_t n)
{
    const size_t b = ceil_div(n, (size_t)256);
    return (unsigned)(b < 8192 ? (b < 1 ? 1 : b) : 8192);
}

// Waves to aim for: enough to cover HBM latency on 256 CUs.
constexpr int kTargetWaves = 4096;

int token_block(size_t M) { return M <= 1 ? 1 : M <= 2 ? 2 : 4; }

template <int MT>
void launch_mq(hipStream_t st, const uint32_t* wq, const float* tau, const float* kscale, const void* B, bool b16,
               int N, int K, int M, int n_chunks, int chunk_words, float* part, void* Y, bool y16)
{
    const int n_tiles = (N + 15) / 16;
    const dim3 grid((unsigned)ceil_div((size_t)n_tiles * n_chunks, (size_t)(kMqBlock / kWave)),
                    (unsigned)ceil_div((size_t)M, (size_t)MT));
    hipLaunchKernelGGL(k_matmul_q<MT>, grid, dim3(kMqBlock), 0, st, wq, tau, kscale, B, b16, N, K, M, n_chunks,
                       chunk_words, part, Y, y16);
}

// Y (N, M) = diag(tau) ((trit(wq)) . diag(kscale) B), partial sums in part when the plan splits K
hipError_t run_mq(hipStream_t st, const uint32_t* wq, const float* tau, const float* kscale, const void* B, bool b16,
                  size_t N, size_t K, size_t M, void* Y, bool y16, const MatqPlan& plan, float* part)
{
    float* pp = plan.n_chunks > 1 ? part : nullptr;
    const int mt = token_block(M);
    if (mt == 1)
        launch_mq<1>(st, wq, tau, kscale, B, b16, (int)N, (int)K, (int)M, plan.n_chunks, plan.chunk, pp, Y, y16);
    else if (mt == 2)
        launch_mq<2>(st, wq, tau, kscale, B, b16, (int)N, (int)K, (int)M, plan.n_chunks, plan.chunk, pp, Y, y16);
    else
        launch_mq<4>(st, wq, tau, kscale, B, b16, (int)N, (int)K, (int)M, plan.n_chunks, plan.chunk, pp, Y, y16);
    if (pp)
        hipLaunchKernelGGL(k_sum_parts, dim3(grid_for(N * M)), dim3(256), 0, st, pp, plan.n_chunks, N, M, tau, Y, y16);
    return hipGetLastError();
}

}  // namespace

MatqPlan plan_matmul_q(size_t N, size_t K, size_t M)
{
    MatqPlan p{};
    const size_t wpr = ceil_div(K, 16);
    const size_t items = ceil_div(N, 16) * ceil_div(M, (size_t)token_block(M));
    size_t chunks = ceil_div((size_t)kTargetWaves, items);
    const size_t max_chunks = ceil_div(wpr, (size_t)kWinWords);
    if (chunks > max_chunks) chunks = max_chunks;
    if (chunks < 1) chunks = 1;
    p.chunk = (int)(ceil_div(ceil_div(wpr, chunks), (size_t)kWinWords) * kWinWords);
    p.n_chunks = (int)ceil_div(wpr, (size_t)p.chunk);
    p.part_bytes = p.n_chunks > 1 ? (size_t)p.n_chunks * N * M * sizeof(float) : 0;
    return p;
}

MatqPlan plan_matmul_q_t(size_t K, size_t M, size_t N)
{
    // the transposed product runs as matmul_q over the (M, ceil(K/16)) transposed container,
    // which the scratch holds in front of the partial sums
    MatqPlan p = plan_matmul_q(M, K, N);
    p.at_bytes = round_up(M * ceil_div(K, 16) * sizeof(uint32_t), 256);
    p.part_bytes += p.at_bytes;
    return p;
}

hipError_t launch_matmul_q(hipStream_t st, const uint32_t* wq, const float* tau, const void* B, bool b16, size_t N,
                           size_t K, size_t M, void* Y, bool y16, const MatqPlan& plan, float* part)
{
    if (N == 0 || M == 0) return hipSuccess;
    return run_mq(st, wq, tau, nullptr, B, b16, N, K, M, Y, y16, plan, part);
}

hipError_t launch_trit_transpose(hipStream_t st, const uint32_t* A, size_t K, size_t M, uint32_t* At)
{
    if (K == 0 || M == 0) return hipSuccess;
    const dim3 tgrid((unsigned)ceil_div(ceil_div(M, 16), (size_t)kTpWords), (unsigned)ceil_div(K, (size_t)kTpRows));
    hipLaunchKernelGGL(k_trit_transpose, tgrid, dim3(256), 0, st, A, (int)K, (int)M, At);
    return hipGetLastError();
}

hipError_t launch_matmul_q_t(hipStream_t st, const uint32_t* A, const float* tau, const void* B, bool b16, size_t K,
                             size_t M, size_t N, void* Y, bool y16, const MatqPlan& plan, float* scratch)
{
    if (N == 0 || M == 0) return hipSuccess;
    uint32_t* At = reinterpret_cast<uint32_t*>(scratch);
    float* part = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(scratch) + plan.at_bytes);
    const dim3 tgrid((unsigned)ceil_div(ceil_div(M, 16), (size_t)kTpWords), (unsigned)ceil_div(K, (size_t)kTpRows));
    hipLaunchKernelGGL(k_trit_transpose, tgrid, dim3(256), 0, st, A, (int)K, (int)M, At);
    return run_mq(st, At, nullptr, tau, B, b16, M, K, N, Y, y16, plan, part);
}

}  // namespace nnhip
