/*
 * nn_oracle.c — CPU restatement of the BitLinear W1.58A8 path (TEST INFRASTRUCTURE).
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this
 * library, as the checker or as the timed CPU baseline. The shipped libnn-hip.so never
 * links it. Citations are file:line in the reference repository (neuralnet.cpp v1.18.0).
 *
 * Build: oracle/Makefile, with -ffp-contract=off so that every fp32 multiply and add
 * rounds on its own, as the reference's epilogue order requires.
 */
#include "nn_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ RNG */

uint64_t orc_splitmix64(uint64_t* state)
{
    uint64_t z = (*state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static double orc_unit(uint64_t* st) /* (0, 1] */
{
    return ((double)(orc_splitmix64(st) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
}

static double orc_unit0(uint64_t* st) /* [0, 1) */
{
    return (double)(orc_splitmix64(st) >> 11) * (1.0 / 9007199254740992.0);
}

void orc_fill_uniform(float* out, size_t n, uint64_t seed, float lo, float hi)
{
    uint64_t st = seed;
    for (size_t i = 0; i < n; ++i)
        out[i] = (float)((double)lo + ((double)hi - (double)lo) * orc_unit0(&st));
}

void orc_fill_normal(float* out, size_t n, uint64_t seed, float mean, float stddev)
{
    /* Box-Muller in double; one normal per pair of uniforms (simple and deterministic). */
    uint64_t st = seed;
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t i = 0; i < n; ++i)
    {
        const double u1 = orc_unit(&st);
        const double u2 = orc_unit(&st);
        const double z = sqrt(-2.0 * log(u1)) * cos(two_pi * u2);
        out[i] = (float)((double)mean + (double)stddev * z);
    }
}

/* ------------------------------------------------------- nn::trit_pack */

/* words_per_row(K) = ceil(K/16): src/ternary_gemm_test.cpp:74-77 */
size_t orc_trit_words_per_row(size_t K) { return (K + 15) / 16; }

/* code_of(w, tau): 3 if w > 0.5*tau, 1 if w < -0.5*tau, else 2 (ties and NaN -> 2).
 * src/ternary_gemm_test.cpp:79-89 (tau=1 KAT), include/neuralnet.cpp/compute_layer_bitlinear.hpp:657-667
 * (strict |W| > 0.5 tau threshold). 0.5f*tau is exact in fp32. */
uint32_t orc_trit_code(float w, float tau)
{
    const float h = 0.5f * tau;
    if (w > h) return 3u;
    if (w < -h) return 1u;
    return 2u;
}

/* pack_row: trit j of the row at (word[j/16] >> 2*(j%16)) & 3, tail codes 2.
 * src/ternary_gemm_test.cpp:79-99 and :224-251 (engine trit_pack == host pack_row). */
void orc_trit_pack_row(const float* w, size_t K, float tau, uint32_t* words)
{
    const size_t wpr = orc_trit_words_per_row(K);
    for (size_t wi = 0; wi < wpr; ++wi)
    {
        uint32_t word = 0;
        for (size_t j = 0; j < 16; ++j)
        {
            const size_t k = wi * 16 + j;
            const uint32_t code = (k < K) ? orc_trit_code(w[k], tau) : 2u;
            word |= code << (2 * j);
        }
        words[wi] = word;
    }
}

void orc_trit_pack(const float* W, const float* tau, size_t N, size_t K, uint32_t* out)
{
    const size_t wpr = orc_trit_words_per_row(K);
    for (size_t n = 0; n < N; ++n) orc_trit_pack_row(W + n * K, K, tau[n], out + n * wpr);
}

/* at(words, i) = value_of(code) = code - 2: src/ternary_gemm_test.cpp:91-99 */
int orc_trit_at(const uint32_t* words, size_t i)
{
    return (int)((words[i / 16] >> (2 * (i % 16))) & 3u) - 2;
}

/* --------------------------------------------------------- absmean tau */

/* tau_o = sum_k fl(|W_ok| * fl(1/K)): include/neuralnet.cpp/compute_layer_bitlinear.hpp:627-640
 * (row_reduce_sum(abs(W) * rparam(1/K))). The summation order inside the reference engine is
 * not available; this build fixes one order, shared with the GPU kernel: 64 lanes, lane l sums
 * k = l, l+64, ... in ascending order, then a xor butterfly over offsets 32,16,8,4,2,1. */
void orc_row_absmean(const float* W, size_t N, size_t K, float* tau)
{
    const float inv_k = 1.0f / (float)K;
    for (size_t n = 0; n < N; ++n)
    {
        float p[64];
        for (int l = 0; l < 64; ++l)
        {
            float acc = 0.0f;
            for (size_t k = (size_t)l; k < K; k += 64)
            {
                const float t = fabsf(W[n * K + k]) * inv_k;
                acc = acc + t;
            }
            p[l] = acc;
        }
        for (int off = 32; off >= 1; off >>= 1)
        {
            float q[64];
            for (int l = 0; l < 64; ++l) q[l] = p[l] + p[l ^ off];
            memcpy(p, q, sizeof p);
        }
        tau[n] = p[0];
    }
}

/* ---------------------------------------------------------- nn::i8_pack */

size_t orc_i8_words_per_row(size_t cols) { return (cols + 3) / 4; }

/* q = round_half_away(clamp(x/s, -127, 127)); NaN -> 0; s == 0 -> 0.
 * docs/internal/21-quantized-weights.md:973-975; src/int8_act_test.cpp:86-137.
 * x/s is a true IEEE division (the docs' formula). */
int8_t orc_quantize_one(float x, float s)
{
    if (s == 0.0f || x != x) return 0;
    float v = x / s;
    if (v != v) return 0;
    if (v > 127.0f) v = 127.0f;
    if (v < -127.0f) v = -127.0f;
    return (int8_t)roundf(v);
}

/* max_k |X[k][m]| per column, starting from 0 and ignoring NaN (a NaN never compares greater).
 * src/int8_act_test.cpp:95-101 / src/layer_bench.cpp:609-615. */
void orc_col_absmax(const float* X, size_t rows, size_t cols, float* mx)
{
    for (size_t c = 0; c < cols; ++c)
    {
        float m = 0.0f;
        for (size_t r = 0; r < rows; ++r)
        {
            const float a = fabsf(X[r * cols + c]);
            if (a > m) m = a;
        }
        mx[c] = m;
    }
}

/* s = col_reduce_max(|X|) * fl(1/127): include/neuralnet.cpp/compute_layer_bitlinear.hpp:443-447
 * (scale_inplace multiplies by the rounded reciprocal; it does not divide). */
void orc_act_scale(const float* X, size_t rows, size_t cols, float* s)
{
    orc_col_absmax(X, rows, cols, s);
    const float r127 = 1.0f / 127.0f;
    for (size_t c = 0; c < cols; ++c) s[c] = s[c] * r127;
}

/* quantize_i8(x (rows, cols), scale, col_scale) -> (rows, ceil(cols/4)) words, byte c%4 of
 * word c/4 (little-endian within the word), tail bytes 0. col_scale: scale is (1, cols),
 * else (rows, 1). docs/internal/21-quantized-weights.md:973-975, src/int8_act_test.cpp:106-136 */
void orc_quantize_i8(const float* x, const float* scale, size_t rows, size_t cols, int col_scale,
                     uint32_t* out)
{
    const size_t wpr = orc_i8_words_per_row(cols);
    for (size_t r = 0; r < rows; ++r)
        for (size_t wi = 0; wi < wpr; ++wi)
        {
            uint32_t word = 0;
            for (size_t b = 0; b < 4; ++b)
            {
                const size_t c = wi * 4 + b;
                if (c >= cols) break;
                const float s = col_scale ? scale[c] : scale[r];
                const int8_t q = orc_quantize_one(x[r * cols + c], s);
                word |= (uint32_t)(uint8_t)q << (8 * b);
            }
            out[r * wpr + wi] = word;
        }
}

int orc_i8_at(const uint32_t* words, size_t i)
{
    return (int)(int8_t)(uint8_t)((words[i / 4] >> (8 * (i % 4))) & 0xFFu);
}

/* unpack_i8(packed (rows, ceil(cols/4)), cols) -> f32 integers: src/int8_act_test.cpp:140-168 */
void orc_unpack_i8(const uint32_t* packed, size_t rows, size_t cols, float* out)
{
    const size_t wpr = orc_i8_words_per_row(cols);
    for (size_t r = 0; r < rows; ++r)
        for (size_t c = 0; c < cols; ++c) out[r * cols + c] = (float)orc_i8_at(packed + r * wpr, c);
}

/* ---------------------------------------------------------- matmul_q_i8 */

/* acc[n][m] = sum_k value_of(code(n,k)) * q(k,m), k ascending, int32:
 * src/int8_act_test.cpp:210-236 */
void orc_matmul_q_i8_acc(const uint32_t* wq, const uint32_t* xq, size_t N, size_t K, size_t M,
                         int32_t* acc)
{
    const size_t wpr_w = orc_trit_words_per_row(K);
    const size_t wpr_q = orc_i8_words_per_row(M);
    for (size_t n = 0; n < N; ++n)
        for (size_t m = 0; m < M; ++m)
        {
            int32_t a = 0;
            for (size_t k = 0; k < K; ++k)
                a += orc_trit_at(wq + n * wpr_w, k) * orc_i8_at(xq + k * wpr_q, m);
            acc[n * M + m] = a;
        }
}

/* Y[n][m] = (tau_n * s_m) * float(acc): the epilogue order of src/int8_act_test.cpp:233
 * (left-to-right: the two scales multiply first, then the converted accumulator). */
void orc_matmul_q_i8(const uint32_t* wq, const float* tau, const uint32_t* xq, const float* s,
                     size_t N, size_t K, size_t M, float* Y)
{
    int32_t* acc = (int32_t*)malloc(sizeof(int32_t) * ((N * M) != 0 ? N * M : 1));
    orc_matmul_q_i8_acc(wq, xq, N, K, M, acc);
    for (size_t n = 0; n < N; ++n)
        for (size_t m = 0; m < M; ++m)
        {
            const float ts = tau[n] * s[m];
            Y[n * M + m] = ts * (float)acc[n * M + m];
        }
    free(acc);
}

/* CpuEngine restatement (AGENTS.md:178-179; docs/internal/21-quantized-weights.md:794-798):
 * decode RB=64 weight rows into f32 scratch, decode the int8 activations once, then a dense
 * f32 dot-product microkernel. Every partial sum is an integer of magnitude <= 127*K < 2^24,
 * so the f32 arithmetic is exact and the result is bit-identical to the int32 loop.
 * Returns 0, or -1 when 127*K >= 2^24 (exactness would not hold). */
int orc_matmul_q_i8_rowblock(const uint32_t* wq, const float* tau, const uint32_t* xq,
                             const float* s, size_t N, size_t K, size_t M, float* Y, int threads)
{
    if ((double)K * 127.0 >= 16777216.0) return -1;
    enum { RB = 64 };
    const size_t wpr_w = orc_trit_words_per_row(K);
    const size_t wpr_q = orc_i8_words_per_row(M);
    /* activations decoded token-major (M, K) so the microkernel is a unit-stride dot */
    float* xd = (float*)malloc(sizeof(float) * ((M * K) != 0 ? M * K : 1));
    for (size_t k = 0; k < K; ++k)
        for (size_t m = 0; m < M; ++m) xd[m * K + k] = (float)orc_i8_at(xq + k * wpr_q, m);
    const long nblocks = (long)((N + RB - 1) / RB);
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel
#endif
    {
        float* wd = (float*)malloc(sizeof(float) * RB * (K ? K : 1));
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
        for (long blk = 0; blk < nblocks; ++blk)
        {
            const size_t n0 = (size_t)blk * RB;
            const size_t nb = (N - n0 < RB) ? N - n0 : RB;
            for (size_t r = 0; r < nb; ++r)
            {
                const uint32_t* row = wq + (n0 + r) * wpr_w;
                float* dst = wd + r * K;
                for (size_t wi = 0; wi < wpr_w; ++wi)
                {
                    const uint32_t word = row[wi];
                    const size_t kend = (wi * 16 + 16 < K) ? 16 : K - wi * 16;
                    for (size_t j = 0; j < kend; ++j)
                        dst[wi * 16 + j] = (float)((int)((word >> (2 * j)) & 3u) - 2);
                }
            }
            for (size_t r = 0; r < nb; ++r)
            {
                const float* wrow = wd + r * K;
                for (size_t m = 0; m < M; ++m)
                {
                    const float* xrow = xd + m * K;
                    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f, a4 = 0.f, a5 = 0.f, a6 = 0.f,
                          a7 = 0.f;
                    size_t k = 0;
                    for (; k + 8 <= K; k += 8)
                    {
                        a0 += wrow[k + 0] * xrow[k + 0];
                        a1 += wrow[k + 1] * xrow[k + 1];
                        a2 += wrow[k + 2] * xrow[k + 2];
                        a3 += wrow[k + 3] * xrow[k + 3];
                        a4 += wrow[k + 4] * xrow[k + 4];
                        a5 += wrow[k + 5] * xrow[k + 5];
                        a6 += wrow[k + 6] * xrow[k + 6];
                        a7 += wrow[k + 7] * xrow[k + 7];
                    }
                    for (; k < K; ++k) a0 += wrow[k] * xrow[k];
                    const float acc = ((a0 + a1) + (a2 + a3)) + ((a4 + a5) + (a6 + a7));
                    const float ts = tau[n0 + r] * s[m];
                    Y[(n0 + r) * M + m] = ts * acc;
                }
            }
        }
        free(wd);
    }
    free(xd);
    return 0;
}

/* y + b (row broadcast): include/neuralnet.cpp/compute_layer_bitlinear.hpp:455-456 */
void orc_add_row_broadcast(float* Y, const float* b, size_t N, size_t M)
{
    for (size_t n = 0; n < N; ++n)
        for (size_t m = 0; m < M; ++m) Y[n * M + m] = Y[n * M + m] + b[n];
}

/* ------------------------------------------------- float-activation GEMM */

/* matmul_q: Y (N, M) = (tau o trit(wq)) . B, accumulated in double and rounded once to float,
 * the host reference of src/ternary_gemm_test.cpp:141-154 (ref_gemm, transA = 0):
 * acc += (double)(tau[m] * trit) * (double)B[k][n]. tau * trit is exact (trit in {-1,0,1}). */
void orc_matmul_q(const uint32_t* wq, const float* tau, const float* B, size_t N, size_t K, size_t M,
                  float* Y)
{
    const size_t wpr = (K + 15) / 16;
    for (size_t n = 0; n < N; ++n)
        for (size_t m = 0; m < M; ++m)
        {
            double acc = 0.0;
            for (size_t k = 0; k < K; ++k)
            {
                const int code = (int)((wq[n * wpr + k / 16] >> (2 * (k % 16))) & 3u);
                const float tw = tau[n] * (float)(code - 2);
                acc += (double)tw * (double)B[k * M + m];
            }
            Y[n * M + m] = (float)acc;
        }
}

/* matmul_q_t: Y (M, N) = (tau o trit(A))^T . B with A (K, ceil(M/16)) one stored row per k and
 * tau per stored row, src/ternary_gemm_test.cpp:155-169 (ref_gemm, transA = 1). */
void orc_matmul_q_t(const uint32_t* A, const float* tau, const float* B, size_t K, size_t M, size_t N,
                    float* Y)
{
    const size_t wpa = (M + 15) / 16;
    for (size_t m = 0; m < M; ++m)
        for (size_t n = 0; n < N; ++n)
        {
            double acc = 0.0;
            for (size_t k = 0; k < K; ++k)
            {
                const int code = (int)((A[k * wpa + m / 16] >> (2 * (m % 16))) & 3u);
                const float tw = tau[k] * (float)(code - 2);
                acc += (double)tw * (double)B[k * N + n];
            }
            Y[m * N + n] = (float)acc;
        }
}

/* -------------------------------------------------------------- RMSNorm */

/* The per-token sum of squares uses a fixed order shared with every GPU kernel: 512 strided
 * parts (feature f goes to part f % 512), each summed in ascending f, then the xor butterfly
 * over offsets 256,128,...,1. (The reference evaluates this reduction inside its JIT engine,
 * whose order is not available; any fixed order is as faithful, and this one lets a GPU
 * thread own whole parts whether it holds one token per wave or 4-8 tokens per block.) */
static float orc_rms_inv(const float* X, float eps, size_t F, size_t M, size_t m)
{
    float p[512];
    for (int l = 0; l < 512; ++l)
    {
        float part = 0.0f;
        for (size_t f = (size_t)l; f < F; f += 512)
        {
            const float x = X[f * M + m];
            const float sq = x * x;
            part = part + sq;
        }
        p[l] = part;
    }
    for (int off = 256; off >= 1; off >>= 1)
    {
        float q[512];
        for (int l = 0; l < 512; ++l) q[l] = p[l] + p[l ^ off];
        memcpy(p, q, sizeof p);
    }
    const float inv_f = 1.0f / (float)F;
    const float ms = p[0] * inv_f;
    const float v = ms + eps;
    return 1.0f / sqrtf(v);
}

/* RMSNorm forward: include/neuralnet.cpp/compute_layer_mlp.hpp:615-619 and :686-707:
 * rms_inv = 1/sqrt(sum_f x^2 * (1/F) + eps); normed = x * rms_inv; out = normed * gamma. */
void orc_rmsnorm(const float* X, const float* gamma, float eps, size_t F, size_t M, float* out)
{
    for (size_t m = 0; m < M; ++m)
    {
        const float ri = orc_rms_inv(X, eps, F, M, m);
        for (size_t f = 0; f < F; ++f)
        {
            const float nrm = X[f * M + m] * ri;
            out[f * M + m] = nrm * gamma[f];
        }
    }
}

/* LayerNorm forward: include/neuralnet.cpp/compute_layer_mlp.hpp:529-545 (the SubLN norm type
 * FeedForward defaults to, compute_layer_feedforward.hpp:50-65):
 * mean = sum_f x * fl(1/F); d = x - mean; sinv = rsqrt(sum_f d*d * fl(1/F) + eps);
 * out = (d * sinv) * gamma + beta, rsqrt as 1/sqrtf (the RMSNorm convention above). The two sums
 * use the order of the GPU kernel: 8 strided parts (f % 8), each ascending, then the tree
 * ((p0 + p1) + (p2 + p3)) + ((p4 + p5) + (p6 + p7)). The reference's engine order is not
 * available; tests pin this restatement against a float64 evaluation and exact special cases. */
static float orc_tree8(const float* v)
{
    const float a = (v[0] + v[1]) + (v[2] + v[3]);
    const float b = (v[4] + v[5]) + (v[6] + v[7]);
    return a + b;
}

void orc_layernorm(const float* X, const float* gamma, const float* beta, float eps, size_t F, size_t M,
                   float* out)
{
    const float inv_f = 1.0f / (float)F;
    for (size_t m = 0; m < M; ++m)
    {
        float p[8];
        for (int l = 0; l < 8; ++l)
        {
            float part = 0.0f;
            for (size_t f = (size_t)l; f < F; f += 8) part = part + X[f * M + m];
            p[l] = part;
        }
        const float mean = orc_tree8(p) * inv_f;
        for (int l = 0; l < 8; ++l)
        {
            float part = 0.0f;
            for (size_t f = (size_t)l; f < F; f += 8)
            {
                const float d = X[f * M + m] - mean;
                const float sq = d * d;
                part = part + sq;
            }
            p[l] = part;
        }
        const float var = orc_tree8(p) * inv_f;
        const float v = var + eps;
        const float sinv = 1.0f / sqrtf(v);
        for (size_t f = 0; f < F; ++f)
        {
            const float d = X[f * M + m] - mean;
            const float nrm = d * sinv;
            const float g = nrm * gamma[f];
            out[f * M + m] = g + beta[f];
        }
    }
}

/* RMSNorm -> per-token absmax scale -> int8, the three steps of
 * include/neuralnet.cpp/compute_layer_mlp.hpp:686-707 followed by
 * include/neuralnet.cpp/compute_layer_bitlinear.hpp:443-448, on the normed values.
 * xq in the reference container layout (F, ceil(M/4)); s is (1, M). */
void orc_rmsnorm_quant_i8(const float* X, const float* gamma, float eps, size_t F, size_t M,
                          uint32_t* xq, float* s)
{
    float* tmp = (float*)malloc(sizeof(float) * ((F * M) != 0 ? F * M : 1));
    orc_rmsnorm(X, gamma, eps, F, M, tmp);
    orc_act_scale(tmp, F, M, s);
    orc_quantize_i8(tmp, s, F, M, 1, xq);
    free(tmp);
}

/* ---------------------------------------------- MI355X tile layout (repack) */

/* Layout T16K256 (this build's own format, no reference counterpart):
 *   rows padded to Np = roundup(N,16), k padded to Kp = roundup(K,256);
 *   tile (rt, kt) of 16 rows x 256 k = 256 words (1 KiB) at word offset (rt*KT + kt)*256;
 *   inside a tile, lane l = 16*g + r (g in 0..3, r in 0..15) owns the 4 words 4*l + q;
 *   bit 8*b + 2*j of word q of lane l holds the code of
 *       row 16*rt + r,  k = 256*kt + 64*j + 16*g + 4*q + b      (j, q, b in 0..3).
 * So (word_q >> 2j) & 0x03030303 gives, in byte b, the code for k = 256kt+64j+16g+4q+b:
 * the four words shifted by 2j are the 16 A-operand bytes of one 16x16x64 int8 MFMA whose
 * B operand is 16 consecutive activation bytes starting at k = 256kt + 64j + 16g.
 * Codes for k in [K, roundup(K,16)) are copied from the source tail, codes beyond are 2. */
size_t orc_repacked_words(size_t N, size_t K)
{
    const size_t Np = (N + 15) / 16 * 16, Kp = (K + 255) / 256 * 256;
    return Np * Kp / 16;
}

static uint32_t orc_src_code(const uint32_t* wq, size_t N, size_t K, size_t n, size_t k)
{
    const size_t wpr = orc_trit_words_per_row(K);
    if (n >= N || k >= wpr * 16) return 2u;
    return (wq[n * wpr + k / 16] >> (2 * (k % 16))) & 3u;
}

void orc_repack(const uint32_t* wq, size_t N, size_t K, uint32_t* out)
{
    const size_t RT = (N + 15) / 16, KT = (K + 255) / 256;
    for (size_t rt = 0; rt < RT; ++rt)
        for (size_t kt = 0; kt < KT; ++kt)
            for (size_t l = 0; l < 64; ++l)
                for (size_t q = 0; q < 4; ++q)
                {
                    const size_t g = l / 16, r = l % 16;
                    uint32_t word = 0;
                    for (size_t j = 0; j < 4; ++j)
                        for (size_t b = 0; b < 4; ++b)
                        {
                            const size_t k = 256 * kt + 64 * j + 16 * g + 4 * q + b;
                            const uint32_t code = orc_src_code(wq, N, K, 16 * rt + r, k);
                            word |= code << (8 * b + 2 * j);
                        }
                    out[(rt * KT + kt) * 256 + 4 * l + q] = word;
                }
}

void orc_unrepack(const uint32_t* rp, size_t N, size_t K, uint32_t* wq)
{
    const size_t KT = (K + 255) / 256;
    const size_t wpr = orc_trit_words_per_row(K);
    for (size_t n = 0; n < N; ++n)
        for (size_t wi = 0; wi < wpr; ++wi)
        {
            uint32_t word = 0;
            for (size_t e = 0; e < 16; ++e)
            {
                const size_t k = wi * 16 + e;
                const size_t rt = n / 16, r = n % 16, kt = k / 256, kk = k % 256;
                const size_t j = kk / 64, g = (kk % 64) / 16, q = (kk % 16) / 4, b = kk % 4;
                const size_t l = 16 * g + r;
                const uint32_t src = rp[(rt * KT + kt) * 256 + 4 * l + q];
                const uint32_t code = (src >> (8 * b + 2 * j)) & 3u;
                word |= code << (2 * e);
            }
            wq[n * wpr + wi] = word;
        }
}

/* ------------------------------------------ gated activations and the FFN block */

/* exp(x) in fp32 built from IEEE-rounded operations only (no fused multiply-add), so a GPU
 * kernel that performs the same operations in the same order reproduces every bit:
 *   k = rint(x * fl(1/ln2));  r = (x - k*L1) - k*L2   (L1 = 22713/32768 has 15 significant
 *   bits, so k*L1 is exact for |k| < 256 and x - k*L1 is exact by Sterbenz; L2 = fl(ln2 - L1));
 *   e^r by its Taylor series to r^7 in Horner form (|r| <= 0.3466: truncation below 6e-9
 *   relative, under half an ulp);  result = ldexp(p, k).
 * x > 100 gives +inf (k would overflow int), x < -87 gives 0 (results below FLT_MIN are
 * flushed: the gated activations only use exp(-g) inside 1 + exp(-g), where such values
 * vanish anyway). NaN propagates. Checked against float64 exp to within 2 ulp in the tests. */
float orc_exp(float x)
{
    if (x != x) return x;
    if (x > 100.0f) return INFINITY;
    if (x < -87.0f) return 0.0f;
    const float inv_ln2 = 0x1.715476p+0f;
    const float ln2_hi = 0x1.62e4p-1f;
    const float ln2_lo = 0x1.7f7d1cp-20f;
    const float k = rintf(x * inv_ln2);
    const float r = (x - k * ln2_hi) - k * ln2_lo;
    float p = 0x1.a01a02p-13f;  /* 1/7! */
    p = p * r + 0x1.6c16c2p-10f; /* 1/6! */
    p = p * r + 0x1.111112p-7f;  /* 1/5! */
    p = p * r + 0x1.555556p-5f;  /* 1/4! */
    p = p * r + 0x1.555556p-3f;  /* 1/3! */
    p = p * r + 0.5f;
    p = p * r + 1.0f;
    p = p * r + 1.0f;
    return ldexpf(p, (int)k);
}

void orc_exp_array(const float* x, size_t n, float* out)
{
    for (size_t i = 0; i < n; ++i) out[i] = orc_exp(x[i]);
}

/* One gated activation (act 0 = SwiGLU, 1 = ReLU^2-GLU), in the reference's evaluation order:
 *   SwiGLU   (g * (1 / (1 + exp(-g)))) * u   include/neuralnet.cpp/compute_layer_mlp.hpp:317-328
 *   ReLU2GLU (r * r) * u, r = g > 0 ? g : 0  include/neuralnet.cpp/compute_layer_mlp.hpp:405-414 */
float orc_glu_one(float g, float u, int act)
{
    if (act == 1)
    {
        const float r = g > 0.0f ? g : 0.0f;
        return (r * r) * u;
    }
    const float sig = 1.0f / (1.0f + orc_exp(-g));
    return (g * sig) * u;
}

/* in (2F, M): gate = rows [0, F), up = rows [F, 2F) (the SwiGLU/ReLU2GLU row split of the
 * fused fc1 output, compute_layer_mlp.hpp:323-325); out (F, M). */
void orc_glu(const float* in, size_t F, size_t M, int act, float* out)
{
    for (size_t f = 0; f < F; ++f)
        for (size_t m = 0; m < M; ++m) out[f * M + m] = orc_glu_one(in[f * M + m], in[(F + f) * M + m], act);
}

/* Row order of the interleaved ("GLU") layout of a fused gate/up weight (this build's own
 * format): 16-row group t holds gate rows 8t .. 8t+7, then up rows 8t .. 8t+7, so one
 * 16-row tile carries both inputs of 8 features. Returns the reference row (in [0, 2F)) of
 * interleaved row r, or -1 for padding rows (features >= F). Interleaved rows: 2*roundup(F, 8). */
long orc_glu_src_row(size_t r, size_t F)
{
    const size_t t = r / 16, i = r % 16;
    const size_t f = 8 * t + (i % 8);
    if (f >= F) return -1;
    return (long)(i < 8 ? f : F + f);
}

/* Reference container wq (2F, ceil(K/16)) + tau/bias (2F) -> interleaved container rows
 * (2*roundup(F,8), ceil(K/16)) and tau/bias in the same order (padding: code 2, tau 0, bias 0). */
void orc_glu_interleave(const uint32_t* wq, const float* tau, const float* bias, size_t F, size_t K,
                        uint32_t* wq_out, float* tau_out, float* bias_out)
{
    const size_t wpr = orc_trit_words_per_row(K), rows = 2 * ((F + 7) / 8 * 8);
    for (size_t r = 0; r < rows; ++r)
    {
        const long src = orc_glu_src_row(r, F);
        for (size_t w = 0; w < wpr; ++w) wq_out[r * wpr + w] = src < 0 ? 0xAAAAAAAAu : wq[(size_t)src * wpr + w];
        tau_out[r] = src < 0 ? 0.0f : tau[src];
        if (bias_out) bias_out[r] = (src < 0 || !bias) ? 0.0f : bias[src];
    }
}

/* BitLinear int8 forward (include/neuralnet.cpp/compute_layer_bitlinear.hpp:441-457) on an
 * already computed per-token scale: y = (tau * s) * float(acc) [+ b as a separate rounding]. */
static void orc_bitlinear_i8(const float* x, size_t K, size_t M, const uint32_t* wq, const float* tau,
                             const float* b, size_t N, int threads, float* y)
{
    float* s = (float*)malloc(sizeof(float) * (M ? M : 1));
    uint32_t* xq = (uint32_t*)malloc(sizeof(uint32_t) * (K * orc_i8_words_per_row(M) + 1));
    orc_act_scale(x, K, M, s);
    orc_quantize_i8(x, s, K, M, 1, xq);
    if (orc_matmul_q_i8_rowblock(wq, tau, xq, s, N, K, M, y, threads) != 0) orc_matmul_q_i8(wq, tau, xq, s, N, K, M, y);
    if (b) orc_add_row_broadcast(y, b, N, M);
    free(xq);
    free(s);
}

/* The W1.58A8 gated feed-forward block of config C4, as the reference composes it
 * (FeedForward::forward, include/neuralnet.cpp/compute_layer_feedforward.hpp:182-204, with the
 * int8 BitLinear forward for fc1 and fc2), preceded by the block's RMSNorm
 * (compute_layer_mlp.hpp:686-707) when gamma is not NULL:
 *   x1 = rmsnorm(X, gamma, eps) (d, M);  y1 = fc1(x1) (2F, M);  h = glu(y1) (F, M);
 *   Y  = fc2(h) (d, M).
 * wq1 (2F, ceil(d/16)) and wq2 (d, ceil(F/16)) are reference containers; b1/b2 may be NULL.
 * h_out (F, M) receives the gated activation if not NULL. */
void orc_ffn_glu_i8(const float* X, const float* gamma, float eps, size_t d, size_t F, size_t M, int act,
                    const uint32_t* wq1, const float* tau1, const float* b1, const float* gamma_sub,
                    float eps_sub, const uint32_t* wq2, const float* tau2, const float* b2, int threads,
                    float* h_out, float* Y)
{
    float* x1 = (float*)malloc(sizeof(float) * (d * M + 1));
    float* y1 = (float*)malloc(sizeof(float) * (2 * F * M + 1));
    float* h = (float*)malloc(sizeof(float) * (F * M + 1));
    float* hn = gamma_sub ? (float*)malloc(sizeof(float) * (F * M + 1)) : NULL;
    if (gamma) orc_rmsnorm(X, gamma, eps, d, M, x1);
    else memcpy(x1, X, sizeof(float) * d * M);
    orc_bitlinear_i8(x1, d, M, wq1, tau1, b1, 2 * F, threads, y1);
    orc_glu(y1, F, M, act, h);
    if (h_out) memcpy(h_out, h, sizeof(float) * F * M);
    /* SubLN: RMSNorm of the gated output before fc2 (compute_layer_feedforward.hpp:201-206) */
    if (gamma_sub) orc_rmsnorm(h, gamma_sub, eps_sub, F, M, hn);
    orc_bitlinear_i8(gamma_sub ? hn : h, F, M, wq2, tau2, b2, d, threads, Y);
    free(hn);
    free(h);
    free(y1);
    free(x1);
}

/* ================================================================ batched decode step */

/* RotaryEmbedding::fill_pos_column_ (include/neuralnet.cpp/compute_position_encoding.hpp:64-80):
 * theta = pos / 10000^(2j/dk) in float, then cos / sin of it; the reference writes each value
 * for j and j + dk/2, this table keeps it once: (max_len, dk/2). */
void orc_rope_table(size_t dk, size_t max_len, float* cos_out, float* sin_out)
{
    const size_t half = dk / 2;
    for (size_t pos = 0; pos < max_len; ++pos)
    {
        const float pd = (float)pos;
        for (size_t j = 0; j < half; ++j)
        {
            const float theta = pd / powf(10000.0f, (float)(2 * j) / (float)dk);
            cos_out[pos * half + j] = cosf(theta);
            sin_out[pos * half + j] = sinf(theta);
        }
    }
}

/* out = x*cos + rotate_half(x)*sin for one head vector (compute_position_encoding.hpp:150-166):
 * rotate_half(x)[j] = -x[j + dk/2] (j < dk/2), x[j - dk/2] (j >= dk/2); every product and the
 * sum are separately rounded. out may not alias x. */
void orc_rope_apply(const float* x, size_t dk, const float* cos_row, const float* sin_row, float* out)
{
    const size_t half = dk / 2;
    for (size_t j = 0; j < half; ++j)
    {
        const float c = cos_row[j], s = sin_row[j];
        const float a = x[j] * c, b = (-x[j + half]) * s;
        out[j] = a + b;
        const float a2 = x[j + half] * c, b2 = x[j] * s;
        out[j + half] = a2 + b2;
    }
}

/* AttentionBase::forward_step steps 1.5-8 (compute_layer_attention.hpp:1022-1083) for B
 * sequences: rotate q and the new key at pos[b] (apply_qk_step), store key and value at row
 * pos[b] (insert_rows), then per query head h (KV head h / (H/Hkv), the gather_rows map of
 * :444-449): scores_t = fl(q_h . K_t) * scale over t <= pos[b] (dot products accumulated in
 * ascending i), softmax exp(s - max) / sum (compute_layer_softmax.hpp:56-66, sum ascending in t),
 * out_i = sum_t attn_t * V_t[i] (ascending t). Layouts as nnhip_attention_decode. cosT == NULL:
 * no rotation. */
/* x rounded to the nearest IEEE binary16 value (ties to even), returned as the float it equals:
 * what a cache of f16 elements stores (compute = F16). Overflow past 65504 gives inf, NaN stays
 * NaN, and below 2^-14 the f16 subnormal quantum 2^-24 applies. */
float orc_round_f16(float x)
{
    uint32_t b;
    memcpy(&b, &x, 4);
    const uint32_t sign = b & 0x80000000u, a = b & 0x7FFFFFFFu;
    if (a >= 0x7F800000u) return x;  /* inf, NaN */
    if (a >= 0x477FF000u)            /* at or past the midpoint of 65504 and 2^16 */
        return sign ? -INFINITY : INFINITY;
    if (a < 0x38800000u)             /* below 2^-14: multiples of 2^-24, exact scaling */
    {
        const float r = rintf(fabsf(x) * 16777216.0f) / 16777216.0f;
        return sign ? -r : r;
    }
    uint32_t r = (a + 0xFFFu + ((a >> 13) & 1u)) & ~0x1FFFu;  /* 10 mantissa bits, ties to even */
    r |= sign;
    float f;
    memcpy(&f, &r, 4);
    return f;
}

void orc_round_f16_n(const float* x, size_t n, float* out)
{
    for (size_t i = 0; i < n; ++i) out[i] = orc_round_f16(x[i]);
}

void orc_attention_decode(const float* q, const float* k, const float* v, size_t B, size_t H, size_t Hkv,
                          size_t dk, const int32_t* pos, const float* cosT, const float* sinT, float* k_cache,
                          float* v_cache, size_t max_len, float scale, float* out)
{
    orc_attention_decode_ct(q, k, v, B, H, Hkv, dk, pos, cosT, sinT, k_cache, v_cache, max_len, scale, 0, out);
}

/* cache_f16: the appended key and value rows are rounded to f16 (orc_round_f16) before they are
 * used, the caches then hold f16 values (as floats), as under compute = F16
 * (include/neuralnet.cpp/compute_layer_gpt.hpp:764-765). */
void orc_attention_decode_ct(const float* q, const float* k, const float* v, size_t B, size_t H, size_t Hkv,
                             size_t dk, const int32_t* pos, const float* cosT, const float* sinT, float* k_cache,
                             float* v_cache, size_t max_len, float scale, int cache_f16, float* out)
{
    const size_t R = H / Hkv, half = dk / 2, row = Hkv * dk;
    float* xbuf = (float*)malloc(dk * sizeof(float));
    float* qr = (float*)malloc(dk * sizeof(float));
    float* sc = (float*)malloc(max_len * sizeof(float));
    for (size_t b = 0; b < B; ++b)
    {
        const int32_t p = pos[b];
        float* kc = k_cache + b * max_len * row;
        float* vc = v_cache + b * max_len * row;
        if (p < 0 || (size_t)p >= max_len)
        {
            for (size_t e = 0; e < H * dk; ++e) out[e * B + b] = NAN;
            continue;
        }
        for (size_t g = 0; g < Hkv; ++g)
        {
            for (size_t i = 0; i < dk; ++i) xbuf[i] = k[(g * dk + i) * B + b];
            if (cosT)
                orc_rope_apply(xbuf, dk, cosT + (size_t)p * half, sinT + (size_t)p * half, kc + (size_t)p * row + g * dk);
            else
                memcpy(kc + (size_t)p * row + g * dk, xbuf, dk * sizeof(float));
            for (size_t i = 0; i < dk; ++i) vc[(size_t)p * row + g * dk + i] = v[(g * dk + i) * B + b];
            if (cache_f16)
                for (size_t i = 0; i < dk; ++i)
                {
                    kc[(size_t)p * row + g * dk + i] = orc_round_f16(kc[(size_t)p * row + g * dk + i]);
                    vc[(size_t)p * row + g * dk + i] = orc_round_f16(vc[(size_t)p * row + g * dk + i]);
                }
        }
        for (size_t h = 0; h < H; ++h)
        {
            const size_t g = h / R;
            for (size_t i = 0; i < dk; ++i) xbuf[i] = q[(h * dk + i) * B + b];
            if (cosT)
                orc_rope_apply(xbuf, dk, cosT + (size_t)p * half, sinT + (size_t)p * half, qr);
            else
                memcpy(qr, xbuf, dk * sizeof(float));
            float m = -INFINITY;
            for (int32_t t = 0; t <= p; ++t)
            {
                const float* kt = kc + (size_t)t * row + g * dk;
                float d = 0.0f;
                for (size_t i = 0; i < dk; ++i)
                {
                    const float pr = qr[i] * kt[i];
                    d = d + pr;
                }
                sc[t] = d * scale;
                if (sc[t] > m) m = sc[t];
            }
            float l = 0.0f;
            for (int32_t t = 0; t <= p; ++t)
            {
                sc[t] = expf(sc[t] - m);
                l = l + sc[t];
            }
            for (int32_t t = 0; t <= p; ++t) sc[t] = sc[t] / l;
            for (size_t i = 0; i < dk; ++i)
            {
                float o = 0.0f;
                for (int32_t t = 0; t <= p; ++t)
                {
                    const float pr = sc[t] * vc[(size_t)t * row + g * dk + i];
                    o = o + pr;
                }
                out[(h * dk + i) * B + b] = o;
            }
        }
    }
    free(xbuf);
    free(qr);
    free(sc);
}

/* gather_rows(token_emb, id) + transpose (compute_layer_gpt.hpp:700-704) for B ids:
 * out (d, B), NaN column for an id outside [0, V). */
void orc_embedding_gather(const float* table, const int32_t* ids, size_t V, size_t d, size_t B, float* out)
{
    for (size_t b = 0; b < B; ++b)
        for (size_t i = 0; i < d; ++i)
            out[i * B + b] = (ids[b] >= 0 && (size_t)ids[b] < V) ? table[(size_t)ids[b] * d + i] : NAN;
}

/* The greedy branch of sample_next_token_ (compute_layer_base.hpp:1152-1160) over
 * logits[v * stride], v < V. */
int32_t orc_argmax(const float* logits, size_t V, size_t stride)
{
    size_t next = 0;
    float best = logits[0];
    for (size_t v = 1; v < V; ++v)
        if (logits[v * stride] > best)
        {
            best = logits[v * stride];
            next = v;
        }
    return (int32_t)next;
}
