/*
 * nn_oracle.h — CPU restatement of neuralnet.cpp's BitLinear W1.58A8 path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the shipped library links, loads or
 * calls this code. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, and only as the checker / the timed CPU baseline.
 *
 * The reference implementation lives in the un-vendored `engine` submodule
 * (compute.neuralnet.cpp @ 2dc4986), so it cannot be built here. Every
 * function below restates the algorithm from the reference's own host-side
 * test loops and call sites; each one cites the file:line it follows
 * (paths relative to the reference repository root).
 *
 * Pinning status per function (what checks it besides its own formula):
 *   orc_trit_code / orc_trit_pack_row / orc_trit_at : KAT src/ternary_gemm_test.cpp:79-99
 *   orc_row_absmean   : KAT src/t1_58_test.cpp:207-252 to 1e-6; ulp order is this
 *                       build's documented order (the reference order is
 *                       unpinned: it lives inside the absent CpuEngine)
 *   orc_quantize_one  : closed form + special cases src/int8_act_test.cpp:86-137;
 *                       tie arithmetic (x/s vs x*(1/s)) is parity unpinned
 *   orc_matmul_q_i8*  : brute force in the tests (int64 numpy) + epilogue order
 *                       src/int8_act_test.cpp:210-236
 *   orc_matmul_q(_t)  : ref_gemm of src/ternary_gemm_test.cpp:141-170 (float64 accumulation);
 *                       checked against numpy float64 products of the decoded trits and the
 *                       reference test's own patterns (:253-334)
 *   orc_rmsnorm*      : textbook formula include/neuralnet.cpp/compute_layer_mlp.hpp:615-619,
 *                       checked against a float64 recomputation within tolerance
 *   orc_layernorm     : LayerNorm::forward (include/neuralnet.cpp/compute_layer_mlp.hpp:529-545),
 *                       checked against a float64 recomputation within tolerance and exact
 *                       special cases (constant token -> beta, F = 1)
 *   orc_repack*       : the MI355X tile layout is this build's own format; pinned by
 *                       the round trip repack -> unrepack == identity
 *   orc_exp           : this build's own fp32 exp (the reference's exp lives in the absent
 *                       engine: ulp-level parity with it is unpinned); checked against float64
 *                       exp to within 2 ulp over a dense sweep and at the range edges
 *   orc_glu*          : the reference's SwiGLU / ReLU2GLU expressions
 *                       (compute_layer_mlp.hpp:317-328, :405-414), checked against float64
 *                       evaluations within tolerance and exact special cases
 *   orc_ffn_glu_i8    : composition of the pinned pieces above in the order of
 *                       FeedForward::forward (compute_layer_feedforward.hpp:182-206, with the
 *                       optional SubLN RMSNorm before fc2); checked against a numpy composition
 *                       (int64 products) in the tests
 *   orc_rope_table    : RotaryEmbedding::fill_pos_column_ (include/neuralnet.cpp/
 *                       compute_position_encoding.hpp:64-80) in float; checked bit for bit
 *                       against libnn-hip.so's host table and against float64 cos/sin
 *   orc_rope_apply    : q*cos + rotate_half(q)*sin (compute_position_encoding.hpp:150-166);
 *                       checked against a float64 complex rotation (z * e^{i theta}) of the
 *                       (j, j + dk/2) pairs and unit-vector cases
 *   orc_attention_decode : AttentionBase::forward_step steps 1.5-8 (compute_layer_attention.hpp:
 *                       1022-1083) per sequence, softmax as Softmax::forward
 *                       (compute_layer_softmax.hpp:56-66); checked against a float64 numpy
 *                       attention, and exactly on the closed forms (one position -> v; equal keys
 *                       -> mean of v) and on a GQA head map with distinct KV heads
 *   orc_round_f16      : the f16 element of a compute = F16 cache (compute_layer_gpt.hpp:764-765);
 *                       checked bit for bit against numpy's float16 conversion over sampled
 *                       float32 bit patterns and every boundary class (overflow, subnormal, ties)
 *   orc_argmax        : the greedy loop of sample_next_token_ (compute_layer_base.hpp:1152-1160)
 */
#ifndef NN_ORACLE_H
#define NN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- deterministic RNG (std::normal_distribution is implementation-defined,
 *      so fixtures use this in-repo generator) ---- */
uint64_t orc_splitmix64(uint64_t* state);
void orc_fill_uniform(float* out, size_t n, uint64_t seed, float lo, float hi);
void orc_fill_normal(float* out, size_t n, uint64_t seed, float mean, float stddev);

/* ---- nn::trit_pack (2 bit / weight, 16 per u32, LSB first, code = trit + 2) ---- */
size_t orc_trit_words_per_row(size_t K);
uint32_t orc_trit_code(float w, float tau);
void orc_trit_pack_row(const float* w, size_t K, float tau, uint32_t* words);
void orc_trit_pack(const float* W, const float* tau, size_t N, size_t K, uint32_t* out);
int orc_trit_at(const uint32_t* words, size_t i);

/* ---- per-row absmean tau (fixed 64-lane order, see nn_oracle.c) ---- */
void orc_row_absmean(const float* W, size_t N, size_t K, float* tau);

/* ---- nn::i8_pack (4 int8 per u32, little-endian, tail bytes 0) ---- */
size_t orc_i8_words_per_row(size_t cols);
int8_t orc_quantize_one(float x, float s);
void orc_col_absmax(const float* X, size_t rows, size_t cols, float* mx);
void orc_act_scale(const float* X, size_t rows, size_t cols, float* s);
void orc_quantize_i8(const float* x, const float* scale, size_t rows, size_t cols, int col_scale,
                     uint32_t* out);
void orc_unpack_i8(const uint32_t* packed, size_t rows, size_t cols, float* out);
int orc_i8_at(const uint32_t* words, size_t i);

/* ---- matmul_q_i8: Y[n,m] = (tau_n * s_m) * float(sum_k trit(n,k) * q(k,m)) ---- */
void orc_matmul_q_i8_acc(const uint32_t* wq, const uint32_t* xq, size_t N, size_t K, size_t M,
                         int32_t* acc);
void orc_matmul_q_i8(const uint32_t* wq, const float* tau, const uint32_t* xq, const float* s,
                     size_t N, size_t K, size_t M, float* Y);
/* CpuEngine restatement: row-block (RB=64) decode to f32 scratch + dense f32
 * microkernel; exact because every partial sum is an integer below 2^24. */
int orc_matmul_q_i8_rowblock(const uint32_t* wq, const float* tau, const uint32_t* xq,
                             const float* s, size_t N, size_t K, size_t M, float* Y, int threads);
void orc_add_row_broadcast(float* Y, const float* b, size_t N, size_t M);
void orc_matmul_q(const uint32_t* wq, const float* tau, const float* B, size_t N, size_t K, size_t M,
                  float* Y);
void orc_matmul_q_t(const uint32_t* A, const float* tau, const float* B, size_t K, size_t M, size_t N,
                    float* Y);

/* ---- RMSNorm and the fused RMSNorm -> absmax -> int8 path ---- */
void orc_rmsnorm(const float* X, const float* gamma, float eps, size_t F, size_t M, float* out);
void orc_layernorm(const float* X, const float* gamma, const float* beta, float eps, size_t F, size_t M,
                   float* out);
void orc_rmsnorm_quant_i8(const float* X, const float* gamma, float eps, size_t F, size_t M,
                          uint32_t* xq, float* s);

/* ---- gated activations (SwiGLU / ReLU^2-GLU) and the gated FFN block (config C4) ---- */
float orc_exp(float x);
void orc_exp_array(const float* x, size_t n, float* out);
float orc_glu_one(float g, float u, int act);
void orc_glu(const float* in, size_t F, size_t M, int act, float* out);
long orc_glu_src_row(size_t r, size_t F);
void orc_glu_interleave(const uint32_t* wq, const float* tau, const float* bias, size_t F, size_t K,
                        uint32_t* wq_out, float* tau_out, float* bias_out);
void orc_ffn_glu_i8(const float* X, const float* gamma, float eps, size_t d, size_t F, size_t M, int act,
                    const uint32_t* wq1, const float* tau1, const float* b1, const float* gamma_sub,
                    float eps_sub, const uint32_t* wq2, const float* tau2, const float* b2, int threads,
                    float* h_out, float* Y);

/* ---- batched decode step (config C5) ---- */
void orc_rope_table(size_t dk, size_t max_len, float* cos_out, float* sin_out);
void orc_rope_apply(const float* x, size_t dk, const float* cos_row, const float* sin_row, float* out);
void orc_attention_decode(const float* q, const float* k, const float* v, size_t B, size_t H, size_t Hkv,
                          size_t dk, const int32_t* pos, const float* cosT, const float* sinT, float* k_cache,
                          float* v_cache, size_t max_len, float scale, float* out);
float orc_round_f16(float x);
void orc_round_f16_n(const float* x, size_t n, float* out);
void orc_attention_decode_ct(const float* q, const float* k, const float* v, size_t B, size_t H, size_t Hkv,
                             size_t dk, const int32_t* pos, const float* cosT, const float* sinT, float* k_cache,
                             float* v_cache, size_t max_len, float scale, int cache_f16, float* out);
void orc_embedding_gather(const float* table, const int32_t* ids, size_t V, size_t d, size_t B, float* out);
int32_t orc_argmax(const float* logits, size_t V, size_t stride);

/* ---- MI355X tile layout of packed ternary weights (checker for the repacker) ---- */
size_t orc_repacked_words(size_t N, size_t K);
void orc_repack(const uint32_t* wq, size_t N, size_t K, uint32_t* out);
void orc_unrepack(const uint32_t* rp, size_t N, size_t K, uint32_t* wq);

#ifdef __cplusplus
}
#endif
#endif
