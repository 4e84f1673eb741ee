/*
 * nnhip.h — C ABI of libnn-hip.so, the MI355X (gfx950) engine for neuralnet.cpp's
 * BitNet b1.58 BitLinear W1.58A8 hot path.
 *
 * Plain C: opaque handles, device pointers as void / scalar pointers, sizes as size_t,
 * a status enum and a thread-local last-error string. No HIP or torch types appear here.
 *
 * The reference exposes this path as C++ virtual methods of nn::ComputeEngine (NVI public
 * entry -> protected *_impl), implemented in the engine submodule (compute.neuralnet.cpp);
 * the C++ layer of this library (nn::HipEngine, neuralnet.cpp_amd/host) implements that
 * interface on top of these entry points. Each declaration names the reference interface
 * it replaces (file:line of the reference call site / contract, relative to the reference
 * repository root).
 *
 * Layouts at this boundary follow the reference exactly:
 *   W      (N, K)            f32 row-major, one output channel per row
 *   tau    (N, 1)            f32 per-row absmean scale
 *   wq     (N, ceil(K/16))   u32 words, 16 trits per word LSB first, code = trit + 2, tail code 2
 *   X      (K, M)            f32 row-major; one column = one token
 *   s      (1, M)            f32 per-token scale (absmax * fl(1/127))
 *   xq     (K, ceil(M/4))    u32 words, 4 int8 per word little-endian, tail bytes 0
 *   Y      (N, M)            f32 row-major
 * The engine-internal layouts (repacked weights, token-major int8 activations) are
 * described with the functions that produce them.
 *
 * Threading: one context = one HIP stream; calls on one context must not overlap
 * (the reference's "one engine per thread" rule, docs/usage/07-thread-safety.md:9-17).
 * All compute entry points are asynchronous on the context's stream.
 */
#ifndef NNHIP_H
#define NNHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum nnhip_status
{
    NNHIP_OK = 0,
    NNHIP_ERR_INVALID_ARG = 1, /* bad pointer, shape, or size */
    NNHIP_ERR_HIP = 2,         /* a HIP runtime call or kernel launch failed */
    NNHIP_ERR_OOM = 3,         /* device allocation failed */
    NNHIP_ERR_NO_DEVICE = 4,   /* no usable gfx950 device */
    NNHIP_ERR_UNSUPPORTED = 5  /* shape or option outside what the kernels support */
} nnhip_status;

typedef struct nnhip_ctx nnhip_ctx;
typedef struct nnhip_group nnhip_group;

/* ------------------------------------------------------------ runtime */

/* Message of the last failed call on this thread ("" if none).
 * Replaces nn::last_error() (modules/nn.engine.cpp:36-48). */
const char* nnhip_last_error(void);

/* Library version string, e.g. "nnhip 0.1.0 gfx950". */
const char* nnhip_version(void);

/* FNV-1a over `bytes` bytes of HOST memory in address order, with the constants of the reference's
 * layer_bench --hash (src/layer_bench.cpp:732-741): start value 1469598103934665603 as the reference
 * writes it (the published FNV-1a 64 offset basis is 14695981039346656037; the reference's value is
 * kept so that hashes compare with its output), prime 1099511628211, each f32's four bytes low to
 * high, i.e. the little-endian memory order. A measurement aid: two kernel versions that agree bit
 * for bit give the same hash. */
uint64_t nnhip_fnv1a64(const void* data, size_t bytes);

/* Number of visible HIP devices. */
nnhip_status nnhip_device_count(int* count);

/* Compute units, peak engine clock (kHz), memory clock (kHz) and memory bus width (bits) of a
 * device, as HIP reports them: the inputs of the roofline peaks (dense int8 MFMA = CUs x clock x
 * 8192 ops per clock on gfx950). No reference counterpart (a measurement aid). */
nnhip_status nnhip_device_info(int device, int* cus, int* clock_khz, int* mem_clock_khz, int* bus_bits);

/* The device's name and architecture as HIP reports them, e.g. "AMD Instinct MI355X (gfx950:...)",
 * written NUL-terminated into buf (truncated to len - 1 characters). Fills EngineInfo::device of
 * ComputeEngine::describe (docs/internal/23-library-design-cleanup-and-model-file-roles.md:240-246). */
nnhip_status nnhip_device_name(int device, char* buf, size_t len);

/* Create a context bound to `device` with its own stream (default priority).
 * Replaces nn::create_gpu_engine(const char* device) (cli/cli_engine_factory.hpp:51-76). */
nnhip_status nnhip_ctx_create(int device, nnhip_ctx** out);
nnhip_status nnhip_ctx_destroy(nnhip_ctx* ctx);

/* Use an external hipStream_t (passed as void*) for all later calls; NULL selects the
 * device's null (legacy default) stream. The caller keeps the external stream alive.
 * nnhip_ctx_reset_stream goes back to the context's own stream. */
nnhip_status nnhip_ctx_set_stream(nnhip_ctx* ctx, void* stream);
nnhip_status nnhip_ctx_reset_stream(nnhip_ctx* ctx);
nnhip_status nnhip_ctx_get_stream(nnhip_ctx* ctx, void** stream);

/* Block tile of the prefill GEMM (M > 16 tokens): automatic (the default) picks, per call, the
 * tile with the fewest estimated block rounds over the CUs, and may split the rows over two
 * launches (256 x 128 blocks over whole rounds of the CUs, a smaller tile over the rest); the
 * others force one tile for all rows. A tuning control of this library (the reference's GEMM
 * shader has a single 64 x 64 tile); results are bit-identical whichever tile runs. */
#define NNHIP_GEMM_TILE_AUTO 0
#define NNHIP_GEMM_TILE_256x128 1
#define NNHIP_GEMM_TILE_128x128 2
#define NNHIP_GEMM_TILE_64x64 3
nnhip_status nnhip_ctx_set_gemm_tile(nnhip_ctx* ctx, int tile);

/* A performance hint with no counterpart in the reference: the next call on this context of
 * nnhip_act_quant_i8 / nnhip_rmsnorm_quant_i8 (at most 64 tokens), nnhip_rmsnorm_quant_i8_tokens,
 * nnhip_embedding_rmsnorm_quant_i8_tokens or nnhip_partial_residual_quant_i8 also reads the given device ranges (count <= 4, each
 * 16-byte aligned; whole 16-byte units inside each range, at most 64 MiB in all) in extra
 * blocks, so that the kernel after it, which reads the same bytes (a decoder's next BitLinear
 * weights), finds them in the GPU's memory-side cache. That call takes the ranges whether or
 * not it can use them (M > 64 cannot); results never depend on them. The ranges must stay
 * allocated until that call has run on the device. count = 0 clears them. */
nnhip_status nnhip_ctx_prefetch_next(nnhip_ctx* ctx, size_t count, const void* const* ptrs, const size_t* bytes);

/* Block the host until all work queued on the context's stream has finished.
 * Replaces ComputeEngine::end_batch()/flush_batch() waits (compute_layer_gpt.hpp:715-719). */
nnhip_status nnhip_sync(nnhip_ctx* ctx);

/* Device memory (hipMalloc/hipFree on the context's device). */
nnhip_status nnhip_malloc(nnhip_ctx* ctx, size_t bytes, void** out);
nnhip_status nnhip_free(nnhip_ctx* ctx, void* ptr);

/* Copies, ordered on the context's stream. h2d/d2h return after the copy completed
 * (the host buffer may be reused). Replace ComputeEngine::from_matrix/to_matrix transfers
 * (src/test_common.hpp:68-92). */
nnhip_status nnhip_memcpy_h2d(nnhip_ctx* ctx, void* dst, const void* src, size_t bytes);
nnhip_status nnhip_memcpy_d2h(nnhip_ctx* ctx, void* dst, const void* src, size_t bytes);
nnhip_status nnhip_memcpy_d2d(nnhip_ctx* ctx, void* dst, const void* src, size_t bytes);

/* Precision casts at the engine boundary: f32 -> IEEE binary16 (round to nearest even; overflow to
 * infinity, NaN stays NaN) and binary16 -> f32 (exact). The reference's public engine entries cast
 * F16 tensors to the f32 of their implementation and their results to the requested precision
 * (docs/development/04-compute-engine-development.md:110-114); these are those casts. */
nnhip_status nnhip_convert_f32_f16(nnhip_ctx* ctx, const float* src, size_t n, uint16_t* dst);
nnhip_status nnhip_convert_f16_f32(nnhip_ctx* ctx, const uint16_t* src, size_t n, float* dst);

/* Fill `words` u32 words with `value` using a kernel (safe inside a captured graph). */
nnhip_status nnhip_fill_u32(nnhip_ctx* ctx, void* dst, uint32_t value, size_t words);

/* ------------------------------------------- reference-layout primitives */

/* tau[n] = sum_k fl(|W[n,k]| * fl(1/K)), fixed order: 64 lanes, lane l sums k = l, l+64, ...
 * ascending, then a xor butterfly 32,16,8,4,2,1.
 * Replaces dsl::compute_reduce_into(row_reduce_sum(abs(W)*rparam(1/K)))
 * (include/neuralnet.cpp/compute_layer_bitlinear.hpp:637-640). */
nnhip_status nnhip_row_absmean(nnhip_ctx* ctx, const float* W, size_t N, size_t K, float* tau);

/* wq = trit_pack(W, tau): code 3 if w > 0.5*tau[n], 1 if w < -0.5*tau[n], else 2.
 * Replaces ComputeEngine::trit_pack / trit_pack_into
 * (include/neuralnet.cpp/compute_layer_bitlinear.hpp:305, :650; src/ternary_gemm_test.cpp:224-251). */
nnhip_status nnhip_trit_pack(nnhip_ctx* ctx, const float* W, const float* tau, size_t N, size_t K,
                             uint32_t* wq);

/* out[c] = max over rows of x[r,c] (NaN ignored; -inf for rows == 0).
 * Replaces ComputeEngine::col_reduce_max (include/neuralnet.cpp/compute_layer_bitlinear.hpp:445). */
nnhip_status nnhip_col_reduce_max(nnhip_ctx* ctx, const float* x, size_t rows, size_t cols,
                                  float* out);

/* out[i] = |x[i]| (out may alias x). Replaces dsl::compute(abs(X))
 * (include/neuralnet.cpp/compute_layer_bitlinear.hpp:443). */
nnhip_status nnhip_abs(nnhip_ctx* ctx, const float* x, size_t n, float* out);

/* x[i] = x[i] * alpha. Replaces ComputeEngine::scale_inplace
 * (include/neuralnet.cpp/compute_layer_bitlinear.hpp:446). */
nnhip_status nnhip_scale_inplace(nnhip_ctx* ctx, float* x, size_t n, float alpha);

/* s[m] = (max_k |X[k,m]|) * fl(1/127): the three calls above fused into one kernel. */
nnhip_status nnhip_act_scale(nnhip_ctx* ctx, const float* X, size_t K, size_t M, float* s);

/* out (rows, ceil(cols/4)) = quantize_i8(x (rows, cols), scale, col_scale):
 * q = round_half_away(clamp(x/s, -127, 127)), NaN -> 0, s == 0 -> 0; scale is (1, cols)
 * when col_scale != 0, else (rows, 1). Replaces ComputeEngine::quantize_i8
 * (include/neuralnet.cpp/compute_layer_bitlinear.hpp:448; src/int8_act_test.cpp:86-137). */
nnhip_status nnhip_quantize_i8(nnhip_ctx* ctx, const float* x, const float* scale, size_t rows,
                               size_t cols, int col_scale, uint32_t* out);

/* out (rows, cols) f32 integers from the int8 container (rows, ceil(cols/4)).
 * Replaces ComputeEngine::unpack_i8 (include/neuralnet.cpp/compute_layer_bitlinear.hpp:516;
 * src/int8_act_test.cpp:140-168). */
nnhip_status nnhip_unpack_i8(nnhip_ctx* ctx, const uint32_t* packed, size_t rows, size_t cols,
                             float* out);

/* Y (N, M) = (tau[n] * s[m]) * float(sum_k trit(n,k) * q(k,m)), int32 accumulation.
 * Reference-layout operands; internally repacks wq and transposes xq into workspace owned
 * by the context (grown on demand), then runs the same kernels as nnhip_ternary_matmul.
 * Replaces ComputeEngine::matmul_q_i8 (include/neuralnet.cpp/compute_layer_bitlinear.hpp:454;
 * contract docs/internal/21-quantized-weights.md:978-980; src/int8_act_test.cpp:171-238). */
nnhip_status nnhip_matmul_q_i8(nnhip_ctx* ctx, const uint32_t* wq, const float* tau,
                               const uint32_t* xq, const float* s, size_t N, size_t K, size_t M,
                               float* Y);

/* nnhip_matmul_q_i8 without any device allocation: the same operands, kernels and bits, with the
 * repacked weights and transposed activations kept in a scratch array that the library holds on
 * each GPU from the first context created on it until the process ends
 * (NNHIP_NOALLOC_SCRATCH_BYTES). A call needs round_up(nnhip_repacked_bytes(N, K), 256) +
 * round_up(nnhip_act_i8_bytes(K, M), 256) + round_up(4 M, 256) bytes of it (e.g. N = 11008,
 * K = 4096, M = 4096 fits); larger calls fail with NNHIP_ERR_UNSUPPORTED before any work is queued.
 * Calls no hipMalloc / hipFree. Every call on one GPU shares that GPU's scratch, whichever context
 * it comes from: calls that overlap in time on one GPU (other streams, other threads) race.
 * No counterpart in the reference: for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid allocation). */
#define NNHIP_NOALLOC_SCRATCH_BYTES (32u << 20)
nnhip_status nnhip_matmul_q_i8_noalloc(nnhip_ctx* ctx, const uint32_t* wq, const float* tau,
                                       const uint32_t* xq, const float* s, size_t N, size_t K,
                                       size_t M, float* Y);

/* Y (N, M) = (tau o trit(wq)) . B: ternary weights times float activations with f32
 * accumulation; B (K, M) and Y (N, M) are f32, or f16 when b_f16 / y_f16 != 0 (16-bit IEEE
 * halves, round to nearest even on output). Accumulation order is not pinned by the reference;
 * results match a float64 evaluation within 1e-4 x max(1, max|Y|) (f32) or 4e-3 (f16 output).
 * Replaces ComputeEngine::matmul_q (include/neuralnet.cpp/compute_layer_bitlinear.hpp:464;
 * src/ternary_gemm_test.cpp:253-289, :435-526). */
nnhip_status nnhip_matmul_q(nnhip_ctx* ctx, const uint32_t* wq, const float* tau, const void* B, int b_f16,
                            size_t N, size_t K, size_t M, void* Y, int y_f16);

/* Y (M, N) = (tau o trit(A))^T . B, with A (K, ceil(M/16)) packed like wq (one stored row per
 * k, tau (K, 1) per stored row) and B (K, N); precisions and tolerance as nnhip_matmul_q.
 * Replaces ComputeEngine::matmul_q_t (include/neuralnet.cpp/compute_layer_bitlinear.hpp:494, the
 * dX = (tau o W)^T . dY of BitLinear::backward; src/ternary_gemm_test.cpp:291-334, :435-526). */
nnhip_status nnhip_matmul_q_t(nnhip_ctx* ctx, const uint32_t* A, const float* tau, const void* B, int b_f16,
                              size_t K, size_t M, size_t N, void* Y, int y_f16);

/* Y[n, m] = Y[n, m] + b[n]. Replaces dsl::compute(leaf(y) + row_broadcast(b))
 * (include/neuralnet.cpp/compute_layer_bitlinear.hpp:455-456). */
nnhip_status nnhip_add_row_broadcast(nnhip_ctx* ctx, float* Y, const float* b, size_t N, size_t M);

/* out (F, M) = RMSNorm(X (F, M)) with gain gamma (F): rms_inv = 1/sqrt(sum_f x^2 * fl(1/F) + eps)
 * (sum in a fixed order: 512 strided parts f % 512, each ascending, then a xor butterfly over
 * offsets 256..1), out = (x * rms_inv) * gamma[f].
 * Replaces RMSNorm::forward (include/neuralnet.cpp/compute_layer_mlp.hpp:686-707). */
nnhip_status nnhip_rmsnorm(nnhip_ctx* ctx, const float* X, const float* gamma, float eps, size_t F,
                           size_t M, float* out);

/* out (F, M) = LayerNorm(X (F, M)) with gain gamma (F) and shift beta (F): mean = sum_f x * fl(1/F),
 * d = x - mean, sinv = 1/sqrt(sum_f d*d * fl(1/F) + eps), out = (d * sinv) * gamma[f] + beta[f], each
 * step rounded to fp32 (both sums in one fixed order: 8 strided parts f % 8, each ascending, then
 * ((p0 + p1) + (p2 + p3)) + ((p4 + p5) + (p6 + p7))).
 * Replaces LayerNorm::forward (include/neuralnet.cpp/compute_layer_mlp.hpp:529-545), the SubLN
 * norm type FeedForward takes by default (include/neuralnet.cpp/compute_layer_feedforward.hpp:50-65). */
nnhip_status nnhip_layernorm(nnhip_ctx* ctx, const float* X, const float* gamma, const float* beta, float eps,
                             size_t F, size_t M, float* out);

/* --------------------------------------------- MI355X-native fast path */

/* Repacked ternary weights, layout T16K256: rows padded to 16, k padded to 256; one
 * 1 KiB tile per (16 rows x 256 k) in row-tile-major order, each tile holding in lane
 * order the A operands of four 16x16x64 int8 MFMAs (see nn_oracle.c for the bit map).
 * Bytes needed for N x K weights: */
size_t nnhip_repacked_bytes(size_t N, size_t K);

/* Load-time repacker: reference container wq (N, ceil(K/16)) -> T16K256 (rp, 16-byte
 * aligned, nnhip_repacked_bytes(N, K) bytes). Lossless: nnhip_unrepack_ternary inverts it
 * bit for bit (including the tail codes of the last word of each row). No reference
 * counterpart (engine-internal layout; the reference consumes wq directly). */
nnhip_status nnhip_repack_ternary(nnhip_ctx* ctx, const uint32_t* wq, size_t N, size_t K, void* rp);
nnhip_status nnhip_unrepack_ternary(nnhip_ctx* ctx, const void* rp, size_t N, size_t K, uint32_t* wq);

/* Token-major int8 activations ("xi"): M rows of Kp = roundup(K, 256) bytes, row m holds the
 * quantized token m in natural k order, bytes K..Kp-1 are 0; plus rowsum[m] = sum_k q(k, m)
 * (int32). Bytes needed for xi: */
size_t nnhip_act_i8_bytes(size_t K, size_t M);

/* Fused abs -> per-token absmax -> scale -> int8 quantization of X (K, M) (reference layout):
 * s[m] = max_k |X[k,m]| * fl(1/127); xi, rowsum as above. xq_ref (nullable) also receives
 * the reference container (K, ceil(M/4)). Replaces the sequence of
 * include/neuralnet.cpp/compute_layer_bitlinear.hpp:443-448 with one kernel. */
nnhip_status nnhip_act_quant_i8(nnhip_ctx* ctx, const float* X, size_t K, size_t M, int8_t* xi,
                                float* s, int32_t* rowsum, uint32_t* xq_ref);

/* Fused RMSNorm -> absmax -> int8: as nnhip_rmsnorm followed by nnhip_act_quant_i8 on its
 * output, without materializing the normalized tensor (bit-identical to that sequence).
 * Replaces RMSNorm::forward + the BitLinear int8 prologue
 * (compute_layer_mlp.hpp:686-707 + compute_layer_bitlinear.hpp:443-448). */
nnhip_status nnhip_rmsnorm_quant_i8(nnhip_ctx* ctx, const float* X, const float* gamma, float eps,
                                    size_t F, size_t M, int8_t* xi, float* s, int32_t* rowsum,
                                    uint32_t* xq_ref);

/* Reference int8 container xq (K, ceil(M/4)) -> xi + rowsum (and back). */
nnhip_status nnhip_act_i8_from_container(nnhip_ctx* ctx, const uint32_t* xq, size_t K, size_t M,
                                         int8_t* xi, int32_t* rowsum);
nnhip_status nnhip_act_i8_to_container(nnhip_ctx* ctx, const int8_t* xi, size_t K, size_t M,
                                       uint32_t* xq);

/* Ternary x int8 product on the fast layouts: Y (N, M) = (tau[n]*s[m]) * float(acc) [+ bias[n]],
 * acc = sum_k trit(n,k) q(k,m) in int32 (exact). The bias add is a separate rounding (no FMA).
 * M <= 16 runs the weight-streaming decode GEMV, larger M the MFMA GEMM. bias may be NULL.
 * Replaces ComputeEngine::matmul_q_i8 + bias (compute_layer_bitlinear.hpp:454-456). */
nnhip_status nnhip_ternary_matmul(nnhip_ctx* ctx, const void* rp, const float* tau, const int8_t* xi,
                                  const float* s, const int32_t* rowsum, const float* bias, size_t N,
                                  size_t K, size_t M, float* Y);

/* Float-activation product on the fast layout: Y (N, M) = (tau o trit(rp)) . B with B (K, M) f32, or
 * f16 when b_f16 != 0, and Y f32 or f16 (y_f16). The activations of each token are split exactly
 * into four int8 digits of a per-token 31-bit fixed point (x rounded to 2^(E-31) where
 * max|x| < 2^E), the digit products run on the int8 MFMA GEMV / GEMM (exact int32) and are
 * combined in int64; results match a float64 evaluation far inside the reference tolerance
 * (1e-4 x max(1, max|Y|)). A token holding NaN or an infinity gets the IEEE result of its
 * non-finite terms per row (NaN for NaN, 0 x inf or opposite infinities, else the infinity).
 * K < 131072. Uses context scratch (grown on demand).
 * Replaces ComputeEngine::matmul_q on the BitLinear f32 branch (include/neuralnet.cpp/
 * compute_layer_bitlinear.hpp:459-466; src/ternary_gemm_test.cpp:253-289) when the weights are
 * kept repacked; nnhip_matmul_q takes the reference container. */
nnhip_status nnhip_ternary_matmul_f(nnhip_ctx* ctx, const void* rp, const float* tau, const void* B, int b_f16,
                                    size_t N, size_t K, size_t M, void* Y, int y_f16);

/* Transposed float-activation product on the fast layout: Y (M, N) = (tau o trit(A))^T . B for a
 * container A (K, ceil(M/16)) with tau (K) per stored row, B (K, N) f32 or f16, given rpT = the
 * T16K256 repack of A's transpose (nnhip_trit_transpose, then nnhip_repack_ternary of the
 * (M, ceil(K/16)) result with M rows and K columns). tau folds into the activations,
 * fl(tau_k * b) * trit = fl(tau_k * trit) * b term by term; then as nnhip_ternary_matmul_f.
 * Replaces ComputeEngine::matmul_q_t, the dX product of BitLinear::backward
 * (include/neuralnet.cpp/compute_layer_bitlinear.hpp:494; src/ternary_gemm_test.cpp:291-334). */
nnhip_status nnhip_ternary_matmul_t_f(nnhip_ctx* ctx, const void* rpT, const float* tau, const void* B, int b_f16,
                                      size_t K, size_t M, size_t N, void* Y, int y_f16);

/* *out ^= the XOR of the bytes / 4 32-bit words at src (bytes a multiple of 4, src 16-byte
 * aligned), in one streaming pass of non-temporal 16-byte loads; zero *out first for the plain
 * checksum. A measurement aid with no reference counterpart: its rate is the achievable HBM read
 * bandwidth that the HBM-bound kernels here are compared with. */
nnhip_status nnhip_stream_xor(nnhip_ctx* ctx, const void* src, size_t bytes, uint32_t* out);

/* Bit transpose of a packed container: A (K, ceil(M/16)) -> At (M, ceil(K/16)), trit (m, k) of At =
 * trit (k, m) of A, tail codes 2. The load-time step before nnhip_ternary_matmul_t_f (no
 * reference counterpart: the reference reads the container transposed in place). */
nnhip_status nnhip_trit_transpose(nnhip_ctx* ctx, const uint32_t* A, size_t K, size_t M, uint32_t* At);

/* Y = nnhip_ternary_matmul(...) + res: the decoder's residual add in the same launch on the decode
 * path and on the prefill GEMM (M > 16: added in its epilogue) (res (N, M) f32, must not alias Y). Same bits as nnhip_ternary_matmul then nnhip_add(res, Y).
 * Replaces w_o's BitLinear::forward followed by the residual add of GPTBlock::forward_step
 * (include/neuralnet.cpp/compute_layer_attention.hpp:1089; compute_layer_gpt.hpp:208-209). */
nnhip_status nnhip_ternary_matmul_add(nnhip_ctx* ctx, const void* rp, const float* tau, const int8_t* xi,
                                      const float* s, const int32_t* rowsum, const float* bias, const float* res,
                                      size_t N, size_t K, size_t M, float* Y);

/* nnhip_ternary_matmul_add with res and Y token-major (M, N): the same bits transposed, for a
 * decoder that keeps its residual stream token-major so that the next per-token quantizer
 * (nnhip_rmsnorm_quant_i8_tokens) reads contiguous rows. Decode sizes only (the single-launch
 * GEMV: M <= 16); NNHIP_ERR_UNSUPPORTED otherwise. Same reference step as
 * nnhip_ternary_matmul_add (compute_layer_attention.hpp:1089; compute_layer_gpt.hpp:208-209). */
nnhip_status nnhip_ternary_matmul_add_tokens(nnhip_ctx* ctx, const void* rp, const float* tau, const int8_t* xi,
                                             const float* s, const int32_t* rowsum, const float* bias, const float* res,
                                             size_t N, size_t K, size_t M, float* Y);

/* Split-k partial sums of a decode ternary GEMV, without the epilogue: part[ks][m][n] (int32,
 * slices x M x N, token-major) = sum over slice ks of the k tiles of trit-code(n, k) * xi(m, k), the
 * integer dot products of nnhip_ternary_matmul's MFMAs, the K range cut into `slices` runs of
 * ceil(K/256 / slices) k tiles (each non-empty; slices in [1, 8], M <= 16). The slices add up
 * exactly to the whole-K sum; nnhip_partial_residual_quant_i8 applies the epilogue. For decode
 * BitLinears whose row count alone leaves most CUs idle (N = 2560: 40 work-groups of the
 * whole-K GEMV): the same weights stream from more CUs. The first half of
 * BitLinear::forward's int8 product (include/neuralnet.cpp/compute_layer_bitlinear.hpp:449-466). */
nnhip_status nnhip_ternary_matmul_partial(nnhip_ctx* ctx, const void* rp, const int8_t* xi, size_t N, size_t K,
                                          size_t M, size_t slices, int32_t* part);

/* The epilogue of nnhip_ternary_matmul_partial, the residual add and the next BitLinear's
 * quantizer in one kernel per token:
 *   x_out[n, m] = (tau[n] * s_in[m]) * float(sum_ks part[ks][m][n] - 2 rowsum_in[m]) [+ bias[n]]
 *                 [+ res[n, m]]          (res may alias x_out; bias, res nullable)
 *   then [RMSNorm(gamma, eps) when gamma is non-null ->] per-token absmax -> int8: xi, s, rowsum
 *   as nnhip_rmsnorm_quant_i8 / nnhip_act_quant_i8 on x_out.
 * Bit-identical to nnhip_ternary_matmul_add (or nnhip_ternary_matmul) followed by that quantizer.
 * M <= 64, N <= 11264. Replaces w_o's (fc2's) BitLinear epilogue, the residual add of
 * GPTBlock::forward_step and the following RMSNorm + int8 prologue (compute_layer_bitlinear.hpp:
 * 459-466; compute_layer_gpt.hpp:208-216; compute_layer_mlp.hpp:686-707). */
nnhip_status nnhip_partial_residual_quant_i8(nnhip_ctx* ctx, const int32_t* part, size_t slices, const float* tau,
                                             const float* s_in, const int32_t* rowsum_in, const float* bias,
                                             const float* res, size_t N, size_t M, float* x_out,
                                             const float* gamma, float eps, int8_t* xi, float* s, int32_t* rowsum);

/* nnhip_partial_residual_quant_i8 with res and x_out token-major (M, N); the same bits
 * transposed (xi, s, rowsum identical). Same reference steps. */
nnhip_status nnhip_partial_residual_quant_i8_tokens(nnhip_ctx* ctx, const int32_t* part, size_t slices,
                                                    const float* tau, const float* s_in, const int32_t* rowsum_in,
                                                    const float* bias, const float* res, size_t N, size_t M,
                                                    float* x_out, const float* gamma, float eps, int8_t* xi, float* s,
                                                    int32_t* rowsum);

/* count (1..4) BitLinears on the same int8 input (xi, s, rowsum; shared K and M):
 * Y[i] (N[i], M) = nnhip_ternary_matmul(rp[i], tau[i], xi, s, rowsum, bias[i], N[i], K, M), as one
 * launch on the decode path. rp / tau / N / Y are HOST arrays of count entries; bias may be NULL
 * (no bias anywhere) or an array holding NULLs. Same bits as count separate calls.
 * Replaces the q / k / v BitLinear::forward calls on one input
 * (include/neuralnet.cpp/compute_layer_attention.hpp:1009-1011). */
nnhip_status nnhip_ternary_matmul_n(nnhip_ctx* ctx, size_t count, const void* const* rp, const float* const* tau,
                                    const float* const* bias, const size_t* N, float* const* Y, const int8_t* xi,
                                    const float* s, const int32_t* rowsum, size_t K, size_t M);

/* nnhip_ternary_matmul_n with each Y[i] token-major (M, N[i]): the same bits transposed, for a
 * decoder whose attention takes token-major q, k, v (nnhip_attention_decode_tokens). Decode
 * sizes only (the single-launch GEMV); NNHIP_ERR_UNSUPPORTED otherwise. Same reference calls. */
nnhip_status nnhip_ternary_matmul_n_tokens(nnhip_ctx* ctx, size_t count, const void* const* rp,
                                           const float* const* tau, const float* const* bias, const size_t* N,
                                           float* const* Y, const int8_t* xi, const float* s, const int32_t* rowsum,
                                           size_t K, size_t M);

/* Grouped decode GEMV: many independent (weights, activations) problems with M <= 16 in one
 * launch, e.g. the q/k/v or gate/up projections of a layer, or a whole layer stack. The
 * descriptors are copied to the device once at creation; run() launches one kernel. */
typedef struct nnhip_gemv_desc
{
    const void* rp;        /* repacked weights (T16K256) */
    const float* tau;      /* (N) */
    const int8_t* xi;      /* (M, roundup(K,256)) */
    const float* s;        /* (M) */
    const int32_t* rowsum; /* (M) */
    const float* bias;     /* (N) or NULL */
    float* y;              /* (N, M) */
    uint64_t N, K, M;
} nnhip_gemv_desc;

nnhip_status nnhip_group_create(nnhip_ctx* ctx, const nnhip_gemv_desc* descs, size_t count,
                                nnhip_group** out);
nnhip_status nnhip_group_run(nnhip_ctx* ctx, nnhip_group* group);
nnhip_status nnhip_group_destroy(nnhip_ctx* ctx, nnhip_group* group);

/* What nnhip_group_create chose for a group: *lds_variant = 1 when every launch of the group
 * stages its activation blocks in LDS and reads its B operands there (one 16-row tile per
 * schedule item), 0 when the group runs the register variant only (activations loaded with the
 * weights), 2 when blocks over the LDS budget put part of the problems on the register variant
 * (one launch each, back to back); *waves = waves launched over all launches; *lds_bytes = the
 * largest staging per block. Any output may be NULL. No reference counterpart (introspection for
 * tests and measurement). */
nnhip_status nnhip_group_info(const nnhip_group* group, int* lds_variant, size_t* waves, size_t* lds_bytes);

/* Number of waves the decode GEMV launches for `items` row tiles (for roofline accounting). */
size_t nnhip_gemv_grid_waves(nnhip_ctx* ctx, size_t items);

/* ---- gated feed-forward block (the reference FeedForward with a SwiGLU or ReLU2GLU
 *      activation and BitLinear fc1/fc2, include/neuralnet.cpp/compute_layer_feedforward.hpp:182-204;
 *      config C4 adds the block's RMSNorm in front) ---- */
#define NNHIP_ACT_SWIGLU 0   /* (g * (1 / (1 + exp(-g)))) * u   compute_layer_mlp.hpp:317-328 */
#define NNHIP_ACT_RELU2GLU 1 /* (r * r) * u, r = max(g, 0)      compute_layer_mlp.hpp:405-414 */

/* Gated activation on fc1's output: Y1 (2F, M) with gate rows [0, F) and up rows [F, 2F)
 * -> h (F, M). exp is this library's fp32 exp (IEEE operations in a fixed order, within 2 ulp).
 * Replaces SwiGLU::forward / ReLU2GLU::forward (compute_layer_mlp.hpp:317-328, :405-414). */
nnhip_status nnhip_glu(nnhip_ctx* ctx, const float* Y1, size_t F, size_t M, int act, float* h);

/* Rows of the interleaved gate/up layout: 2 * roundup(F, 8). */
size_t nnhip_glu_rows(size_t F);

/* Load-time interleave of fc1's fused gate/up container wq (2F, ceil(K/16)) (the reference
 * fc1 is one BitLinear of 2F rows, compute_layer_feedforward.hpp:54-60) and of its tau / bias
 * (2F) into the engine-private order: 16-row group t = gate rows 8t..8t+7, then up rows
 * 8t..8t+7; padding rows (features >= F) get code 2, tau 0, bias 0. Outputs: wq_out
 * (nnhip_glu_rows(F), ceil(K/16)), tau_out / bias_out (nnhip_glu_rows(F)); bias may be NULL
 * (then bias_out may be NULL too). Repack wq_out with nnhip_repack_ternary for the kernels. */
nnhip_status nnhip_glu_interleave(nnhip_ctx* ctx, const uint32_t* wq, const float* tau, const float* bias,
                                  size_t F, size_t K, uint32_t* wq_out, float* tau_out, float* bias_out);

/* fc1 with the gated activation fused: h (F, M) = act(Y1), Y1 = the interleaved rows of
 * (tau*s)*float(acc) [+ bias] exactly as nnhip_ternary_matmul computes them (rp, tau, bias in
 * the interleaved order, N = nnhip_glu_rows(F)). M > 16 applies the activation in the GEMM
 * epilogue; M <= 16 runs the decode GEMV into context scratch, then the activation. */
nnhip_status nnhip_ternary_matmul_glu(nnhip_ctx* ctx, const void* rp, const float* tau, const int8_t* xi,
                                      const float* s, const int32_t* rowsum, const float* bias, size_t F,
                                      size_t K, size_t M, int act, float* h);

/* nnhip_ternary_matmul_glu with h written token-major, (M, F): token m's F features contiguous,
 * for a following per-token quantizer (nnhip_rmsnorm_quant_i8_tokens) that then reads each token
 * as one contiguous row. Decode sizes only (the deep GEMV: M <= 16); other shapes return
 * NNHIP_ERR_UNSUPPORTED. Same values as nnhip_ternary_matmul_glu, transposed. Replaces the fc1 +
 * gated activation of FeedForward::forward (include/neuralnet.cpp/compute_layer_feedforward.hpp:
 * 182-206; compute_layer_mlp.hpp:317-328, :405-414) inside the decode step. */
nnhip_status nnhip_ternary_matmul_glu_tokens(nnhip_ctx* ctx, const void* rp, const float* tau, const int8_t* xi,
                                             const float* s, const int32_t* rowsum, const float* bias, size_t F,
                                             size_t K, size_t M, int act, float* h);

/* nnhip_rmsnorm_quant_i8 (gamma != NULL) / nnhip_act_quant_i8 (gamma == NULL) on a token-major X
 * (M, K): the same codes, scales and row sums as on X transposed, for 1 <= M <= 64 and K <= 11264
 * (NNHIP_ERR_UNSUPPORTED otherwise). Replaces the SubLN RMSNorm -> quantize_i8 of the FFN's down
 * projection (compute_layer_feedforward.hpp:201-206; compute_layer_mlp.hpp:686-707;
 * compute_layer_bitlinear.hpp:443-448) in the decode step. */
nnhip_status nnhip_rmsnorm_quant_i8_tokens(nnhip_ctx* ctx, const float* X, const float* gamma, float eps, size_t K,
                                           size_t M, int8_t* xi, float* s, int32_t* rowsum);

/* nnhip_embedding_gather_tokens followed by nnhip_rmsnorm_quant_i8_tokens on its rows, in one
 * launch: x (B, d) = rows ids[b] of table (V, d) (NaN rows for ids outside [0, V)), and xi / s /
 * rowsum their [RMSNorm (gamma != NULL, eps) ->] absmax int8 quantization, the same bits as the
 * two calls. 1 <= B <= 64 and d <= 11264 (NNHIP_ERR_UNSUPPORTED otherwise); takes the
 * nnhip_ctx_prefetch_next ranges like the quantizer. The first steps of GPTModel::forward_step
 * (token embedding, compute_layer_gpt.hpp:697-702) and the first block's RMSNorm1 ->
 * quantize_i8 (compute_layer_gpt.hpp:203; compute_layer_bitlinear.hpp:443-448). */
nnhip_status nnhip_embedding_rmsnorm_quant_i8_tokens(nnhip_ctx* ctx, const float* table, const int32_t* ids,
                                                     size_t V, size_t d, size_t B, const float* gamma, float eps,
                                                     float* x, int8_t* xi, float* s, int32_t* rowsum);

/* Context scratch the block below uses (grown on demand, kept by the context). */
size_t nnhip_ffn_glu_workspace_bytes(size_t d, size_t F, size_t M);

/* The whole W1.58A8 gated block on X (d, M) f32:
 *   [RMSNorm(gamma, eps) if gamma != NULL] -> absmax int8 -> fc1 (interleaved rp1, tau1, b1)
 *   -> act -> [SubLN: RMSNorm(gamma_sub, eps_sub) over the F features if gamma_sub != NULL]
 *   -> absmax int8 -> fc2 (rp2 = repack of the (d, ceil(F/16)) container, tau2, b2) -> Y (d, M) f32.
 * Same bits as the reference sequence RMSNorm::forward, BitLinear::forward (int8 branch),
 * SwiGLU/ReLU2GLU::forward, [sub_norm_ RMSNorm::forward], BitLinear::forward
 * (compute_layer_mlp.hpp:686-707, compute_layer_bitlinear.hpp:441-457,
 * compute_layer_feedforward.hpp:182-206). b1/b2 may be NULL. */
nnhip_status nnhip_ffn_glu_i8(nnhip_ctx* ctx, const float* X, const float* gamma, float eps, size_t d,
                              size_t F, size_t M, int act, const void* rp1, const float* tau1, const float* b1,
                              const float* gamma_sub, float eps_sub, const void* rp2, const float* tau2,
                              const float* b2, float* Y);

/* ---- batched decode step (config C5): one new token for each of B sequences through the
 *      GPT block's attention (AttentionBase::forward_step, include/neuralnet.cpp/
 *      compute_layer_attention.hpp:1003-1091; GPTBlock::forward_step, compute_layer_gpt.hpp:
 *      201-219; GPTModel::forward_step, compute_layer_gpt.hpp:693-724). The reference advances
 *      one sequence per call; these entry points take B sequences, each at its own position. ---- */

/* RoPE tables on the HOST: cos_out / sin_out (max_len, dk/2), entry (pos, j) = cos / sin of
 * theta = float(pos) / powf(10000, float(2j) / float(dk)), evaluated in float as the reference's
 * RotaryEmbedding::fill_pos_column_ does (include/neuralnet.cpp/compute_position_encoding.hpp:64-80;
 * the reference stores each value twice, for j and j + dk/2). Upload them once per model. */
nnhip_status nnhip_rope_table(size_t dk, size_t max_len, float* cos_out, float* sin_out);

/* Context scratch nnhip_attention_decode uses for len_bound (0 when len_bound <= 128): the
 * per-chunk partial results. It grows on demand, so a first call of a new size allocates and
 * later ones do not (call once before capturing a graph). */
size_t nnhip_attention_workspace_bytes(size_t B, size_t H, size_t Hkv, size_t dk, size_t len_bound);

/* Attention of B new tokens over their sequences' KV caches (grouped-query heads, RoPE):
 *   q (H*dk, B), k / v (Hkv*dk, B): the projections of the new tokens (column b = sequence b);
 *   pos (B) int32, DEVICE: position of sequence b's new token (its cache length so far);
 *   k_cache / v_cache (B, max_len, Hkv*dk), 16-byte aligned: row t of sequence b = the rotated
 *   key (value) at position t; this call writes row pos[b] of each sequence;
 *   rope_cos / rope_sin (max_len, dk/2) from nnhip_rope_table, or both NULL (no position encoding);
 *   out (H*dk, B) = per head h: softmax((rot(q_h) . K^T) * scale) . V over positions [0, pos[b]],
 *   with query head h reading KV head h / (H / Hkv).
 * The new key is rotated at pos[b] ((q*cos + rotate_half(q)*sin), two rounded products and a
 * rounded sum) and stored bit-exactly; the products and the softmax are f32 with an order the
 * reference does not pin (results within 1e-5 relative of a float64 evaluation).
 * len_bound bounds every pos[b] + 1 (it sizes the launch; len_bound <= max_len); a sequence
 * whose pos[b] is outside [0, len_bound) gets NaN outputs and its cache is left unchanged.
 * dk in {64, 128, 256}; H / Hkv <= 8.
 * Replaces AttentionBase::forward_step steps 1.5-8 (compute_layer_attention.hpp:1022-1083: RoPE
 * apply_qk_step, GQA gather_rows, insert_rows into the caches, batched scores, softmax,
 * V^T . attn). */
nnhip_status nnhip_attention_decode(nnhip_ctx* ctx, const float* q, const float* k, const float* v, size_t B,
                                    size_t H, size_t Hkv, size_t dk, const int32_t* pos, size_t len_bound,
                                    const float* rope_cos, const float* rope_sin, float* k_cache, float* v_cache,
                                    size_t max_len, float scale, float* out);

/* nnhip_attention_decode on token-major rows: q (B, H*dk), k / v (B, Hkv*dk) and out (B, H*dk),
 * row b = sequence b's heads; the same bits as nnhip_attention_decode on the transposes (same
 * kernels, other load and store indices), and the same cache rows. For a decode step whose
 * producing and consuming kernels work on whole tokens (nnhip_ternary_matmul_n_tokens,
 * nnhip_rmsnorm_quant_i8_tokens: each token's values are then one contiguous row instead of
 * elements B*4 bytes apart). No separate counterpart in the reference: the same steps of
 * AttentionBase::forward_step (compute_layer_attention.hpp:1022-1083) in the layout of the
 * neighbouring steps. */
nnhip_status nnhip_attention_decode_tokens(nnhip_ctx* ctx, const float* q, const float* k, const float* v, size_t B,
                                           size_t H, size_t Hkv, size_t dk, const int32_t* pos, size_t len_bound,
                                           const float* rope_cos, const float* rope_sin, float* k_cache,
                                           float* v_cache, size_t max_len, float scale, float* out);

/* KV caches of IEEE binary16 elements (compute = F16): the reference creates each layer's KV
 * caches in the profile's compute precision, engine.create_tensor(seq_len_, d_model_, p_.compute)
 * (include/neuralnet.cpp/compute_layer_gpt.hpp:764-765), F16 under the t1_58 preset
 * (src/t1_58_test.cpp:668-690). The same attention as nnhip_attention_decode /
 * nnhip_attention_decode_tokens with k_cache / v_cache holding f16 bit patterns: the appended
 * rotated key and value are rounded to the nearest f16 (ties to even) and this call's scores use
 * the rounded values, as every later call reads them; cached elements are widened exactly and
 * q, k, v, out and the arithmetic stay f32. Half the cache bytes per call. */
nnhip_status nnhip_attention_decode_h(nnhip_ctx* ctx, const float* q, const float* k, const float* v, size_t B,
                                      size_t H, size_t Hkv, size_t dk, const int32_t* pos, size_t len_bound,
                                      const float* rope_cos, const float* rope_sin, uint16_t* k_cache,
                                      uint16_t* v_cache, size_t max_len, float scale, float* out);
nnhip_status nnhip_attention_decode_tokens_h(nnhip_ctx* ctx, const float* q, const float* k, const float* v, size_t B,
                                             size_t H, size_t Hkv, size_t dk, const int32_t* pos, size_t len_bound,
                                             const float* rope_cos, const float* rope_sin, uint16_t* k_cache,
                                             uint16_t* v_cache, size_t max_len, float scale, float* out);

/* ---- batched prefill (config C5's 2048-token context): T new tokens of each of B sequences at
 *      positions pos0 .. pos0 + T - 1 in one pass. The reference fills the cache by running
 *      forward_step once per context token (GPTModel::generate, include/neuralnet.cpp/
 *      compute_layer_gpt.hpp:774-794); these give every token the result of its own step. Token
 *      column m = b * T + t of the (rows, B * T) feature-major tensors below. ---- */

/* Append T tokens per sequence to the KV caches: k / v (Hkv*dk, B*T) are the k / v projections;
 * cache row pos0 + t of sequence b gets the key of token t rotated at position pos0 + t (as
 * nnhip_attention_decode stores it, bit for bit) and its value. Needs pos0 + T <= max_len;
 * dk in {64, 128}; rope tables as nnhip_attention_decode (both NULL: no position encoding).
 * Replaces the insert_rows steps of T AttentionBase::forward_step calls
 * (include/neuralnet.cpp/compute_layer_attention.hpp:1040-1060). */
nnhip_status nnhip_kv_cache_fill(nnhip_ctx* ctx, const float* k, const float* v, size_t B, size_t T, size_t Hkv,
                                 size_t dk, size_t pos0, const float* rope_cos, const float* rope_sin, float* k_cache,
                                 float* v_cache, size_t max_len);

/* nnhip_kv_cache_fill into f16 caches (compute = F16, compute_layer_gpt.hpp:764-765): each rotated
 * key and value rounded to the nearest f16, the rows nnhip_attention_decode_h would append. */
nnhip_status nnhip_kv_cache_fill_h(nnhip_ctx* ctx, const float* k, const float* v, size_t B, size_t T, size_t Hkv,
                                   size_t dk, size_t pos0, const float* rope_cos, const float* rope_sin,
                                   uint16_t* k_cache, uint16_t* v_cache, size_t max_len);

/* Causal attention of the T tokens over caches already holding rows [0, pos0 + T) (after
 * nnhip_kv_cache_fill): out (H*dk, B*T), column b*T + t = per query head h the softmax
 * ((rot(q_h) . K^T) * scale) . V over cache rows [0, pos0 + t] of sequence b, KV head h / (H/Hkv),
 * q rotated at pos0 + t. f32 on the fp32 MFMA with an online softmax: within 2e-6 relative of a
 * float64 evaluation (the reference does not pin the order). dk in {64, 128}; H / Hkv in
 * {1, 2, 4, 8}. Replaces the attention steps of T AttentionBase::forward_step calls
 * (compute_layer_attention.hpp:1022-1083). */
nnhip_status nnhip_attention_prefill(nnhip_ctx* ctx, const float* q, const float* k_cache, const float* v_cache,
                                     size_t B, size_t T, size_t H, size_t Hkv, size_t dk, size_t pos0,
                                     const float* rope_cos, const float* rope_sin, size_t max_len, float scale,
                                     float* out);

/* nnhip_attention_prefill over f16 caches (compute = F16, compute_layer_gpt.hpp:764-765): the
 * cached elements widened exactly, everything else as nnhip_attention_prefill. */
nnhip_status nnhip_attention_prefill_h(nnhip_ctx* ctx, const float* q, const uint16_t* k_cache,
                                       const uint16_t* v_cache, size_t B, size_t T, size_t H, size_t Hkv, size_t dk,
                                       size_t pos0, const float* rope_cos, const float* rope_sin, size_t max_len,
                                       float scale, float* out);

/* dst (rows, n): column j = column col0 + j * stride of src (rows, src_cols), e.g. the last token of
 * each sequence after a prefill (col0 = T - 1, stride = T) for the LM head. Replaces the reference's
 * use of the last step's output (last_logits_t, compute_layer_gpt.hpp:785-790). */
nnhip_status nnhip_copy_columns(nnhip_ctx* ctx, const float* src, size_t rows, size_t src_cols, size_t col0,
                                size_t stride, size_t n, float* dst);

/* out[i] = x[i] + y[i] (one IEEE add; out may alias x or y). Replaces the residual adds
 * dsl::compute(leaf(x) + leaf(a)) of GPTBlock::forward_step (compute_layer_gpt.hpp:208-218). */
nnhip_status nnhip_add(nnhip_ctx* ctx, const float* x, const float* y, size_t n, float* out);

/* out (d, B): column b = row ids[b] of the (V, d) embedding table (ids DEVICE int32; an id
 * outside [0, V) gives a NaN column). Replaces gather_rows(token_emb, id) + transpose
 * (compute_layer_gpt.hpp:700-704). */
nnhip_status nnhip_embedding_gather(nnhip_ctx* ctx, const float* table, const int32_t* ids, size_t V, size_t d,
                                    size_t B, float* out);

/* nnhip_embedding_gather with out token-major (B, d): row b = row ids[b] of the table (NaN row for
 * an id outside [0, V)). Replaces gather_rows(token_emb, id) (compute_layer_gpt.hpp:700-704)
 * without the transpose. */
nnhip_status nnhip_embedding_gather_tokens(nnhip_ctx* ctx, const float* table, const int32_t* ids, size_t V, size_t d,
                                           size_t B, float* out);

/* ids[b] = greedy choice over column b of logits (V, B): the first index of the largest value,
 * NaN never chosen except that a NaN at index 0 keeps index 0 (the reference's
 * best = l[0]; if (l[v] > best) ... loop, compute_layer_base.hpp:1152-1160; the reference
 * runs it on the softmax of the logits, which orders the same except where exp rounding
 * merges two nearly equal logits). */
nnhip_status nnhip_argmax_cols(nnhip_ctx* ctx, const float* logits, size_t V, size_t B, int32_t* ids);

/* nnhip_argmax_cols on token-major logits (B, V) (row b = sequence b's logits, read as one
 * contiguous row): the same ids as on the transpose. When pos != NULL, pos[b] += 1 for every
 * sequence after its choice, the position advance of the generation loop (GPTModel::generate,
 * compute_layer_gpt.hpp:800-849: the chosen token is fed back at the next position), so that a
 * captured decode step needs no separate position update; ids may then be the step's own input
 * ids (the embedding gather that read them ran earlier on the stream). */
nnhip_status nnhip_argmax_rows(nnhip_ctx* ctx, const float* logits, size_t V, size_t B, int32_t* ids, int32_t* pos);

/* Y = res + the gated block of nnhip_ffn_glu_i8 on X (res (d, M) f32, must not alias Y): the second
 * residual add of GPTBlock::forward_step in fc2's launch (decode GEMV or prefill GEMM epilogue). Same bits as
 * nnhip_ffn_glu_i8 then nnhip_add(res, Y) (compute_layer_gpt.hpp:212-218). */
nnhip_status nnhip_ffn_glu_i8_add(nnhip_ctx* ctx, const float* X, const float* gamma, float eps, size_t d, size_t F,
                                  size_t M, int act, const void* rp1, const float* tau1, const float* b1,
                                  const float* gamma_sub, float eps_sub, const void* rp2, const float* tau2,
                                  const float* b2, const float* res, float* Y);

#ifdef __cplusplus
}
#endif
#endif /* NNHIP_H */
