#pragma once
// compute_engine.hpp — nn::Tensor and the nn::ComputeEngine interface, the subset of the
// reference engine API that the BitLinear W1.58A8 path calls.
//
// Reference shape (compute_engine.hpp lives in the un-vendored engine submodule; the
// signatures below are reconstructed from its call sites, e.g.
// include/neuralnet.cpp/compute_layer_bitlinear.hpp:305, :443-456, :650,
// src/int8_act_test.cpp:106-204, src/ternary_gemm_test.cpp:224-320):
//   * public non-virtual entries (NVI) check the device domain, shapes and precision, then
//     call protected *_impl (docs/development/04-compute-engine-development.md:110-114);
//   * every result is a Result<T>; errors never throw (-fno-exceptions convention);
//   * Tensor is a value type with shared storage: a copy aliases the same device buffer;
//   * packed containers (ternary words, int8 words) are Precision::F32 tensors holding raw
//     32-bit words, transferred bitwise (docs/internal/21-quantized-weights.md:649-652);
//   * F16 tensors hold IEEE binary16 values (2 bytes each). The public entries of the
//     BitLinear products cast F16 operands to f32 and their f32 result to the requested
//     precision P (round to nearest even), the reference NVI's boundary cast
//     (docs/development/04-compute-engine-development.md:110-114); from_matrix / to_matrix
//     convert at the host boundary (to_matrix widens f16 exactly, src/test_common.hpp:84-91);
//   * every write entry advances the destination storage's write epoch, which BitLinear
//     uses to know when its quantized weights are stale (AGENTS.md:160-164).

#include <cstddef>
#include <cstdint>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "matrix.hpp"
#include "precision.hpp"
#include "result.hpp"

namespace nn
{

inline constexpr std::uint64_t kInitSeed = 0x5EEDB17Aull;

// Bytes per element of a tensor's storage (packed containers are F32 tensors of raw words).
[[nodiscard]] inline constexpr std::size_t element_bytes(Precision p) noexcept
{
    return p == Precision::F16 ? 2 : 4;
}

struct InitSpec
{
    enum class Kind : std::uint8_t { Zero, Constant, Uniform };
    Kind kind = Kind::Zero;
    float a = 0.0f, b = 0.0f;
    std::uint64_t seed = 0;
    [[nodiscard]] static InitSpec zero() noexcept { return {}; }
    [[nodiscard]] static InitSpec constant(float v) noexcept { return {Kind::Constant, v, 0.0f, 0}; }
    [[nodiscard]] static InitSpec uniform(double lo, double hi, std::uint64_t seed) noexcept
    {
        return {Kind::Uniform, static_cast<float>(lo), static_cast<float>(hi), seed};
    }
};

struct EngineInfo
{
    std::string engine;
    std::string device;
    bool ternary_gemm = false;          // trit_pack / matmul_q_i8 available
    bool int8_dot = false;              // int8 dot products available
    bool int8_dot_accelerated = false;  // ... on matrix hardware
    [[nodiscard]] std::string text() const
    {
        return engine + " on " + device + " | ternary_gemm=" + (ternary_gemm ? "yes" : "no") +
               " int8_dot=" + (int8_dot ? "yes" : "no") +
               " int8_dot_accelerated=" + (int8_dot_accelerated ? "yes" : "no");
    }
};

class ComputeEngine;

namespace detail
{
// Device storage shared by tensor copies. `mem` frees itself through the owning engine.
struct Storage
{
    std::shared_ptr<void> mem;
    std::size_t bytes = 0;
    const ComputeEngine* owner = nullptr;
    std::uint64_t write_epoch = 0;
    // Engine-private data derived from the contents (e.g. repacked weights); the engine records
    // the write epoch each derived piece was made from and remakes it when the epoch moved on.
    std::shared_ptr<void> derived;
};
}  // namespace detail

class Tensor
{
public:
    Tensor() = default;
    [[nodiscard]] bool valid() const noexcept { return static_cast<bool>(st_); }
    [[nodiscard]] std::size_t rows() const noexcept { return rows_; }
    [[nodiscard]] std::size_t cols() const noexcept { return cols_; }
    [[nodiscard]] std::size_t size() const noexcept { return rows_ * cols_; }
    [[nodiscard]] Precision precision() const noexcept { return p_; }
    [[nodiscard]] std::uint64_t write_epoch() const noexcept { return st_ ? st_->write_epoch : 0; }
    [[nodiscard]] bool same_storage(const Tensor& o) const noexcept { return st_ == o.st_; }

private:
    friend class TensorAccess;
    std::shared_ptr<detail::Storage> st_;
    std::size_t rows_ = 0, cols_ = 0;
    Precision p_ = Precision::F32;
};

// Reference to a tensor member (layers hand these to optimizers / serializers).
using TensorRef = std::reference_wrapper<Tensor>;

// Engine-side access to tensor internals. Layers and user code never need it.
class TensorAccess
{
public:
    [[nodiscard]] static Tensor make(std::shared_ptr<detail::Storage> st, std::size_t rows, std::size_t cols,
                                     Precision p)
    {
        Tensor t;
        t.st_ = std::move(st);
        t.rows_ = rows;
        t.cols_ = cols;
        t.p_ = p;
        return t;
    }
    [[nodiscard]] static detail::Storage* storage(const Tensor& t) noexcept { return t.st_.get(); }
    [[nodiscard]] static std::weak_ptr<detail::Storage> storage_ref(const Tensor& t) noexcept { return t.st_; }
    [[nodiscard]] static void* ptr(const Tensor& t) noexcept { return t.st_ ? t.st_->mem.get() : nullptr; }
    static void mark_written(const Tensor& t) noexcept
    {
        if (t.st_) ++t.st_->write_epoch;
    }
};

class ComputeEngine
{
public:
    virtual ~ComputeEngine() = default;
    ComputeEngine() = default;
    ComputeEngine(const ComputeEngine&) = delete;
    ComputeEngine& operator=(const ComputeEngine&) = delete;

    // ---- tensors and transfers
    [[nodiscard]] Tensor create_tensor(std::size_t rows, std::size_t cols, Precision p = Precision::F32,
                                       InitSpec init = InitSpec::zero());
    [[nodiscard]] Result<Tensor> from_matrix(const Matrix& m, Precision p = Precision::F32);
    [[nodiscard]] Result<Matrix> to_matrix(const Tensor& t, Precision p = Precision::F32);
    [[nodiscard]] Result<void> copy_from(Tensor& dst, const Matrix& src);
    // device-to-device copy of equal shapes (the layers' import_param uses it)
    [[nodiscard]] Result<void> copy_into(Tensor& dst, const Tensor& src);

    // ---- the BitLinear W1.58A8 primitives (reference names and semantics)
    [[nodiscard]] Result<Tensor> trit_pack(const Tensor& W, const Tensor& tau);
    [[nodiscard]] Result<void> trit_pack_into(const Tensor& W, const Tensor& tau, Tensor& out);
    // tau = per-row absmean of W (the reduction BitLinear runs through its DSL)
    [[nodiscard]] Result<void> row_absmean_into(const Tensor& W, Tensor& tau);
    [[nodiscard]] Result<Tensor> abs(const Tensor& x);
    [[nodiscard]] Result<Tensor> col_reduce_max(const Tensor& x, Precision p = Precision::F32);
    [[nodiscard]] Result<void> scale_inplace(Tensor& x, Scalar s);
    [[nodiscard]] Result<Tensor> quantize_i8(const Tensor& x, const Tensor& scale, bool col_scale);
    [[nodiscard]] Result<Tensor> unpack_i8(const Tensor& packed, std::size_t cols);
    [[nodiscard]] Result<Tensor> matmul_q_i8(const Tensor& wq, const Tensor& tau, const Tensor& xq, const Tensor& s,
                                             Precision p = Precision::F32);
    // Float-activation ternary products (compute_layer_bitlinear.hpp:464 forward, :494 dX):
    //   matmul_q   Y (N, M) = (tau o trit(wq)) . B,   wq (N, ceil(K/16)), B (K, M), tau (N, 1)
    //   matmul_q_t Y (M, N) = (tau o trit(A))^T . B,  A (K, ceil(M/16)),  B (K, N), tau (K, 1)
    [[nodiscard]] Result<Tensor> matmul_q(const Tensor& wq, const Tensor& tau, const Tensor& B,
                                          Precision p = Precision::F32);
    [[nodiscard]] Result<Tensor> matmul_q_t(const Tensor& A, const Tensor& tau, const Tensor& B, std::size_t M,
                                            Precision p = Precision::F32);
    // y + row_broadcast(b), computed in f32 and returned in y's precision
    [[nodiscard]] Result<Tensor> add_row_broadcast(const Tensor& y, const Tensor& b);
    // RMSNorm forward: (x * rsqrt(mean_f x^2 + eps)) * gamma, per column (token)
    [[nodiscard]] Result<Tensor> rmsnorm(const Tensor& x, const Tensor& gamma, Scalar eps);
    // LayerNorm forward: ((x - mean) * rsqrt(var + eps)) * gamma + beta, per column (token), with
    // the biased variance (include/neuralnet.cpp/compute_layer_mlp.hpp:529-545); x f32
    [[nodiscard]] Result<Tensor> layernorm(const Tensor& x, const Tensor& gamma, const Tensor& beta, Scalar eps);

    // Fused BitLinear int8 forward, the sequence of compute_layer_bitlinear.hpp:443-456:
    // s = col_reduce_max(|x|) * fl(1/127); xq = quantize_i8(x, s); y = matmul_q_i8(wq, tau, xq, s, p);
    // out = y + row_broadcast(b) in p. With p = F32 the bias rides in the product's epilogue (one
    // launch); with p = F16, y is rounded to f16 and the bias added to it in f32 and rounded
    // again, the reference's two steps. xq_out / s_out (nullable) receive the activation cache of
    // the reference layer. The default implementation composes the primitives; an engine may
    // fuse them.
    [[nodiscard]] Result<Tensor> bitlinear_i8_forward(const Tensor& x, const Tensor& wq, const Tensor& tau,
                                                      const Tensor& b, Precision p, Tensor* xq_out, Tensor* s_out);

    // Gated activation on a fused fc1 output y1 (2F, M): gate rows [0, F), up rows [F, 2F) ->
    // (F, M). act 0: SwiGLU (g * (1 / (1 + exp(-g)))) * u (compute_layer_mlp.hpp:317-328);
    // act 1: ReLU^2-GLU (r * r) * u, r = max(g, 0) (:405-414).
    [[nodiscard]] Result<Tensor> glu(const Tensor& y1, int act);

    // Gated feed-forward block in the int8 branch (FeedForward::forward,
    // compute_layer_feedforward.hpp:182-206): [RMSNorm(gamma, eps) if gamma] -> fc1 (BitLinear
    // int8, 2F rows: gate then up) -> glu -> [SubLN: RMSNorm(gamma_sub, eps_sub) if gamma_sub]
    // -> fc2 (BitLinear int8). The default implementation composes rmsnorm /
    // bitlinear_i8_forward / glu; an engine may fuse them (same bits).
    [[nodiscard]] Result<Tensor> ffn_glu_i8_forward(const Tensor& x, const Tensor* gamma, Scalar eps, const Tensor& wq1,
                                                    const Tensor& tau1, const Tensor& b1, const Tensor& wq2,
                                                    const Tensor& tau2, const Tensor& b2, int act,
                                                    const Tensor* gamma_sub = nullptr, Scalar eps_sub = 1e-5f);

    // ---- batched decode step (config C5): one new token for each of B sequences. Index tensors
    // (positions, token ids) are (B, 1) Precision::F32 containers of raw int32 words, like the
    // packed containers (upload_indices / download_indices below).
    // Decode attention, AttentionBase::forward_step steps 1.5-8 (compute_layer_attention.hpp:
    // 1022-1083) for B sequences: q (H*dk, B), k / v (Hkv*dk, B); the caches are
    // (B*max_len, Hkv*dk), sequence b's rows [b*max_len, (b+1)*max_len), and row pos[b] of each
    // sequence receives the rotated key / the value; rope tables (max_len, dk/2) or null;
    // len_bound >= every pos[b] + 1. Returns (H*dk, B).
    [[nodiscard]] Result<Tensor> attention_decode(const Tensor& q, const Tensor& k, const Tensor& v, Tensor& k_cache,
                                                  Tensor& v_cache, std::size_t max_len, const Tensor& positions,
                                                  std::size_t len_bound, const Tensor* rope_cos, const Tensor* rope_sin,
                                                  std::size_t heads, std::size_t kv_heads, Scalar scale);
    // x + y (the residual adds of GPTBlock::forward_step, compute_layer_gpt.hpp:208-218)
    [[nodiscard]] Result<Tensor> add(const Tensor& x, const Tensor& y);
    // t in precision p (F32 or F16): f16 -> f32 widens exactly, f32 -> f16 rounds to nearest even
    // (the reference's boundary cast); t itself when it already has p
    [[nodiscard]] Result<Tensor> cast(const Tensor& t, Precision p);
    // gather_rows(table, ids) + transpose (compute_layer_gpt.hpp:700-704): table (V, d) -> (d, B)
    [[nodiscard]] Result<Tensor> embedding_gather(const Tensor& table, const Tensor& ids);
    // greedy token per column of logits (V, B) (compute_layer_base.hpp:1152-1160) -> (B, 1) ids
    [[nodiscard]] Result<Tensor> argmax_cols(const Tensor& logits);

    [[nodiscard]] EngineInfo describe() const { return describe_impl(); }
    // Activation quantizations bitlinear_i8_forward has run (an engine may reuse the last one
    // for another BitLinear on the same input, e.g. the q / k / v projections). Diagnostic of
    // this engine layer; the reference has no counterpart.
    [[nodiscard]] virtual std::uint64_t activation_quantizations() const noexcept { return 0; }
    void begin_batch() {}
    void end_batch() { sync_impl(); }
    void flush_batch() { sync_impl(); }

protected:
    [[nodiscard]] virtual Result<Tensor> alloc_impl(std::size_t rows, std::size_t cols, Precision p) = 0;
    [[nodiscard]] virtual Result<void> upload_impl(const Tensor& dst, const void* src, std::size_t bytes) = 0;
    [[nodiscard]] virtual Result<void> download_impl(const Tensor& src, void* dst, std::size_t bytes) = 0;
    [[nodiscard]] virtual Result<void> copy_impl(const Tensor& dst, const Tensor& src, std::size_t bytes) = 0;
    [[nodiscard]] virtual Result<void> trit_pack_impl(const Tensor& W, const Tensor& tau, const Tensor& out) = 0;
    [[nodiscard]] virtual Result<void> row_absmean_impl(const Tensor& W, const Tensor& tau) = 0;
    [[nodiscard]] virtual Result<void> abs_impl(const Tensor& x, const Tensor& out) = 0;
    [[nodiscard]] virtual Result<void> col_reduce_max_impl(const Tensor& x, const Tensor& out) = 0;
    [[nodiscard]] virtual Result<void> scale_impl(const Tensor& x, Scalar s) = 0;
    [[nodiscard]] virtual Result<void> quantize_i8_impl(const Tensor& x, const Tensor& scale, bool col_scale,
                                                        const Tensor& out) = 0;
    [[nodiscard]] virtual Result<void> unpack_i8_impl(const Tensor& packed, std::size_t cols, const Tensor& out) = 0;
    [[nodiscard]] virtual Result<void> matmul_q_i8_impl(const Tensor& wq, const Tensor& tau, const Tensor& xq,
                                                        const Tensor& s, const Tensor& y) = 0;
    [[nodiscard]] virtual Result<void> matmul_q_impl(const Tensor& wq, const Tensor& tau, const Tensor& B,
                                                     const Tensor& y) = 0;
    [[nodiscard]] virtual Result<void> matmul_q_t_impl(const Tensor& A, const Tensor& tau, const Tensor& B,
                                                       std::size_t M, const Tensor& y) = 0;
    [[nodiscard]] virtual Result<void> add_row_broadcast_impl(const Tensor& y, const Tensor& b, const Tensor& out) = 0;
    [[nodiscard]] virtual Result<void> rmsnorm_impl(const Tensor& x, const Tensor& gamma, Scalar eps,
                                                    const Tensor& out) = 0;
    [[nodiscard]] virtual Result<void> layernorm_impl(const Tensor& x, const Tensor& gamma, const Tensor& beta,
                                                      Scalar eps, const Tensor& out) = 0;
    // b may be null (no bias); x is f32 here (the public entry casts f16 inputs)
    [[nodiscard]] virtual Result<Tensor> bitlinear_i8_impl(const Tensor& x, const Tensor& wq, const Tensor& tau,
                                                           const Tensor* b, Tensor* xq_out, Tensor* s_out);
    // elementwise precision cast between equal-shape tensors (F32 <-> F16)
    [[nodiscard]] virtual Result<void> convert_impl(const Tensor& src, const Tensor& dst) = 0;
    [[nodiscard]] virtual Result<void> glu_impl(const Tensor& y1, int act, const Tensor& out) = 0;
    [[nodiscard]] virtual Result<Tensor> ffn_glu_i8_impl(const Tensor& x, const Tensor* gamma, Scalar eps,
                                                         const Tensor& wq1, const Tensor& tau1, const Tensor& b1,
                                                         const Tensor& wq2, const Tensor& tau2, const Tensor& b2,
                                                         int act, const Tensor* gamma_sub, Scalar eps_sub);
    [[nodiscard]] virtual Result<void> attention_decode_impl(const Tensor& q, const Tensor& k, const Tensor& v,
                                                             const Tensor& k_cache, const Tensor& v_cache,
                                                             std::size_t max_len, const Tensor& positions,
                                                             std::size_t len_bound, const Tensor* rope_cos,
                                                             const Tensor* rope_sin, std::size_t heads,
                                                             std::size_t kv_heads, Scalar scale, const Tensor& out) = 0;
    [[nodiscard]] virtual Result<void> add_impl(const Tensor& x, const Tensor& y, const Tensor& out) = 0;
    [[nodiscard]] virtual Result<void> embedding_gather_impl(const Tensor& table, const Tensor& ids,
                                                             const Tensor& out) = 0;
    [[nodiscard]] virtual Result<void> argmax_cols_impl(const Tensor& logits, const Tensor& out) = 0;
    [[nodiscard]] virtual EngineInfo describe_impl() const = 0;
    virtual void sync_impl() = 0;

    // helpers for implementations
    [[nodiscard]] Result<void> check_owned(const Tensor& t, const char* what) const;
    // t as f32 (F16 tensors are widened into a new tensor; F32 tensors are returned as they are)
    [[nodiscard]] Result<Tensor> widen_f32(const Tensor& t);
    // an f32 result in precision p (rounded into a new F16 tensor when p is F16)
    [[nodiscard]] Result<Tensor> narrow_to(const Tensor& y32, Precision p);
};

// int32 index vectors (positions, token ids) as (n, 1) containers of raw words, and back
[[nodiscard]] inline Result<Tensor> upload_indices(ComputeEngine& engine, const std::int32_t* ids, std::size_t n)
{
    Matrix m(n, 1);
    if (n) std::memcpy(m.data(), ids, n * sizeof(std::int32_t));
    return engine.from_matrix(m, Precision::F32);
}

[[nodiscard]] inline Result<std::vector<std::int32_t>> download_indices(ComputeEngine& engine, const Tensor& t)
{
    EX_TRY(m, engine.to_matrix(t, Precision::F32));
    std::vector<std::int32_t> out(m->size());
    if (!out.empty()) std::memcpy(out.data(), m->data(), out.size() * sizeof(std::int32_t));
    return out;
}

}  // namespace nn
