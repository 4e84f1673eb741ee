#pragma once
// decoder.hpp — the decoder around the W1.58A8 path, for batched incremental decoding
// (config C5): nn::RotaryTable, nn::KVCache, nn::Embedding, nn::CausalSelfAttention,
// nn::GPTBlock and nn::GPTModel with forward_step / generate_greedy.
//
// Mirrors the reference's inference surface:
//   RotaryEmbedding      include/neuralnet.cpp/compute_position_encoding.hpp:45-166 (LLaMA
//                        half-swap tables, fill_pos_column_ in float)
//   CausalSelfAttention  include/neuralnet.cpp/compute_layer_attention.hpp:436-1127, 1163-1246
//                        (BitLinear q/k/v/o via make_linear_layer with WeightQuant::T1_58, GQA
//                        with block head map h -> h / (H / Hkv), optional SubLN before w_o,
//                        forward_step :1003-1091)
//   GPTBlock             include/neuralnet.cpp/compute_layer_gpt.hpp:26-235 (pre-norm residual
//                        blocks, forward_step :201-219)
//   GPTModel             include/neuralnet.cpp/compute_layer_gpt.hpp:237-866 (token embedding,
//                        blocks, final norm, BitLinear LM head; forward_step :693-724,
//                        greedy generation :741-851)
// Differences, each kept behind the reference's semantics:
//   * forward_step takes B sequences at once, each at its own position (the reference advances
//     one sequence of width 1); the single-sequence overloads keep the reference signature;
//   * the KV caches hold the Hkv KV heads (the reference expands them to H heads with
//     gather_rows before insert_rows; the expansion only duplicates rows), so a cache is
//     (B*max_len, Hkv*d_k) instead of (max_len, H*d_k);
//   * norms are RMSNorm and position encoding is RoPE or none (BitNet b1.58's choices); the
//     full-sequence training forward and the sliding-window cache rebuild are not provided
//     (decode only: generate_greedy refuses prompts + tokens beyond max_len);
//   * under compute = F16 (the t1_58 preset) the tensors the reference hands between layers in
//     the compute precision are f16 here too: the BitLinear outputs, the attention output, the
//     residual sums (x + a, r2 + f) and the KV caches; the norms (stable = F32) and the LM head
//     (compute = stable, compute_layer_gpt.hpp:335-337) give f32. Inside the attention the
//     scores, softmax and weighted sums run in f32 on the widened f16 operands (the reference
//     rounds them to f16 too), as do the gated activation and the residual additions before
//     their results are rounded.

#include <algorithm>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "layers.hpp"

namespace nn
{

namespace detail
{
// Parameter entries of a composite layer: its parts' entries in order.
inline std::size_t parts_param_count(const std::vector<Layer*>& parts)
{
    std::size_t n = 0;
    for (Layer* l : parts) n += l->param_count();
    return n;
}
inline Result<ParamEntry> parts_export(const std::vector<Layer*>& parts, std::size_t index, ModelRole role)
{
    for (Layer* l : parts)
    {
        const std::size_t n = l->param_count();
        if (index < n) return l->export_param(index, role);
        index -= n;
    }
    return Error{"export_param: index out of range"};
}
inline Result<void> parts_import(const std::vector<Layer*>& parts, std::size_t index, const ParamEntry& e)
{
    for (Layer* l : parts)
    {
        const std::size_t n = l->param_count();
        if (index < n) return l->import_param(index, e);
        index -= n;
    }
    return Error{"import_param: index out of range"};
}
inline std::vector<TensorRef> parts_parameters(const std::vector<Layer*>& parts)
{
    std::vector<TensorRef> r;
    for (Layer* l : parts)
    {
        auto p = l->parameters();
        r.insert(r.end(), p.begin(), p.end());
    }
    return r;
}
// A ternary composite takes any profile; its BitLinears get param T1_58, everything else f32
// (split_ternary_profile, include/neuralnet.cpp/compute_layer_base.hpp:151-164).
inline PrecisionProfile ternary_part(PrecisionProfile p)
{
    p.param = Precision::T1_58;
    return p;
}
inline PrecisionProfile float_part(PrecisionProfile p)
{
    p.param = Precision::F32;
    return p;
}
// The decoder takes compute = F32 or F16 (the reference's t1_58 preset, src/t1_58_test.cpp:668-690);
// act_precision is the precision of the activations handed between its layers.
inline PrecisionSet decoder_compute() { return PrecisionSet::of({Precision::F32, Precision::F16}); }
inline Precision act_precision(const PrecisionProfile& p)
{
    return p.compute == Precision::F16 ? Precision::F16 : Precision::F32;
}
}  // namespace detail

// KV cache of one attention layer for B sequences: rows [b*max_len, (b+1)*max_len) of k / v
// belong to sequence b; row b*max_len + t holds the (rotated) key / the value at position t.
struct KVCache
{
    Tensor k, v;
    std::size_t batch = 0, max_len = 0;
};

// RoPE tables (max_len, d_k/2): entry (pos, j) = cos / sin of pos / 10000^(2j/d_k), computed in
// float as RotaryEmbedding::fill_pos_column_ (compute_position_encoding.hpp:64-80), which
// stores each value for j and j + d_k/2; uploaded once.
class RotaryTable
{
public:
    [[nodiscard]] Result<void> build(ComputeEngine& engine, std::size_t d_k, std::size_t max_len)
    {
        if (d_k == 0 || d_k % 2 != 0) return Error{"RotaryTable: d_k must be positive and even"};
        const std::size_t half = d_k / 2;
        Matrix c(max_len, half), s(max_len, half);
        for (std::size_t pos = 0; pos < max_len; ++pos)
        {
            const Scalar pd = static_cast<Scalar>(pos);
            for (std::size_t j = 0; j < half; ++j)
            {
                const Scalar theta =
                    pd / std::pow(Scalar{10000}, static_cast<Scalar>(2 * j) / static_cast<Scalar>(d_k));
                c.set_value(pos, j, std::cos(theta));
                s.set_value(pos, j, std::sin(theta));
            }
        }
        EX_TRY(ct, engine.from_matrix(c));
        EX_TRY(st, engine.from_matrix(s));
        cos_ = *ct;
        sin_ = *st;
        return {};
    }
    [[nodiscard]] const Tensor& cos() const noexcept { return cos_; }
    [[nodiscard]] const Tensor& sin() const noexcept { return sin_; }

private:
    Tensor cos_, sin_;
};

// Token embedding table (V, d) (include/neuralnet.cpp/compute_layer_embedding.hpp), looked up
// by id; forward() takes a (B, 1) container of int32 ids and returns (d, B).
class Embedding final : public Layer
{
public:
    Embedding(std::size_t vocab, std::size_t dim) : vocab_(vocab), dim_(dim) {}
    [[nodiscard]] const char* layer_name() const noexcept override { return "Embedding"; }
    [[nodiscard]] std::vector<TensorRef> parameters() override { return {table_}; }
    [[nodiscard]] Tensor& table() noexcept { return table_; }
    [[nodiscard]] Result<Tensor> forward(const Tensor& ids) override { return engine_ref().embedding_gather(table_, ids); }

protected:
    [[nodiscard]] Result<void> init_impl(ComputeEngine& engine) override
    {
        table_ = engine.create_tensor(vocab_, dim_, Precision::F32, InitSpec::uniform(-0.1, 0.1, kInitSeed + 7));
        if (!table_.valid()) return Error{"Embedding: parameter init failed"};
        return {};
    }

private:
    std::size_t vocab_, dim_;
    Tensor table_;
};

// Causal self-attention with BitLinear projections, grouped-query heads and RoPE; incremental
// (KV-cache) inference only.
class CausalSelfAttention final : public Layer
{
public:
    CausalSelfAttention(std::size_t d_model, std::size_t num_heads, std::size_t max_len, std::size_t n_head_kv = 0,
                        bool rope = true, bool subln = false, bool inference_only = false)
        : d_model_(d_model), num_heads_(num_heads), n_head_kv_(n_head_kv == 0 ? num_heads : n_head_kv),
          d_k_(num_heads ? d_model / num_heads : 0), max_len_(max_len), rope_(rope),
          scale_(Scalar{1} / std::sqrt(static_cast<Scalar>(num_heads ? d_model / num_heads : 1))),
          w_q_(d_model, d_model, inference_only), w_k_(d_model, n_head_kv_ * d_k_, inference_only),
          w_v_(d_model, n_head_kv_ * d_k_, inference_only), w_o_(d_model, d_model, inference_only)
    {
        if (subln) sub_norm_ = std::make_unique<RMSNorm>(d_model);
    }

    [[nodiscard]] const char* layer_name() const noexcept override { return "CausalSelfAttention"; }
    [[nodiscard]] PrecisionSupport precision_support() const override
    {
        PrecisionSupport sup = PrecisionSupport::rounding_all_slots();
        sup.param.mask |= PrecisionSet::of({Precision::T1_58}).mask;
        sup.compute = detail::decoder_compute();
        return sup;
    }

    void set_activation_quant(bool enabled) noexcept
    {
        for (BitLinear* l : {&w_q_, &w_k_, &w_v_, &w_o_}) l->set_activation_quant(enabled);
    }
    [[nodiscard]] BitLinear& w_q() noexcept { return w_q_; }
    [[nodiscard]] BitLinear& w_k() noexcept { return w_k_; }
    [[nodiscard]] BitLinear& w_v() noexcept { return w_v_; }
    [[nodiscard]] BitLinear& w_o() noexcept { return w_o_; }
    [[nodiscard]] RMSNorm* sub_norm() noexcept { return sub_norm_.get(); }
    [[nodiscard]] std::size_t num_heads() const noexcept { return num_heads_; }
    [[nodiscard]] std::size_t kv_heads() const noexcept { return n_head_kv_; }
    [[nodiscard]] std::size_t d_k() const noexcept { return d_k_; }
    [[nodiscard]] std::size_t max_len() const noexcept { return max_len_; }
    [[nodiscard]] Scalar scale() const noexcept { return scale_; }
    [[nodiscard]] const RotaryTable* rotary() const noexcept { return rope_ ? &table_ : nullptr; }

    // q, k, v, o (weights, bias each), then the SubLN gain (compute_layer_attention.hpp:612-622)
    [[nodiscard]] std::vector<TensorRef> parameters() override { return detail::parts_parameters(parts_()); }
    [[nodiscard]] std::size_t param_count() override { return detail::parts_param_count(parts_()); }
    [[nodiscard]] Result<ParamEntry> export_param(std::size_t i, ModelRole role) override
    {
        return detail::parts_export(parts_(), i, role);
    }
    [[nodiscard]] Result<void> import_param(std::size_t i, const ParamEntry& e) override
    {
        return detail::parts_import(parts_(), i, e);
    }
    void clear_cache() override
    {
        for (BitLinear* l : {&w_q_, &w_k_, &w_v_, &w_o_}) l->clear_cache();
    }

    [[nodiscard]] Result<Tensor> forward(const Tensor&) override
    {
        return Error{"CausalSelfAttention: the full-sequence forward is not provided by this engine; "
                     "decode with forward_step"};
    }

    // Zero-filled caches for `batch` sequences, in the compute precision as the reference creates
    // them (compute_layer_gpt.hpp:764-765): f16 under compute = F16, else f32.
    [[nodiscard]] Result<KVCache> make_cache(std::size_t batch)
    {
        KVCache c;
        c.batch = batch;
        c.max_len = max_len_;
        const Precision cp = detail::act_precision(p_);
        c.k = engine_ref().create_tensor(batch * max_len_, n_head_kv_ * d_k_, cp, InitSpec::zero());
        c.v = engine_ref().create_tensor(batch * max_len_, n_head_kv_ * d_k_, cp, InitSpec::zero());
        if (!c.k.valid() || !c.v.valid()) return Error{"CausalSelfAttention: KV cache allocation failed"};
        return c;
    }

    // B sequences: x_new (d_model, B), positions (B, 1) int32 (each sequence's cache length so far),
    // len_bound > every position. Returns (d_model, B).
    [[nodiscard]] Result<Tensor> forward_step(ComputeEngine& engine, const Tensor& x_new, KVCache& cache,
                                              const Tensor& positions, std::size_t len_bound)
    {
        if (x_new.rows() != d_model_) return Error{"CausalSelfAttention forward_step: x_new must be (d_model, B)"};
        if (cache.batch != x_new.cols() || cache.max_len != max_len_)
            return Error{"CausalSelfAttention forward_step: cache does not match (batch " + std::to_string(cache.batch) +
                         ", max_len " + std::to_string(cache.max_len) + ")"};
        if (len_bound == 0 || len_bound > max_len_)
            return Error{"CausalSelfAttention forward_step: len_bound must be in [1, max_len]"};
        // 1. projections (the HIP engine quantizes x_new once for the three)
        EX_TRY(q, w_q_.forward(x_new));
        EX_TRY(k, w_k_.forward(x_new));
        EX_TRY(v, w_v_.forward(x_new));
        // 1.5-8. RoPE, cache append, scores, softmax, weighted values (f32 arithmetic; under
        // compute = F16 on the widened f16 projections and f16 caches, the output rounded to f16)
        const RotaryTable* rt = rotary();
        const Precision P = detail::act_precision(p_);
        EX_TRY(q32, engine.cast(*q, Precision::F32));
        EX_TRY(k32, engine.cast(*k, Precision::F32));
        EX_TRY(v32, engine.cast(*v, Precision::F32));
        EX_TRY(a32, engine.attention_decode(*q32, *k32, *v32, cache.k, cache.v, max_len_, positions, len_bound,
                                            rt ? &rt->cos() : nullptr, rt ? &rt->sin() : nullptr, num_heads_,
                                            n_head_kv_, scale_));
        // 9. SubLN (f32 in, f32 out), output projection
        if (sub_norm_)
        {
            if (P == Precision::F32)
            {
                EX_TRY(n, sub_norm_->forward(*a32));
                return w_o_.forward(*n);
            }
            EX_TRY(a16, engine.cast(*a32, P));
            EX_TRY(aw, engine.cast(*a16, Precision::F32));
            EX_TRY(n, sub_norm_->forward(*aw));
            return w_o_.forward(*n);
        }
        EX_TRY(a, engine.cast(*a32, P));
        return w_o_.forward(*a);
    }

    // The reference signature (compute_layer_attention.hpp:1003): one sequence, x_new (d_model, 1),
    // caches (max_len, Hkv*d_k), the new token at position cur_len.
    [[nodiscard]] Result<Tensor> forward_step(ComputeEngine& engine, const Tensor& x_new, Tensor& k_cache,
                                              Tensor& v_cache, std::size_t cur_len)
    {
        if (x_new.cols() != 1) return Error{"CausalSelfAttention forward_step: x_new must be (d_model, 1)"};
        if (cur_len >= max_len_) return Error{"CausalSelfAttention forward_step: cur_len beyond max_len"};
        const std::int32_t p = static_cast<std::int32_t>(cur_len);
        EX_TRY(pos, upload_indices(engine, &p, 1));
        KVCache c{k_cache, v_cache, 1, max_len_};
        EX_TRY(y, forward_step(engine, x_new, c, *pos, cur_len + 1));
        return *y;
    }

protected:
    [[nodiscard]] Result<void> init_impl(ComputeEngine& engine) override
    {
        if (num_heads_ == 0 || d_model_ % num_heads_ != 0)
            return Error{"CausalSelfAttention: d_model must be divisible by num_heads"};
        if (n_head_kv_ == 0 || num_heads_ % n_head_kv_ != 0)
            return Error{"CausalSelfAttention: num_heads must be divisible by n_head_kv"};
        for (BitLinear* l : {&w_q_, &w_k_, &w_v_, &w_o_})
        {
            l->set_precision_profile(detail::ternary_part(p_));
            EX_TRY_CHECK(l->init(engine));
        }
        if (sub_norm_)
        {
            sub_norm_->set_precision_profile(detail::float_part(p_));
            EX_TRY_CHECK(sub_norm_->init(engine));
        }
        if (rope_) EX_TRY_CHECK(table_.build(engine, d_k_, max_len_));
        return {};
    }

private:
    std::vector<Layer*> parts_()
    {
        std::vector<Layer*> p{&w_q_, &w_k_, &w_v_, &w_o_};
        if (sub_norm_) p.push_back(sub_norm_.get());
        return p;
    }

    std::size_t d_model_, num_heads_, n_head_kv_, d_k_, max_len_;
    bool rope_;
    Scalar scale_;
    BitLinear w_q_, w_k_, w_v_, w_o_;
    std::unique_ptr<RMSNorm> sub_norm_;
    RotaryTable table_;
};

// Pre-norm decoder block: x = x + attn(norm1(x)); x = x + ffn(norm2(x)).
class GPTBlock final : public Layer
{
public:
    GPTBlock(std::size_t d_model, std::size_t num_heads, std::size_t d_ff, std::size_t max_len,
             std::size_t n_head_kv = 0, ActivationType activation = ActivationType::SwiGLU, bool subln = false,
             Scalar norm_eps = 1e-5f, bool inference_only = false)
        : attn_(d_model, num_heads, max_len, n_head_kv, true, subln, inference_only), norm1_(d_model, norm_eps),
          ff_(d_model, d_ff, activation, subln, NormType::RMSNorm, WeightQuant::T1_58, inference_only),
          norm2_(d_model, norm_eps)
    {
    }

    [[nodiscard]] const char* layer_name() const noexcept override { return "GPTBlock"; }
    [[nodiscard]] PrecisionSupport precision_support() const override
    {
        PrecisionSupport sup = PrecisionSupport::rounding_all_slots();
        sup.param.mask |= PrecisionSet::of({Precision::T1_58}).mask;
        sup.compute = detail::decoder_compute();
        return sup;
    }
    void set_activation_quant(bool enabled) noexcept
    {
        attn_.set_activation_quant(enabled);
        ff_.set_activation_quant(enabled);
    }
    [[nodiscard]] CausalSelfAttention& attention() noexcept { return attn_; }
    [[nodiscard]] FeedForward& feed_forward() noexcept { return ff_; }
    [[nodiscard]] RMSNorm& norm1() noexcept { return norm1_; }
    [[nodiscard]] RMSNorm& norm2() noexcept { return norm2_; }

    // attention, norm1, feed-forward, norm2 (compute_layer_gpt.hpp:89-93)
    [[nodiscard]] std::vector<TensorRef> parameters() override { return detail::parts_parameters(parts_()); }
    [[nodiscard]] std::size_t param_count() override { return detail::parts_param_count(parts_()); }
    [[nodiscard]] Result<ParamEntry> export_param(std::size_t i, ModelRole role) override
    {
        return detail::parts_export(parts_(), i, role);
    }
    [[nodiscard]] Result<void> import_param(std::size_t i, const ParamEntry& e) override
    {
        return detail::parts_import(parts_(), i, e);
    }
    void clear_cache() override
    {
        attn_.clear_cache();
        ff_.clear_cache();
    }

    [[nodiscard]] Result<Tensor> forward(const Tensor&) override
    {
        return Error{"GPTBlock: the full-sequence forward is not provided by this engine; decode with forward_step"};
    }

    // compute_layer_gpt.hpp:201-219 for B sequences: x (d_model, B) -> (d_model, B)
    [[nodiscard]] Result<Tensor> forward_step(ComputeEngine& engine, const Tensor& x, KVCache& cache,
                                              const Tensor& positions, std::size_t len_bound)
    {
        const Precision P = detail::act_precision(p_);
        if (P == Precision::F32)
        {
            EX_TRY(n1, norm1_.forward(x));
            EX_TRY(a, attn_.forward_step(engine, *n1, cache, positions, len_bound));
            EX_TRY(r2, engine.add(x, *a));
            // norm2 -> FFN; with int8 activations the engine runs the norm inside the fused block
            EX_TRY(f, ff_.forward_with_norm(*r2, norm2_));
            return engine.add(*r2, *f);
        }
        // compute = F16: x, the attention and FFN outputs and both residual sums are f16; each sum
        // is taken in f32 on the widened operands and rounded once (:208-216)
        EX_TRY(xw, engine.cast(x, Precision::F32));
        EX_TRY(n1, norm1_.forward(*xw));
        EX_TRY(a, attn_.forward_step(engine, *n1, cache, positions, len_bound));
        EX_TRY(aw, engine.cast(*a, Precision::F32));
        EX_TRY(s1, engine.add(*xw, *aw));
        EX_TRY(r2, engine.cast(*s1, P));
        EX_TRY(r2w, engine.cast(*r2, Precision::F32));
        EX_TRY(n2, norm2_.forward(*r2w));
        EX_TRY(f, ff_.forward(*n2));
        EX_TRY(fw, engine.cast(*f, Precision::F32));
        EX_TRY(s2, engine.add(*r2w, *fw));
        return engine.cast(*s2, P);
    }

protected:
    [[nodiscard]] Result<void> init_impl(ComputeEngine& engine) override
    {
        attn_.set_precision_profile(p_);
        ff_.set_precision_profile(p_);
        norm1_.set_precision_profile(detail::float_part(p_));
        norm2_.set_precision_profile(detail::float_part(p_));
        EX_TRY_CHECK(attn_.init(engine));
        EX_TRY_CHECK(norm1_.init(engine));
        EX_TRY_CHECK(ff_.init(engine));
        EX_TRY_CHECK(norm2_.init(engine));
        return {};
    }

private:
    std::vector<Layer*> parts_() { return {&attn_, &norm1_, &ff_, &norm2_}; }

    CausalSelfAttention attn_;
    RMSNorm norm1_;
    FeedForward ff_;
    RMSNorm norm2_;
};

// Decoder-only language model: token embedding, blocks, final RMSNorm, BitLinear LM head.
class GPTModel final : public Layer
{
public:
    GPTModel(std::size_t vocab_size, std::size_t d_model, std::size_t max_len, std::size_t num_heads,
             std::size_t d_ff, std::size_t num_layers, std::size_t n_head_kv = 0,
             ActivationType activation = ActivationType::SwiGLU, bool subln = false, Scalar norm_eps = 1e-5f,
             bool inference_only = false)
        : vocab_(vocab_size), d_model_(d_model), max_len_(max_len), emb_(vocab_size, d_model),
          ln_f_(d_model, norm_eps), head_(d_model, vocab_size, inference_only)
    {
        for (std::size_t i = 0; i < num_layers; ++i)
            blocks_.push_back(std::make_unique<GPTBlock>(d_model, num_heads, d_ff, max_len, n_head_kv, activation, subln,
                                                         norm_eps, inference_only));
    }

    [[nodiscard]] const char* layer_name() const noexcept override { return "GPTModel"; }
    [[nodiscard]] PrecisionSupport precision_support() const override
    {
        PrecisionSupport sup = PrecisionSupport::rounding_all_slots();
        sup.param.mask |= PrecisionSet::of({Precision::T1_58}).mask;
        sup.compute = detail::decoder_compute();
        return sup;
    }
    void set_activation_quant(bool enabled) noexcept
    {
        for (auto& b : blocks_) b->set_activation_quant(enabled);
        head_.set_activation_quant(enabled);
    }
    [[nodiscard]] std::size_t num_layers() const noexcept { return blocks_.size(); }
    [[nodiscard]] GPTBlock& block(std::size_t i) noexcept { return *blocks_[i]; }
    [[nodiscard]] Embedding& embedding() noexcept { return emb_; }
    [[nodiscard]] RMSNorm& final_norm() noexcept { return ln_f_; }
    [[nodiscard]] BitLinear& lm_head() noexcept { return head_; }
    [[nodiscard]] std::size_t vocab_size() const noexcept { return vocab_; }
    [[nodiscard]] std::size_t d_model() const noexcept { return d_model_; }
    [[nodiscard]] std::size_t max_len() const noexcept { return max_len_; }

    // embedding, blocks, final norm, LM head
    [[nodiscard]] std::vector<TensorRef> parameters() override { return detail::parts_parameters(parts_()); }
    [[nodiscard]] std::size_t param_count() override { return detail::parts_param_count(parts_()); }
    [[nodiscard]] Result<ParamEntry> export_param(std::size_t i, ModelRole role) override
    {
        return detail::parts_export(parts_(), i, role);
    }
    [[nodiscard]] Result<void> import_param(std::size_t i, const ParamEntry& e) override
    {
        return detail::parts_import(parts_(), i, e);
    }

    [[nodiscard]] Result<Tensor> forward(const Tensor&) override
    {
        return Error{"GPTModel: the full-sequence forward is not provided by this engine; decode with forward_step"};
    }

    // One zero-filled cache per block for `batch` sequences.
    [[nodiscard]] Result<std::vector<KVCache>> make_caches(std::size_t batch)
    {
        std::vector<KVCache> caches;
        for (auto& b : blocks_)
        {
            EX_TRY(c, b->attention().make_cache(batch));
            caches.push_back(*c);
        }
        return caches;
    }

    // compute_layer_gpt.hpp:693-724 for B sequences: ids / positions (B, 1) int32 containers,
    // len_bound > every position. Returns logits (vocab, B).
    [[nodiscard]] Result<Tensor> forward_step(ComputeEngine& engine, const Tensor& ids, const Tensor& positions,
                                              std::size_t len_bound, std::vector<KVCache>& caches)
    {
        if (caches.size() != blocks_.size()) return Error{"GPTModel forward_step: one cache per block expected"};
        EX_TRY(x0, emb_.forward(ids));
        Tensor x = *x0;
        for (std::size_t i = 0; i < blocks_.size(); ++i)
        {
            auto r = blocks_[i]->forward_step(engine, x, caches[i], positions, len_bound);
            if (!r) return Error{"GPTBlock " + std::to_string(i) + ": " + r.error().message};
            x = *r;
        }
        EX_TRY(xw, engine.cast(x, Precision::F32));
        EX_TRY(n, ln_f_.forward(*xw));
        return head_.forward(*n);
    }

    // The reference signature (:693): one sequence, one token at position cur_len.
    [[nodiscard]] Result<Tensor> forward_step(ComputeEngine& engine, std::size_t token_id, std::size_t cur_len,
                                              std::vector<KVCache>& caches)
    {
        const std::int32_t id = static_cast<std::int32_t>(token_id), p = static_cast<std::int32_t>(cur_len);
        if (cur_len >= max_len_) return Error{"GPTModel forward_step: cur_len beyond max_len"};
        EX_TRY(ids, upload_indices(engine, &id, 1));
        EX_TRY(pos, upload_indices(engine, &p, 1));
        return forward_step(engine, *ids, *pos, cur_len + 1, caches);
    }

    // Greedy generation for B prompts in lockstep (temperature <= 0 in the reference sampler,
    // :741-851): step s feeds each sequence its prompt token s while it has one and its own
    // greedy choice afterwards, at position s; sequence b's output is the max_new_tokens tokens
    // chosen after its prompt. Prompts must be non-empty and every prompt plus max_new_tokens
    // must fit max_len (no sliding window).
    [[nodiscard]] Result<std::vector<std::vector<std::int32_t>>>
    generate_greedy(ComputeEngine& engine, const std::vector<std::vector<std::int32_t>>& prompts,
                    std::size_t max_new_tokens)
    {
        const std::size_t B = prompts.size();
        if (B == 0) return std::vector<std::vector<std::int32_t>>{};
        std::size_t longest = 0;
        for (const auto& p : prompts)
        {
            if (p.empty()) return Error{"generate_greedy: empty prompt"};
            longest = std::max(longest, p.size());
        }
        if (longest + max_new_tokens > max_len_) return Error{"generate_greedy: prompt + new tokens exceed max_len"};
        EX_TRY(caches, make_caches(B));
        std::vector<std::vector<std::int32_t>> out(B);
        std::vector<std::int32_t> cur(B), pos(B);
        const std::size_t steps = longest + max_new_tokens - 1;
        for (std::size_t s = 0; s < steps; ++s)
        {
            for (std::size_t b = 0; b < B; ++b)
            {
                if (s < prompts[b].size()) cur[b] = prompts[b][s];
                pos[b] = static_cast<std::int32_t>(s);
            }
            EX_TRY(ids, upload_indices(engine, cur.data(), B));
            EX_TRY(pt, upload_indices(engine, pos.data(), B));
            EX_TRY(logits, forward_step(engine, *ids, *pt, s + 1, *caches));
            EX_TRY(lw, engine.cast(*logits, Precision::F32));
            EX_TRY(next_t, engine.argmax_cols(*lw));
            EX_TRY(next, download_indices(engine, *next_t));
            for (std::size_t b = 0; b < B; ++b)
            {
                if (s + 1 < prompts[b].size()) continue;   // still reading its prompt
                if (out[b].size() < max_new_tokens) out[b].push_back((*next)[b]);
                cur[b] = (*next)[b];
            }
        }
        return out;
    }

protected:
    [[nodiscard]] Result<void> init_impl(ComputeEngine& engine) override
    {
        emb_.set_precision_profile(detail::float_part(p_));
        EX_TRY_CHECK(emb_.init(engine));
        for (auto& b : blocks_)
        {
            b->set_precision_profile(p_);
            EX_TRY_CHECK(b->init(engine));
        }
        ln_f_.set_precision_profile(detail::float_part(p_));
        EX_TRY_CHECK(ln_f_.init(engine));
        // the LM head computes in the stable precision (f32 logits under t1_58), as the
        // reference's head profile does (compute_layer_gpt.hpp:335-337)
        PrecisionProfile hp = detail::ternary_part(p_);
        hp.compute = p_.stable;
        head_.set_precision_profile(hp);
        EX_TRY_CHECK(head_.init(engine));
        return {};
    }

private:
    std::vector<Layer*> parts_()
    {
        std::vector<Layer*> p{&emb_};
        for (auto& b : blocks_) p.push_back(b.get());
        p.push_back(&ln_f_);
        p.push_back(&head_);
        return p;
    }

    std::size_t vocab_, d_model_, max_len_;
    Embedding emb_;
    std::vector<std::unique_ptr<GPTBlock>> blocks_;
    RMSNorm ln_f_;
    BitLinear head_;
};

}  // namespace nn
