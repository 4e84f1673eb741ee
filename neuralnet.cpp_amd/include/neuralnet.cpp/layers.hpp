#pragma once
// layers.hpp — nn::Layer, nn::BitLinear, nn::FeedForward and nn::RMSNorm: the layer side of
// the W1.58A8 path.
//
// Mirrors the reference classes' public surface and semantics for the inference path:
//   Layer      include/neuralnet.cpp/compute_layer_base.hpp:261-363 (init -> init_impl NVI,
//              precision profile fixed at init, forward)
//   BitLinear  include/neuralnet.cpp/compute_layer_bitlinear.hpp:46-675
//   FeedForward include/neuralnet.cpp/compute_layer_feedforward.hpp:22-204 (gated activations)
//   RMSNorm    include/neuralnet.cpp/compute_layer_mlp.hpp:627-707
// BitLinear keeps the reference's weight-side state machine: f32 latent weights, per-row
// absmean tau and the packed ternary container recomputed only when the latent storage's
// write epoch changed (:100-111, :607-674), and the packed-only deploy state loaded with
// load_packed_weights (:359-380). forward() runs the int8 branch (set_activation_quant(true),
// :441-457) through ComputeEngine::bitlinear_i8_forward; with activation quantization off it
// runs the f32-activation branch (:459-466) through ComputeEngine::matmul_q. Training
// (backward, STE gradients) is outside this engine's scope.

#include <memory>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

#include "compute_engine.hpp"
#include "ternary_pack.hpp"

namespace nn
{

// Parameter entry protocol of the v7+ model files (include/neuralnet.cpp/compute_layer_base.hpp:193-208,
// :425-533): every layer exposes its parameters by index as entries of one kind.
enum class ParamKind : std::uint8_t
{
    Dense = 0,           // plain float parameter (bias, norm gain, ...)
    TernaryLatent = 1,   // BitLinear f32 latent weights (checkpoint files)
    TernaryPacked2 = 2,  // BitLinear 2-bit container + tau (the run-time form)
    TernaryPacked3 = 3,  // base-3 on-disk form of the same (1.6 bpw)
    I8Packed4 = 4,       // reserved
};

[[nodiscard]] inline const char* param_kind_name(ParamKind k) noexcept
{
    switch (k)
    {
    case ParamKind::Dense: return "Dense";
    case ParamKind::TernaryLatent: return "TernaryLatent";
    case ParamKind::TernaryPacked2: return "TernaryPacked2";
    case ParamKind::TernaryPacked3: return "TernaryPacked3";
    case ParamKind::I8Packed4: return "I8Packed4";
    }
    return "?";
}

// File role byte: Model = inference file (.nnmodel, ternary layers packed), Checkpoint =
// training file (.nnckpt, ternary layers as f32 latents).
enum class ModelRole : std::uint8_t
{
    Model = 0,
    Checkpoint = 1,
};

struct ParamEntry
{
    ParamKind kind = ParamKind::Dense;
    Precision precision = Precision::F32;
    std::size_t rows = 0, cols = 0;  // logical shape (for packed kinds: out x in features)
    Tensor payload;                  // values, latent, or packed words (raw u32 in an f32 tensor)
    Tensor aux;                      // tau (rows, 1) for the ternary kinds
};

class Layer
{
public:
    virtual ~Layer() = default;
    [[nodiscard]] virtual const char* layer_name() const noexcept = 0;
    [[nodiscard]] virtual PrecisionSupport precision_support() const { return PrecisionSupport::rounding_all_slots(); }

    // The profile is fixed before init (setting it afterwards aborts, compute_layer_base.hpp:193-259).
    void set_precision_profile(const PrecisionProfile& p)
    {
        EX_UNWRAP(engine_ == nullptr, std::string(layer_name()) + ": set_precision_profile after init");
        p_ = p;
    }
    [[nodiscard]] const PrecisionProfile& precision_profile() const noexcept { return p_; }

    [[nodiscard]] Result<void> init(ComputeEngine& engine)
    {
        const PrecisionSupport sup = precision_support();
        if (!sup.param.has(p_.param))
            return Error{std::string(layer_name()) + ": param precision " + precision_name(p_.param) +
                         " not supported (supported: " + sup.param.to_string() + ")"};
        if (!sup.compute.has(p_.compute))
            return Error{std::string(layer_name()) + ": compute precision " + precision_name(p_.compute) +
                         " not supported (supported: " + sup.compute.to_string() + ")"};
        engine_ = &engine;
        return init_impl(engine);
    }

    [[nodiscard]] virtual Result<Tensor> forward(const Tensor& input) = 0;
    [[nodiscard]] virtual Result<Tensor> backward(const Tensor&)
    {
        return Error{std::string(layer_name()) + ": backward is not provided by this inference engine"};
    }
    [[nodiscard]] virtual std::vector<TensorRef> parameters() { return {}; }
    virtual void clear_cache() {}

    // Parameter entries by index (the model file's order). Default: every parameter is Dense.
    [[nodiscard]] virtual std::size_t param_count() { return parameters().size(); }
    [[nodiscard]] virtual Result<ParamEntry> export_param(std::size_t index, ModelRole /*role*/)
    {
        auto ps = parameters();
        if (index >= ps.size()) return Error{std::string("export_param: index out of range (layer ") + layer_name() + ")"};
        return dense_entry_(ps[index].get());
    }
    [[nodiscard]] virtual Result<void> import_param(std::size_t index, const ParamEntry& e)
    {
        if (e.kind != ParamKind::Dense)
            return Error{std::string("import_param: layer ") + layer_name() + " takes Dense entries, got " +
                         param_kind_name(e.kind)};
        auto ps = parameters();
        if (index >= ps.size()) return Error{std::string("import_param: index out of range (layer ") + layer_name() + ")"};
        return import_into_(ps[index].get(), e);
    }

protected:
    [[nodiscard]] virtual Result<void> init_impl(ComputeEngine& engine) = 0;
    [[nodiscard]] ComputeEngine& engine_ref() const noexcept { return *engine_; }

    [[nodiscard]] static ParamEntry dense_entry_(const Tensor& t)
    {
        ParamEntry e;
        e.kind = ParamKind::Dense;
        e.precision = t.precision();
        e.rows = t.rows();
        e.cols = t.cols();
        e.payload = t;
        return e;
    }
    [[nodiscard]] Result<void> import_into_(Tensor& dst, const ParamEntry& e)
    {
        if (e.rows != dst.rows() || e.cols != dst.cols() || !e.payload.valid())
            return Error{std::string("import_param: shape mismatch (layer ") + layer_name() + ", expected " +
                         std::to_string(dst.rows()) + "x" + std::to_string(dst.cols()) + ", got " +
                         std::to_string(e.rows) + "x" + std::to_string(e.cols) + ")"};
        return engine_ref().copy_into(dst, e.payload);
    }
    PrecisionProfile p_{};

private:
    ComputeEngine* engine_ = nullptr;
};

class BitLinear final : public Layer
{
public:
    BitLinear(std::size_t in_features, std::size_t out_features, bool inference_only = false)
        : in_features_(in_features), out_features_(out_features), inference_only_(inference_only)
    {
    }

    [[nodiscard]] const char* layer_name() const noexcept override { return "BitLinear"; }

    [[nodiscard]] PrecisionSupport precision_support() const override
    {
        PrecisionSupport sup = PrecisionSupport::rounding_all_slots();
        sup.param = PrecisionSet::of({Precision::T1_58});
        return sup;
    }

    // int8 activation quantization (W1.58A8): s = per-token absmax/127 (:181-189)
    void set_activation_quant(bool enabled) noexcept { act_quant_ = enabled; }
    [[nodiscard]] bool activation_quant() const noexcept { return act_quant_; }

    [[nodiscard]] std::vector<TensorRef> parameters() override
    {
        std::vector<TensorRef> r;
        if (latent_w_.valid()) r.emplace_back(latent_w_);
        r.emplace_back(b_);
        return r;
    }

    [[nodiscard]] const Tensor& latent_weights() const noexcept { return latent_w_; }
    [[nodiscard]] const Tensor& row_scales() const noexcept { return tau_; }
    [[nodiscard]] const Tensor& bias() const noexcept { return b_; }
    [[nodiscard]] bool uses_packed_weights() const noexcept { return true; }
    [[nodiscard]] const Tensor& quantized_weights_packed() const noexcept { return wq_packed_; }
    [[nodiscard]] std::uint64_t quantize_calls() const noexcept { return quantize_calls_; }
    [[nodiscard]] bool packed_only() const noexcept { return packed_only_; }
    [[nodiscard]] std::size_t in_features() const noexcept { return in_features_; }
    [[nodiscard]] std::size_t out_features() const noexcept { return out_features_; }
    // activation cache: the int8 branch keeps the packed int8 input (K, ceil(M/4)) and its scales
    // (1, M); the f32 branch keeps the input itself and no scales
    [[nodiscard]] const Tensor& input_cache() const noexcept { return input_cache_; }
    [[nodiscard]] const Tensor& activation_scales() const noexcept { return act_scale_; }

    // Entries (compute_layer_bitlinear.hpp:221-339): 0 = weights, 1 = bias (Dense). Weights go
    // out as TernaryPacked2 (words + tau) in an inference file and as TernaryLatent in a
    // checkpoint; they come in as either.
    [[nodiscard]] std::size_t param_count() override { return 2; }

    [[nodiscard]] Result<ParamEntry> export_param(std::size_t index, ModelRole role) override
    {
        if (index == 1) return dense_entry_(b_);
        if (index != 0) return Error{"BitLinear::export_param: index must be 0 or 1"};
        ParamEntry e;
        e.rows = out_features_;
        e.cols = in_features_;
        e.precision = Precision::F32;
        if (role == ModelRole::Checkpoint)
        {
            if (!latent_w_.valid())
                return Error{"BitLinear::export_param: a deploy-state layer has no latent weights for a checkpoint"};
            e.kind = ParamKind::TernaryLatent;
            e.payload = latent_w_;
            return e;
        }
        EX_TRY_CHECK(ensure_quantized());
        e.kind = ParamKind::TernaryPacked2;
        e.payload = wq_packed_;
        e.aux = tau_;
        return e;
    }

    [[nodiscard]] Result<void> import_param(std::size_t index, const ParamEntry& e) override
    {
        if (index == 1)
        {
            if (e.kind != ParamKind::Dense)
                return Error{std::string("BitLinear::import_param: the bias must be Dense, got ") + param_kind_name(e.kind)};
            return import_into_(b_, e);
        }
        if (index != 0) return Error{"BitLinear::import_param: index must be 0 or 1"};
        if (e.rows != out_features_ || e.cols != in_features_)
            return Error{"BitLinear::import_param: entry is " + std::to_string(e.rows) + "x" + std::to_string(e.cols) +
                         ", layer is " + std::to_string(out_features_) + "x" + std::to_string(in_features_)};
        switch (e.kind)
        {
        case ParamKind::TernaryPacked2:
            return load_packed_weights(e.payload, e.aux);
        case ParamKind::TernaryLatent:
        {
            if (!latent_w_.valid())
            {
                // back from the deploy state: a fresh latent and quantization buffers
                latent_w_ = engine_ref().create_tensor(out_features_, in_features_, Precision::F32, InitSpec::zero());
                wq_packed_ = engine_ref().create_tensor(out_features_, trit_pack::words_per_row(in_features_),
                                                        Precision::F32, InitSpec::zero());
                tau_ = engine_ref().create_tensor(out_features_, 1, Precision::F32, InitSpec::zero());
                if (!latent_w_.valid() || !wq_packed_.valid() || !tau_.valid())
                    return Error{"BitLinear::import_param: latent allocation failed"};
                packed_only_ = false;
            }
            quant_valid_ = false;
            return import_into_(latent_w_, e);
        }
        default:
            return Error{std::string("BitLinear::import_param: entry kind ") + param_kind_name(e.kind) +
                         " is not accepted (TernaryLatent, TernaryPacked2)"};
        }
    }

    // Deploy state: packed words + tau replace the latent weights (read-only inference).
    [[nodiscard]] Result<void> load_packed_weights(Tensor packed_words, Tensor tau)
    {
        if (!packed_words.valid() || !tau.valid()) return Error{"BitLinear: empty deploy tensors"};
        if (packed_words.rows() != out_features_ || packed_words.cols() != trit_pack::words_per_row(in_features_))
            return Error{"BitLinear: packed word shape mismatch (expected " + std::to_string(out_features_) + "x" +
                         std::to_string(trit_pack::words_per_row(in_features_)) + ")"};
        if (tau.rows() != out_features_ || tau.cols() != 1)
            return Error{"BitLinear: tau shape mismatch (expected " + std::to_string(out_features_) + "x1)"};
        wq_packed_ = std::move(packed_words);
        tau_ = std::move(tau);
        quant_valid_ = true;
        packed_only_ = true;
        latent_w_ = Tensor{};
        return {};
    }

    [[nodiscard]] Result<void> ensure_quantized()
    {
        if (needs_quantize_()) return quantize_weights_();
        return {};
    }

    void clear_cache() override
    {
        input_cache_ = Tensor{};
        act_scale_ = Tensor{};
    }

    [[nodiscard]] Result<Tensor> forward(const Tensor& input) override
    {
        ComputeEngine& engine = engine_ref();
        if (input.rows() != in_features_) return Error{"bitlinear forward: input shape mismatch"};
        if (packed_only_ && !(wq_packed_.valid() && tau_.valid()))
            return Error{"BitLinear(packed-only): deploy weights / tau missing"};
        if (needs_quantize_()) EX_TRY_CHECK(quantize_weights_());
        // the compute slot sets the precision of the product and of the bias add (:454-456, :464-466)
        const Precision P = p_.compute == Precision::F16 ? Precision::F16 : Precision::F32;
        if (!act_quant_)
        {
            // float-activation branch (:459-466): one ternary x float product, then the bias.
            input_cache_ = input;
            act_scale_ = Tensor{};
            EX_TRY(y, engine.matmul_q(wq_packed_, tau_, input, P));
            return engine.add_row_broadcast(*y, b_);
        }
        Tensor xq, s;
        EX_TRY(y, engine.bitlinear_i8_forward(input, wq_packed_, tau_, b_, P, &xq, &s));
        input_cache_ = xq;
        act_scale_ = s;
        return *y;
    }

protected:
    [[nodiscard]] Result<void> init_impl(ComputeEngine& engine) override
    {
        if (inference_only_) packed_only_ = true;
        if (!packed_only_)
        {
            const double limit = std::sqrt(6.0 / static_cast<double>(in_features_ + out_features_));
            latent_w_ = engine.create_tensor(out_features_, in_features_, Precision::F32,
                                             InitSpec::uniform(-limit, limit, kInitSeed));
            if (!latent_w_.valid()) return Error{"BitLinear: latent weight init failed"};
            wq_packed_ = engine.create_tensor(out_features_, trit_pack::words_per_row(in_features_),
                                              Precision::F32, InitSpec::zero());
            tau_ = engine.create_tensor(out_features_, 1, Precision::F32, InitSpec::zero());
            if (!wq_packed_.valid() || !tau_.valid()) return Error{"BitLinear: quantization buffer init failed"};
        }
        b_ = engine.create_tensor(out_features_, 1, Precision::F32, InitSpec::zero());
        if (!b_.valid()) return Error{"BitLinear: bias init failed"};
        return {};
    }

private:
    [[nodiscard]] bool needs_quantize_() const noexcept
    {
        if (packed_only_) return !(wq_packed_.valid() && tau_.valid());
        if (!quant_valid_) return true;
        return quant_epoch_ != latent_w_.write_epoch();
    }

    // tau = per-row absmean(latent); wq = trit_pack(latent, tau)   (:627-674)
    [[nodiscard]] Result<void> quantize_weights_()
    {
        if (packed_only_) return Error{"BitLinear(packed-only): no latent weights to quantize"};
        ComputeEngine& engine = engine_ref();
        EX_TRY_CHECK(engine.row_absmean_into(latent_w_, tau_));
        EX_TRY_CHECK(engine.trit_pack_into(latent_w_, tau_, wq_packed_));
        quant_epoch_ = latent_w_.write_epoch();
        quant_valid_ = true;
        ++quantize_calls_;
        return {};
    }

    std::size_t in_features_, out_features_;
    bool inference_only_ = false;
    bool packed_only_ = false;
    bool act_quant_ = false;
    Tensor latent_w_, b_, wq_packed_, tau_;
    Tensor input_cache_, act_scale_;
    std::uint64_t quant_epoch_ = 0;
    bool quant_valid_ = false;
    std::uint64_t quantize_calls_ = 0;
};

class RMSNorm final : public Layer
{
public:
    explicit RMSNorm(std::size_t normalized_shape, Scalar epsilon = 1e-5f)
        : normalized_shape_(normalized_shape), epsilon_(epsilon)
    {
    }
    [[nodiscard]] const char* layer_name() const noexcept override { return "RMSNorm"; }
    [[nodiscard]] std::vector<TensorRef> parameters() override { return {gamma_}; }
    [[nodiscard]] Tensor& gamma() noexcept { return gamma_; }
    [[nodiscard]] Scalar epsilon() const noexcept { return epsilon_; }

    [[nodiscard]] Result<Tensor> forward(const Tensor& input) override
    {
        if (input.rows() != normalized_shape_) return Error{"rmsnorm forward: input shape mismatch"};
        return engine_ref().rmsnorm(input, gamma_, epsilon_);
    }

protected:
    [[nodiscard]] Result<void> init_impl(ComputeEngine& engine) override
    {
        gamma_ = engine.create_tensor(normalized_shape_, 1, Precision::F32, InitSpec::constant(1.0f));
        if (!gamma_.valid()) return Error{"RMSNorm: parameter init failed"};
        return {};
    }

private:
    std::size_t normalized_shape_;
    Scalar epsilon_;
    Tensor gamma_;
};

// LayerNorm over the features of each token (include/neuralnet.cpp/compute_layer_mlp.hpp:462-545):
// gain gamma (initialized to 1) and shift beta (0), both f32; forward is ComputeEngine::layernorm,
// ((x - mean) * rsqrt(var + eps)) * gamma + beta with the biased variance.
class LayerNorm final : public Layer
{
public:
    explicit LayerNorm(std::size_t normalized_shape, Scalar epsilon = 1e-5f)
        : normalized_shape_(normalized_shape), epsilon_(epsilon)
    {
    }
    [[nodiscard]] const char* layer_name() const noexcept override { return "LayerNorm"; }
    [[nodiscard]] std::vector<TensorRef> parameters() override { return {gamma_, beta_}; }
    [[nodiscard]] Tensor& gamma() noexcept { return gamma_; }
    [[nodiscard]] Tensor& beta() noexcept { return beta_; }
    [[nodiscard]] Scalar epsilon() const noexcept { return epsilon_; }

    [[nodiscard]] Result<Tensor> forward(const Tensor& input) override
    {
        if (input.rows() != normalized_shape_) return Error{"layernorm forward: input shape mismatch"};
        return engine_ref().layernorm(input, gamma_, beta_, epsilon_);
    }

protected:
    [[nodiscard]] Result<void> init_impl(ComputeEngine& engine) override
    {
        gamma_ = engine.create_tensor(normalized_shape_, 1, Precision::F32, InitSpec::constant(1.0f));
        beta_ = engine.create_tensor(normalized_shape_, 1, Precision::F32, InitSpec::zero());
        if (!gamma_.valid() || !beta_.valid()) return Error{"LayerNorm: parameter init failed"};
        return {};
    }

private:
    std::size_t normalized_shape_;
    Scalar epsilon_;
    Tensor gamma_, beta_;
};

// Activation of the feed-forward block (include/neuralnet.cpp/model_spec.hpp:47-54).
enum class ActivationType : std::uint32_t
{
    GeLU = 0,
    SwiGLU = 1,
    ReLU2 = 2,
};

// Normalization layer type (include/neuralnet.cpp/model_spec.hpp:56-62). FeedForward's SubLN
// takes LayerNorm (the reference's default) or RMSNorm (BitNet b1.58's); BatchNorm is refused.
enum class NormType : std::uint32_t
{
    LayerNorm = 0,
    RMSNorm = 1,
    BatchNorm = 2,
};

// Weight quantization of the linear sublayers (include/neuralnet.cpp/model_spec.hpp:112-116):
// T1_58 = BitLinear projections, the only kind this engine provides; None = float Linear.
enum class WeightQuant : std::uint32_t
{
    None = 0,
    T1_58 = 1,
};

// Gated feed-forward block with ternary BitLinear projections
// (include/neuralnet.cpp/compute_layer_feedforward.hpp:22-206, WeightQuant::T1_58), with the
// reference's constructor (:50-65): fc1 = BitLinear(d_model -> 2*d_ff) whose rows [0, d_ff) are
// the gate and [d_ff, 2*d_ff) the up projection, the gated activation (SwiGLU or ReLU^2-GLU),
// optionally SubLN of width d_ff (:37-45, :201-206; LayerNorm by default as in the reference,
// RMSNorm for BitNet b1.58), fc2 = BitLinear(d_ff -> d_model). With int8 activation
// quantization on both projections and an RMSNorm (or no) SubLN, forward() is one
// ComputeEngine::ffn_glu_i8_forward (the HIP engine fuses the block); otherwise it chains the
// layers. Only the gated activations and BitLinear projections are provided: init refuses
// GeLU, WeightQuant::None (float Linear projections) and a BatchNorm SubLN.
class FeedForward final : public Layer
{
public:
    FeedForward(std::size_t d_model, std::size_t d_ff, ActivationType activation = ActivationType::GeLU,
                bool subln = false, NormType subln_norm_type = NormType::LayerNorm,
                WeightQuant weight_quant = WeightQuant::None, bool inference_only = false)
        : d_model_(d_model), d_ff_(d_ff), activation_(activation), subln_(subln), norm_type_(subln_norm_type),
          weight_quant_(weight_quant), fc1_(d_model, 2 * d_ff, inference_only), fc2_(d_ff, d_model, inference_only)
    {
        if (subln && subln_norm_type == NormType::RMSNorm)
        {
            auto n = std::make_unique<RMSNorm>(d_ff);
            sub_rms_ = n.get();
            sub_norm_ = std::move(n);
        }
        else if (subln && subln_norm_type == NormType::LayerNorm)
        {
            auto n = std::make_unique<LayerNorm>(d_ff);
            sub_ln_ = n.get();
            sub_norm_ = std::move(n);
        }
    }

    [[nodiscard]] const char* layer_name() const noexcept override { return "FeedForward"; }

    // A ternary composite takes any profile and splits it (split_ternary_profile,
    // include/neuralnet.cpp/compute_layer_base.hpp:151-164): the projections get param T1_58.
    [[nodiscard]] PrecisionSupport precision_support() const override
    {
        PrecisionSupport sup = PrecisionSupport::rounding_all_slots();
        sup.param.mask |= PrecisionSet::of({Precision::T1_58}).mask;
        return sup;
    }

    void set_activation_quant(bool enabled) noexcept
    {
        fc1_.set_activation_quant(enabled);
        fc2_.set_activation_quant(enabled);
    }

    [[nodiscard]] BitLinear& fc1() noexcept { return fc1_; }
    [[nodiscard]] BitLinear& fc2() noexcept { return fc2_; }
    // the SubLN layer (nullptr without one), and the same as its type
    [[nodiscard]] Layer* sub_norm() noexcept { return sub_norm_.get(); }
    [[nodiscard]] RMSNorm* sub_rmsnorm() noexcept { return sub_rms_; }
    [[nodiscard]] LayerNorm* sub_layernorm() noexcept { return sub_ln_; }
    [[nodiscard]] NormType subln_norm_type() const noexcept { return norm_type_; }
    [[nodiscard]] WeightQuant weight_quant() const noexcept { return weight_quant_; }
    [[nodiscard]] std::size_t d_model() const noexcept { return d_model_; }
    [[nodiscard]] std::size_t d_ff() const noexcept { return d_ff_; }

    // fc1, fc2, then the SubLN's gamma [and beta] (compute_layer_feedforward.hpp:87-105)
    [[nodiscard]] std::vector<TensorRef> parameters() override
    {
        auto r = fc1_.parameters();
        auto r2 = fc2_.parameters();
        r.insert(r.end(), r2.begin(), r2.end());
        if (sub_norm_)
        {
            auto r3 = sub_norm_->parameters();
            r.insert(r.end(), r3.begin(), r3.end());
        }
        return r;
    }

    // entries: fc1 (weights, bias), fc2 (weights, bias), [SubLN gamma [, beta]] (same order)
    [[nodiscard]] std::size_t param_count() override
    {
        return fc1_.param_count() + fc2_.param_count() + (sub_norm_ ? sub_norm_->param_count() : 0);
    }
    [[nodiscard]] Result<ParamEntry> export_param(std::size_t index, ModelRole role) override
    {
        const std::size_t n1 = fc1_.param_count(), n2 = n1 + fc2_.param_count();
        if (index < n1) return fc1_.export_param(index, role);
        if (index < n2 || !sub_norm_) return fc2_.export_param(index - n1, role);
        return sub_norm_->export_param(index - n2, role);
    }
    [[nodiscard]] Result<void> import_param(std::size_t index, const ParamEntry& e) override
    {
        const std::size_t n1 = fc1_.param_count(), n2 = n1 + fc2_.param_count();
        if (index < n1) return fc1_.import_param(index, e);
        if (index < n2 || !sub_norm_) return fc2_.import_param(index - n1, e);
        return sub_norm_->import_param(index - n2, e);
    }

    void clear_cache() override
    {
        fc1_.clear_cache();
        fc2_.clear_cache();
    }

    [[nodiscard]] Result<Tensor> forward(const Tensor& input) override { return forward_normed_(input, nullptr); }

    // `norm` (an RMSNorm of width d_model) and then the block, as a pre-norm residual block calls
    // them (GPTBlock's norm2_ -> ff_, compute_layer_gpt.hpp:212-214). With int8 activations the
    // engine runs the norm inside the fused block; the bits are those of norm.forward + forward.
    [[nodiscard]] Result<Tensor> forward_with_norm(const Tensor& input, RMSNorm& norm)
    {
        return forward_normed_(input, &norm);
    }

private:
    [[nodiscard]] Result<Tensor> forward_normed_(const Tensor& input, RMSNorm* norm)
    {
        if (input.rows() != d_model_) return Error{"feedforward forward: input shape mismatch"};
        ComputeEngine& engine = engine_ref();
        const int act = activation_ == ActivationType::ReLU2 ? 1 : 0;
        // compute = F16: the projections and the gated activation give f16 (the reference's
        // compute precision), the SubLN f32 (stable); the chain below rounds where they do
        const Precision P = p_.compute == Precision::F16 ? Precision::F16 : Precision::F32;
        // the fused block takes an RMSNorm SubLN in f32; a LayerNorm SubLN runs the chain below
        if (fc1_.activation_quant() && fc2_.activation_quant() && sub_ln_ == nullptr && P == Precision::F32)
        {
            EX_TRY_CHECK(fc1_.ensure_quantized());
            EX_TRY_CHECK(fc2_.ensure_quantized());
            return engine.ffn_glu_i8_forward(input, norm ? &norm->gamma() : nullptr, norm ? norm->epsilon() : 0.0f,
                                             fc1_.quantized_weights_packed(), fc1_.row_scales(),
                                             fc1_.bias(), fc2_.quantized_weights_packed(), fc2_.row_scales(),
                                             fc2_.bias(), act, sub_rms_ ? &sub_rms_->gamma() : nullptr,
                                             sub_rms_ ? sub_rms_->epsilon() : 0.0f);
        }
        Tensor in = input;
        if (norm)
        {
            EX_TRY(iw, engine.cast(input, Precision::F32));
            EX_TRY(n, norm->forward(*iw));
            in = *n;
        }
        EX_TRY(h1, fc1_.forward(in));
        EX_TRY(h1w, engine.cast(*h1, Precision::F32));
        EX_TRY(g32, engine.glu(*h1w, act));
        EX_TRY(h2, engine.cast(*g32, P));
        if (sub_norm_)
        {
            EX_TRY(h2w, engine.cast(*h2, Precision::F32));
            EX_TRY(h3, sub_norm_->forward(*h2w));
            return fc2_.forward(*h3);
        }
        return fc2_.forward(*h2);
    }

public:
protected:
    [[nodiscard]] Result<void> init_impl(ComputeEngine& engine) override
    {
        if (activation_ == ActivationType::GeLU)
            return Error{"FeedForward: only the gated activations (SwiGLU, ReLU2) are provided by this engine"};
        if (weight_quant_ != WeightQuant::T1_58)
            return Error{"FeedForward: only BitLinear projections (WeightQuant::T1_58) are provided by this engine"};
        if (subln_ && !sub_norm_)
            return Error{"FeedForward: the SubLN norm type must be LayerNorm or RMSNorm (BatchNorm is not provided)"};
        PrecisionProfile linear = p_;
        linear.param = Precision::T1_58;
        fc1_.set_precision_profile(linear);
        fc2_.set_precision_profile(linear);
        EX_TRY_CHECK(fc1_.init(engine));
        EX_TRY_CHECK(fc2_.init(engine));
        if (sub_norm_)
        {
            PrecisionProfile norm = p_;
            norm.param = Precision::F32;
            sub_norm_->set_precision_profile(norm);
            EX_TRY_CHECK(sub_norm_->init(engine));
        }
        return {};
    }

private:
    std::size_t d_model_, d_ff_;
    ActivationType activation_;
    bool subln_;
    NormType norm_type_;
    WeightQuant weight_quant_;
    BitLinear fc1_, fc2_;
    std::unique_ptr<Layer> sub_norm_;  // SubLN, or none
    RMSNorm* sub_rms_ = nullptr;       // sub_norm_ as its type
    LayerNorm* sub_ln_ = nullptr;
};

}  // namespace nn
