#pragma once
// model_container.hpp — nn::Model: an ordered stack of layers on one engine.
// Mirrors include/neuralnet.cpp/model_container.hpp:91-125 (add<T>(args...) constructs the
// layer, applies the model's default precision profile and initializes it on the engine,
// returning a Result) and :229-247 (forward runs the layers in order inside one batch).

#include <memory>
#include <utility>
#include <vector>

#include "compute_engine.hpp"
#include "layers.hpp"

namespace nn
{

class Model
{
public:
    explicit Model(ComputeEngine& engine) : engine_(&engine) {}

    void set_default_precision_profile(const PrecisionProfile& p) noexcept { profile_ = p; }

    template <class T, class... Args>
    [[nodiscard]] Result<void> add(Args&&... args)
    {
        auto layer = std::make_unique<T>(std::forward<Args>(args)...);
        layer->set_precision_profile(profile_);
        EX_TRY_CHECK(layer->init(*engine_));
        layers_.push_back(std::move(layer));
        return {};
    }

    // An already built layer, with the model's default profile or an explicit one
    // (include/neuralnet.cpp/model_container.hpp:103-124: e.g. BitLinear at param=T1_58 next
    // to norm layers at the f32 default).
    [[nodiscard]] Result<void> add_layer(std::unique_ptr<Layer> layer)
    {
        return add_layer(std::move(layer), profile_);
    }
    [[nodiscard]] Result<void> add_layer(std::unique_ptr<Layer> layer, const PrecisionProfile& profile)
    {
        layer->set_precision_profile(profile);
        EX_TRY_CHECK(layer->init(*engine_));
        layers_.push_back(std::move(layer));
        return {};
    }

    [[nodiscard]] Result<Tensor> forward(const Tensor& input)
    {
        if (layers_.empty()) return Error{"Model::forward: no layers"};
        engine_->begin_batch();
        Tensor x = input;
        for (auto& l : layers_)
        {
            auto y = l->forward(x);
            if (!y)
            {
                engine_->end_batch();
                return Error{std::string(l->layer_name()) + ": " + y.error().message};
            }
            x = *y;
        }
        engine_->end_batch();
        return x;
    }

    [[nodiscard]] std::size_t num_layers() const noexcept { return layers_.size(); }
    [[nodiscard]] Layer& layer_at(std::size_t i) { return *layers_[i]; }
    [[nodiscard]] ComputeEngine& engine() noexcept { return *engine_; }

private:
    ComputeEngine* engine_;
    PrecisionProfile profile_{};
    std::vector<std::unique_ptr<Layer>> layers_;
};

}  // namespace nn
