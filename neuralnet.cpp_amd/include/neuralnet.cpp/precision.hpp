#pragma once
// precision.hpp — nn::Precision and the per-layer precision profile, the subset the
// BitLinear path uses (reference: include/neuralnet.cpp/precision.hpp and
// compute_layer_base.hpp:144-181). T1_58 marks "effective weights are ternary"; it only
// ever occupies the param slot.

#include <cstdint>
#include <initializer_list>
#include <string>

namespace nn
{

enum class Precision : std::uint8_t
{
    F16 = 0,
    F32 = 1,
    T1_58 = 2,
};

[[nodiscard]] inline const char* precision_name(Precision p) noexcept
{
    switch (p)
    {
    case Precision::F16: return "f16";
    case Precision::F32: return "f32";
    case Precision::T1_58: return "t1_58";
    }
    return "?";
}

struct PrecisionSet
{
    std::uint32_t mask = 0;
    [[nodiscard]] static PrecisionSet of(std::initializer_list<Precision> ps) noexcept
    {
        PrecisionSet s;
        for (Precision p : ps) s.mask |= 1u << static_cast<unsigned>(p);
        return s;
    }
    [[nodiscard]] bool has(Precision p) const noexcept { return (mask >> static_cast<unsigned>(p)) & 1u; }
    [[nodiscard]] std::string to_string() const
    {
        std::string r;
        for (unsigned i = 0; i < 3; ++i)
            if ((mask >> i) & 1u) r += (r.empty() ? "" : "|") + std::string(precision_name(static_cast<Precision>(i)));
        return r;
    }
};

[[nodiscard]] inline PrecisionSet rounding_precision_set() noexcept
{
    return PrecisionSet::of({Precision::F16, Precision::F32});
}

struct PrecisionSupport
{
    PrecisionSet param, compute, stable, optimizer;
    [[nodiscard]] static PrecisionSupport rounding_all_slots() noexcept
    {
        const PrecisionSet r = rounding_precision_set();
        return {r, r, r, r};
    }
};

struct PrecisionProfile
{
    Precision param = Precision::F32;
    Precision compute = Precision::F32;
    Precision stable = Precision::F32;
    Precision optimizer = Precision::F32;
};

// CLI --t1_58 preset: ternary weights, f16 elsewhere (src/t1_58_test.cpp:668-690).
[[nodiscard]] inline PrecisionProfile profile_t1_58() noexcept
{
    return {Precision::T1_58, Precision::F16, Precision::F32, Precision::F32};
}

}  // namespace nn
