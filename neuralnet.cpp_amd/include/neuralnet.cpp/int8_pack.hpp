#pragma once
// int8_pack.hpp — host-side codec of the int8 activation container (nn::i8_pack).
//
// Same names and semantics as the reference's engine header (docs/internal/21-quantized-
// weights.md:966-990; behaviour pinned by src/int8_act_test.cpp:86-168): 4 int8 per u32
// word, element c of a row in byte c%4 of word c/4 (little-endian), tail bytes 0.
// quantize(x, s) = round_half_away(clamp(x/s, -127, 127)); NaN -> 0; s == 0 -> 0.

#include <cmath>
#include <cstddef>
#include <cstdint>

namespace nn::i8_pack
{

[[nodiscard]] constexpr std::size_t words_per_row(std::size_t cols) noexcept { return (cols + 3) / 4; }

[[nodiscard]] inline std::int8_t quantize(float x, float s) noexcept
{
    if (s == 0.0f || std::isnan(x)) return 0;
    float v = x / s;
    if (std::isnan(v)) return 0;
    if (v > 127.0f) v = 127.0f;
    if (v < -127.0f) v = -127.0f;
    return static_cast<std::int8_t>(std::round(v));
}

[[nodiscard]] inline std::int8_t at(const std::uint32_t* words, std::size_t i) noexcept
{
    return static_cast<std::int8_t>(static_cast<std::uint8_t>((words[i / 4] >> (8 * (i % 4))) & 0xFFu));
}

inline void pack_row(const float* x, std::size_t cols, const float* scale, std::uint32_t* words) noexcept
{
    for (std::size_t wi = 0; wi < words_per_row(cols); ++wi)
    {
        std::uint32_t w = 0;
        for (std::size_t b = 0; b < 4 && wi * 4 + b < cols; ++b)
            w |= static_cast<std::uint32_t>(static_cast<std::uint8_t>(quantize(x[wi * 4 + b], scale[wi * 4 + b])))
                 << (8 * b);
        words[wi] = w;
    }
}

}  // namespace nn::i8_pack
