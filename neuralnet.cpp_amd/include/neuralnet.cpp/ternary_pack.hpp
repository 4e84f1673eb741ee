#pragma once
// ternary_pack.hpp — host-side codec of the packed ternary container (nn::trit_pack).
//
// Same names and semantics as the reference's engine header (exported by
// modules/nn.engine.cpp:17-35; behaviour pinned by src/ternary_gemm_test.cpp:74-137):
// 2 bits per weight, 16 weights per u32 word, weight j of a row at
// (word[j/16] >> 2*(j%16)) & 3, code = trit + 2 in {1,2,3}, tail codes 2 (trit 0).
// code_of(w, tau) = 3 if w > 0.5*tau, 1 if w < -0.5*tau, else 2 (the strict threshold of
// include/neuralnet.cpp/compute_layer_bitlinear.hpp:657-667).

#include <cstddef>
#include <cstdint>

namespace nn::trit_pack
{

inline constexpr std::uint32_t kBits = 2;
inline constexpr std::uint32_t kPerByte = 4;
inline constexpr std::uint32_t kPerWord = 16;
inline constexpr std::uint32_t kMask = 3;

[[nodiscard]] constexpr std::size_t words_per_row(std::size_t k) noexcept { return (k + kPerWord - 1) / kPerWord; }
[[nodiscard]] constexpr std::size_t bytes_per_row(std::size_t k) noexcept { return words_per_row(k) * 4; }

[[nodiscard]] constexpr std::uint32_t code_of(float w, float tau) noexcept
{
    const float h = 0.5f * tau;
    return w > h ? 3u : (w < -h ? 1u : 2u);
}

[[nodiscard]] constexpr float value_of(std::uint32_t code) noexcept { return static_cast<float>(static_cast<int>(code) - 2); }

inline void pack_row(const float* w, std::size_t k, float tau, std::uint32_t* words) noexcept
{
    const std::size_t wpr = words_per_row(k);
    for (std::size_t wi = 0; wi < wpr; ++wi)
    {
        std::uint32_t word = 0;
        for (std::uint32_t j = 0; j < kPerWord; ++j)
        {
            const std::size_t idx = wi * kPerWord + j;
            const std::uint32_t code = idx < k ? code_of(w[idx], tau) : 2u;
            word |= code << (kBits * j);
        }
        words[wi] = word;
    }
}

[[nodiscard]] inline float at(const std::uint32_t* words, std::size_t i) noexcept
{
    return value_of((words[i / kPerWord] >> (kBits * (i % kPerWord))) & kMask);
}

}  // namespace nn::trit_pack
