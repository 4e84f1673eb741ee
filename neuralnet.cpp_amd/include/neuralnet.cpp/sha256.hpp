#pragma once
// sha256.hpp — SHA-256 (FIPS 180-4) for the whole-file checksum of v8 model files
// (include/neuralnet.cpp/model_serialization.hpp:73-82: [sha256 32B]["NNEND"] tail).
// Incremental interface: Sha256 h; h.update(bytes); h.digest().

#include <array>
#include <cstddef>
#include <cstdint>

namespace nn
{

class Sha256
{
public:
    Sha256() noexcept;
    void update(const void* data, std::size_t n) noexcept;
    [[nodiscard]] std::array<std::uint8_t, 32> digest() noexcept;  // finalizes; call once

private:
    void block(const std::uint8_t* p) noexcept;
    std::uint32_t h_[8];
    std::uint8_t buf_[64];
    std::size_t buf_len_ = 0;
    std::uint64_t total_ = 0;
};

}  // namespace nn
