#pragma once
// matrix.hpp — nn::Matrix: the host-side f32 carrier of engine I/O.
//
// Row-major data_[r * cols + c], as the reference's algebra_matrix.hpp
// (docs/introduction/01-architecture.md:254-260, :312-322). Packed containers (ternary
// words, int8 words) travel through it as raw 32-bit patterns: copies are bitwise, nothing
// here does float arithmetic on the stored values.

#include <cstddef>
#include <span>
#include <vector>

namespace nn
{

using Scalar = float;

class Matrix
{
public:
    Matrix() = default;
    Matrix(std::size_t rows, std::size_t cols) : rows_(rows), cols_(cols), data_(rows * cols, 0.0f) {}

    [[nodiscard]] std::size_t rows() const noexcept { return rows_; }
    [[nodiscard]] std::size_t cols() const noexcept { return cols_; }
    [[nodiscard]] std::size_t size() const noexcept { return data_.size(); }
    [[nodiscard]] std::span<float> span() noexcept { return data_; }
    [[nodiscard]] std::span<const float> span() const noexcept { return data_; }
    [[nodiscard]] float* data() noexcept { return data_.data(); }
    [[nodiscard]] const float* data() const noexcept { return data_.data(); }
    [[nodiscard]] float at(std::size_t r, std::size_t c) const noexcept { return data_[r * cols_ + c]; }
    void set_value(std::size_t r, std::size_t c, float v) noexcept { data_[r * cols_ + c] = v; }

private:
    std::size_t rows_ = 0, cols_ = 0;
    std::vector<float> data_;
};

}  // namespace nn
