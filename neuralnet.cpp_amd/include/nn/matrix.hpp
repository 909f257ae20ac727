// matrix.hpp — host-side row-major fp32 container.
//
// The reference's Matrix (include/neuralnet.cpp/algebra_matrix.hpp:42-120) is
// both the host data carrier of from_matrix/to_matrix/copy_from and the CPU
// engine's arithmetic. The HIP engine only needs the carrier: shape, flat
// span access and element get/set. The CPU arithmetic lives with the CPU
// engine restatement, not in the product.
#pragma once

#include <algorithm>
#include <cstddef>
#include <span>
#include <vector>

namespace nn
{

using Scalar = float;   // reference include/neuralnet.cpp/config.hpp:18

class Matrix
{
public:
    Matrix() = default;
    Matrix(std::size_t rows, std::size_t cols) : data_(rows * cols), rows_(rows), cols_(cols) {}
    Matrix(std::size_t rows, std::size_t cols, Scalar value)
        : data_(rows * cols, value), rows_(rows), cols_(cols) {}

    void resize(std::size_t rows, std::size_t cols)
    {
        rows_ = rows;
        cols_ = cols;
        data_.resize(rows * cols);
    }

    [[nodiscard]] std::span<const Scalar> span() const noexcept { return {data_.data(), data_.size()}; }
    [[nodiscard]] std::span<Scalar> span() noexcept { return {data_.data(), data_.size()}; }
    [[nodiscard]] const Scalar* data() const noexcept { return data_.data(); }
    [[nodiscard]] Scalar* data() noexcept { return data_.data(); }

    [[nodiscard]] std::size_t rows() const noexcept { return rows_; }
    [[nodiscard]] std::size_t cols() const noexcept { return cols_; }
    [[nodiscard]] std::size_t size() const noexcept { return data_.size(); }
    [[nodiscard]] bool empty() const noexcept { return data_.empty(); }

    [[nodiscard]] Scalar at(std::size_t r, std::size_t c) const { return data_.at(r * cols_ + c); }
    void set_value(std::size_t r, std::size_t c, Scalar v) { data_.at(r * cols_ + c) = v; }
    [[nodiscard]] Scalar at_unchecked(std::size_t r, std::size_t c) const noexcept { return data_[r * cols_ + c]; }
    void set_value_unchecked(std::size_t r, std::size_t c, Scalar v) noexcept { data_[r * cols_ + c] = v; }

    void zero() noexcept { std::fill(data_.begin(), data_.end(), Scalar{0}); }

private:
    std::vector<Scalar> data_{};
    std::size_t rows_ = 0;
    std::size_t cols_ = 0;
};

} // namespace nn
