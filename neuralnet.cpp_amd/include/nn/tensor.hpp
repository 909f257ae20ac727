// tensor.hpp — cross-device tensor handle.
//
// Same public surface as the reference Tensor (include/neuralnet.cpp/tensor.hpp:44-218):
// a cheap-to-copy handle {device, rows, cols, shared storage}. Copies share the
// buffer, so in-place engine ops are visible through every copy. The
// reference keeps one storage slot per compiled backend behind #ifdefs
// (tensor.hpp:54-62); here there is exactly one device slot, an opaque
// DeviceBuffer owned by whichever engine allocated it (the HIP engine's pool).
#pragma once

#include <cstddef>
#include <cstdio>
#include <cstdlib>
#include <functional>
#include <memory>
#include <string>

#include "core_errors.hpp"
#include "matrix.hpp"

namespace nn
{

enum class Device : std::uint8_t
{
    CPU,
    GPU,
};

// Device memory owned by an engine. Destroying the last reference hands the
// memory back to the owner (the HIP engine's stream-ordered caching pool).
class DeviceBuffer
{
public:
    virtual ~DeviceBuffer() = default;
    [[nodiscard]] virtual float* data() noexcept = 0;
    [[nodiscard]] virtual std::size_t capacity() const noexcept = 0;   // in floats
};

[[noreturn]] inline void tensor_fatal_(const char* what)
{
    std::fprintf(stderr, "nn::Tensor fatal: %s\n", what);
    std::abort();
}

class Tensor
{
public:
    Tensor() = default;

    explicit Tensor(std::shared_ptr<Matrix> m)
        : device_(Device::CPU), rows_(m->rows()), cols_(m->cols()), cpu_(std::move(m)) {}

    Tensor(std::shared_ptr<DeviceBuffer> buf, std::size_t rows, std::size_t cols)
        : device_(Device::GPU), rows_(rows), cols_(cols), dev_(std::move(buf))
    {
        if (dev_ && dev_->capacity() < rows * cols)
            tensor_fatal_("device buffer smaller than tensor shape");
    }

    static Tensor from_matrix(Matrix m) { return Tensor(std::make_shared<Matrix>(std::move(m))); }
    static Tensor cpu(std::size_t rows, std::size_t cols) { return Tensor(std::make_shared<Matrix>(rows, cols)); }

    [[nodiscard]] Device device() const noexcept { return device_; }
    [[nodiscard]] std::size_t rows() const noexcept { return rows_; }
    [[nodiscard]] std::size_t cols() const noexcept { return cols_; }
    [[nodiscard]] std::size_t size() const noexcept { return rows_ * cols_; }
    [[nodiscard]] bool is_cpu() const noexcept { return device_ == Device::CPU; }
    [[nodiscard]] bool is_gpu() const noexcept { return device_ == Device::GPU; }
    [[nodiscard]] bool valid() const noexcept
    {
        return device_ == Device::CPU ? static_cast<bool>(cpu_) : static_cast<bool>(dev_);
    }

    [[nodiscard]] Matrix& cpu_matrix()
    {
        if (device_ != Device::CPU || !cpu_)
            tensor_fatal_("cpu_matrix() on non-CPU tensor");
        return *cpu_;
    }
    [[nodiscard]] const Matrix& cpu_matrix() const
    {
        if (device_ != Device::CPU || !cpu_)
            tensor_fatal_("cpu_matrix() on non-CPU tensor");
        return *cpu_;
    }
    [[nodiscard]] std::shared_ptr<Matrix> cpu_shared() const noexcept { return cpu_; }

    [[nodiscard]] const std::shared_ptr<DeviceBuffer>& device_buffer() const noexcept { return dev_; }
    // Raw device pointer (nullptr for CPU / invalid tensors).
    [[nodiscard]] float* dev_ptr() const noexcept { return dev_ ? dev_->data() : nullptr; }

    [[nodiscard]] std::string shape_str() const
    {
        return "(" + std::to_string(rows_) + "x" + std::to_string(cols_) + ")" +
               (device_ == Device::CPU ? "[CPU]" : "[GPU]");
    }

    // Reshape: device tensors alias the same buffer; CPU tensors copy into a
    // Matrix of the new shape (reference tensor.hpp:185-217 does the same,
    // because the CPU Matrix carries its own shape).
    [[nodiscard]] Tensor reshape(std::size_t new_rows, std::size_t new_cols) const
    {
        if (new_rows * new_cols != rows_ * cols_)
            tensor_fatal_("reshape: element count mismatch");
        Tensor t;
        t.device_ = device_;
        t.rows_ = new_rows;
        t.cols_ = new_cols;
        if (device_ == Device::CPU)
        {
            auto m = std::make_shared<Matrix>(new_rows, new_cols);
            const auto src = cpu_->span();
            std::copy(src.begin(), src.end(), m->span().begin());
            t.cpu_ = std::move(m);
        }
        else
        {
            t.dev_ = dev_;
        }
        return t;
    }

private:
    Device device_ = Device::CPU;
    std::size_t rows_ = 0;
    std::size_t cols_ = 0;
    std::shared_ptr<Matrix> cpu_;
    std::shared_ptr<DeviceBuffer> dev_;
};

// Non-owning reference used by Layer::parameters() and the optimizers
// (reference tensor.hpp:222).
using TensorRef = std::reference_wrapper<Tensor>;

} // namespace nn
