// compute_loss.hpp — sparse (label-index) cross-entropy over column logits.
//
// Follows CrossEntropyLoss::forward_sparse / fused_forward_sparse_
// (reference include/neuralnet.cpp/compute_loss.hpp:229-309):
//   1. upload labels as a (1,N) float tensor and the optional 0/1 mask;
//   2. count num_valid on the host (mask >= 0.5 and label < vocab);
//   3. col_softmax_sparse_forward -> dense grad (V,N) and loss_vec (1,N);
//   4. loss = -sum(loss_vec) / num_valid via row_reduce_sum + to_matrix.
// No fallback path: an engine error is returned as is.
#pragma once

#include <optional>
#include <span>

#include "compute_engine.hpp"
#include "compute_layer.hpp"

namespace nn
{

class CrossEntropyLoss
{
public:
    Result<Scalar> forward_sparse(ComputeEngine& engine, const Tensor& logits, std::span<const std::size_t> labels,
                                  std::span<const Scalar> loss_mask = {}, std::size_t vocab_size = 0)
    {
        const std::size_t classes = logits.rows(), total = logits.cols();
        if (vocab_size == 0)
            vocab_size = classes;
        if (labels.size() != total)
            return fail("sparse CE: labels size mismatch");
        if (!loss_mask.empty() && loss_mask.size() != total)
            return fail("sparse CE: mask size mismatch");
        if (classes == 0 || total == 0)
            return fail("sparse CE: empty input");

        Matrix lab(1, total);
        for (std::size_t i = 0; i < total; ++i)
            lab.span()[i] = static_cast<Scalar>(labels[i]);
        NN_TRY(labels_t, engine.from_matrix(lab));

        std::optional<Tensor> mask_t;
        const Tensor* mask_ptr = nullptr;
        if (!loss_mask.empty())
        {
            Matrix mm(1, total);
            for (std::size_t i = 0; i < total; ++i)
                mm.span()[i] = loss_mask[i] >= Scalar{0.5f} ? Scalar{1} : Scalar{0};
            NN_TRY(mt, engine.from_matrix(mm));
            mask_t = mt;
            mask_ptr = &*mask_t;
        }

        return forward_sparse_resident(engine, logits, labels_t, mask_ptr, vocab_size,
                                       count_valid(labels, loss_mask, vocab_size));
    }

    // Host count of contributing columns (reference compute_loss.hpp:284-289).
    static std::size_t count_valid(std::span<const std::size_t> labels, std::span<const Scalar> loss_mask,
                                   std::size_t vocab_size)
    {
        std::size_t num_valid = 0;
        for (std::size_t i = 0; i < labels.size(); ++i)
        {
            const bool masked = !loss_mask.empty() && loss_mask[i] < Scalar{0.5f};
            if (!masked && labels[i] < vocab_size)
                ++num_valid;
        }
        return num_valid;
    }

    // Steps 3-5 with labels / mask already resident on the engine's device
    // (a training loop that keeps its batch in device memory uploads them
    // once; forward_sparse above uploads them every call like the reference).
    Result<Scalar> forward_sparse_resident(ComputeEngine& engine, const Tensor& logits, const Tensor& labels_t,
                                           const Tensor* mask_ptr, std::size_t vocab_size, std::size_t num_valid)
    {
        NN_TRY(tot, forward_sparse_total(engine, logits, labels_t, mask_ptr, vocab_size, num_valid));
        NN_TRY(host, engine.to_matrix(tot));
        return loss_of_total(host, num_valid);
    }

    // Steps 3-4 without the host read: the (1,1) device sum of loss_vec, for a
    // loop that reads the loss once its step's later work is queued (the value
    // is the same; only the wait moves). loss_of_total finishes step 5.
    Result<Tensor> forward_sparse_total(ComputeEngine& engine, const Tensor& logits, const Tensor& labels_t,
                                        const Tensor* mask_ptr, std::size_t vocab_size, std::size_t num_valid)
    {
        const Scalar inv = num_valid > 0 ? Scalar{1} / static_cast<Scalar>(num_valid) : Scalar{0};
        Tensor loss_vec;
        NN_TRY(grad, engine.col_softmax_sparse_forward(logits, labels_t, mask_ptr, vocab_size, inv, loss_vec));
        grad_ = grad;
        return engine.row_reduce_sum(loss_vec);
    }

    static Scalar loss_of_total(const Matrix& total, std::size_t num_valid)
    {
        return num_valid > 0 ? -total.at_unchecked(0, 0) / static_cast<Scalar>(num_valid) : Scalar{0};
    }

    Result<Tensor> backward() { return grad_; }

private:
    Tensor grad_;
};

} // namespace nn
