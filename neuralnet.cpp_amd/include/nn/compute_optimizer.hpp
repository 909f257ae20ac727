// compute_optimizer.hpp — optimizers expressed as engine primitives.
//
// AdamW follows the reference step exactly (include/neuralnet.cpp/compute_optimizer.hpp:
// clip_grad_norm :90-140, zero_grad :142-151, adam_update_ :252-304,
// bias_correction_ :314-319, AdamW::step :388-412), i.e. per parameter tensor:
//   scale_inplace(p, 1 - lr*wd)
//   scale_inplace(m, b1); axpy_inplace(m, 1-b1, g)
//   scale_inplace(v, b2); g2 = g*g; scale_inplace(g2, 1-b2); add_inplace(v, g2)
//   mh = clone(m)*inv_bc1; vh = clone(v)*inv_bc2
//   ratio = mh / (sqrt(vh) + eps); scale_inplace(ratio, -lr); add_inplace(p, ratio)
// with inv_bc = 1 / (1 - beta^t) computed once per step.
#pragma once

#include <cmath>
#include <utility>
#include <vector>

#include "compute_engine.hpp"
#include "compute_layer.hpp"

namespace nn
{

class Optimizer
{
public:
    Optimizer(ComputeEngine& engine, std::vector<TensorRef> params, std::vector<TensorRef> grads)
        : engine_(engine), params_(std::move(params)), grads_(std::move(grads))
    {
    }
    virtual ~Optimizer() = default;
    virtual void set_lr(Scalar lr) = 0;
    [[nodiscard]] virtual Result<void> step() = 0;

    // Global L2-norm clipping: sum of squares per tensor reduced on the
    // device, one download, then scale every grad if the norm exceeds max_norm.
    [[nodiscard]] Result<void> clip_grad_norm(Scalar max_norm)
    {
        if (max_norm <= 0 || grads_.empty())
            return {};
        Tensor acc;
        for (auto& gr : grads_)
        {
            Tensor& g = gr.get();
            NN_TRY(sq, engine_.elementwise_binary(BinaryOp::Mul, g, g));
            NN_TRY(rs, engine_.row_reduce_sum(sq));
            NN_TRY(cs, engine_.col_reduce_sum(rs));
            if (acc.valid())
            {
                NN_TRY(sum, engine_.elementwise_binary(BinaryOp::Add, acc, cs));
                acc = sum;
            }
            else
                acc = cs;
        }
        NN_TRY(host, engine_.to_matrix(acc));
        const Scalar norm = std::sqrt(host.at(0, 0));
        if (norm <= max_norm)
            return {};
        const Scalar s = max_norm / norm;
        for (auto& gr : grads_)
            NN_CHECK(engine_.scale_inplace(gr.get(), s));
        return {};
    }

    [[nodiscard]] virtual Result<void> zero_grad()
    {
        for (auto& g : grads_)
            NN_CHECK(engine_.zero(g.get()));
        return {};
    }

protected:
    [[nodiscard]] Result<void> validate_sizes_() const
    {
        if (params_.size() != grads_.size())
            return fail("Optimizer: params/grads size mismatch");
        return {};
    }
    std::vector<Tensor> zero_buffers_() const
    {
        std::vector<Tensor> out;
        out.reserve(params_.size());
        for (auto& p : params_)
        {
            Tensor t = engine_.create_tensor(p.get().rows(), p.get().cols());
            layer_take_(engine_.zero(t));
            out.push_back(std::move(t));
        }
        return out;
    }

    ComputeEngine& engine_;
    std::vector<TensorRef> params_;
    std::vector<TensorRef> grads_;
};

class Adam : public Optimizer
{
public:
    Adam(ComputeEngine& engine, std::vector<TensorRef> params, std::vector<TensorRef> grads, Scalar lr,
         Scalar beta1 = Scalar{0.9f}, Scalar beta2 = Scalar{0.999f}, Scalar eps = Scalar{1e-8f})
        : Optimizer(engine, std::move(params), std::move(grads)), lr_(lr), beta1_(beta1), beta2_(beta2), eps_(eps)
    {
        m_ = zero_buffers_();
        v_ = zero_buffers_();
    }
    void set_lr(Scalar lr) override { lr_ = lr; }

    Result<void> step() override
    {
        NN_CHECK(validate_sizes_());
        const std::size_t t_next = t_ + 1;
        const auto [ib1, ib2] = bias_correction_(t_next);
        for (std::size_t i = 0; i < params_.size(); ++i)
            NN_CHECK(adam_update_(i, ib1, ib2));
        t_ = t_next;
        return {};
    }

protected:
    [[nodiscard]] std::pair<Scalar, Scalar> bias_correction_(std::size_t t) const
    {
        const Scalar bc1 = Scalar{1} - std::pow(beta1_, static_cast<Scalar>(t));
        const Scalar bc2 = Scalar{1} - std::pow(beta2_, static_cast<Scalar>(t));
        return {Scalar{1} / bc1, Scalar{1} / bc2};
    }

    [[nodiscard]] Result<void> adam_update_(std::size_t i, Scalar inv_bc1, Scalar inv_bc2)
    {
        const Tensor& g = grads_[i].get();
        NN_CHECK(engine_.scale_inplace(m_[i], beta1_));
        NN_CHECK(engine_.axpy_inplace(m_[i], Scalar{1} - beta1_, g));
        NN_CHECK(engine_.scale_inplace(v_[i], beta2_));
        NN_TRY(g2, engine_.elementwise_binary(BinaryOp::Mul, g, g));
        NN_CHECK(engine_.scale_inplace(g2, Scalar{1} - beta2_));
        NN_CHECK(engine_.add_inplace(v_[i], g2));
        NN_TRY(mh, engine_.clone(m_[i]));
        NN_CHECK(engine_.scale_inplace(mh, inv_bc1));
        NN_TRY(vh, engine_.clone(v_[i]));
        NN_CHECK(engine_.scale_inplace(vh, inv_bc2));
        NN_TRY(sq, engine_.elementwise_unary(UnaryOp::Sqrt, vh));
        NN_TRY(den, engine_.elementwise_binary_scalar(BinaryOp::Add, sq, eps_));
        NN_TRY(ratio, engine_.elementwise_binary(BinaryOp::Div, mh, den));
        NN_CHECK(engine_.scale_inplace(ratio, -lr_));
        return engine_.add_inplace(params_[i].get(), ratio);
    }

    Scalar lr_, beta1_, beta2_, eps_;
    std::size_t t_ = 0;
    std::vector<Tensor> m_, v_;
};

class AdamW final : public Adam
{
public:
    AdamW(ComputeEngine& engine, std::vector<TensorRef> params, std::vector<TensorRef> grads, Scalar lr,
          Scalar beta1 = Scalar{0.9f}, Scalar beta2 = Scalar{0.999f}, Scalar eps = Scalar{1e-8f},
          Scalar weight_decay = Scalar{0.01f})
        : Adam(engine, std::move(params), std::move(grads), lr, beta1, beta2, eps), wd_(weight_decay)
    {
    }

    Result<void> step() override
    {
        NN_CHECK(validate_sizes_());
        const std::size_t t_next = t_ + 1;
        const auto [ib1, ib2] = bias_correction_(t_next);
        const Scalar decay = Scalar{1} - lr_ * wd_;
        for (std::size_t i = 0; i < params_.size(); ++i)
        {
            if (wd_ != Scalar{0})
                NN_CHECK(engine_.scale_inplace(params_[i].get(), decay));
            NN_CHECK(adam_update_(i, ib1, ib2));
        }
        t_ = t_next;
        return {};
    }

private:
    Scalar wd_;
};

} // namespace nn
