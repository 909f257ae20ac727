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
// with inv_bc = 1 / (1 - beta^t) computed once per step. SGD, SGD with
// momentum and Muon (with its Newton-Schulz orthogonalisation) follow the
// reference's primitive sequences as well; create_optimizer picks one by name.
#pragma once

#include <cmath>
#include <memory>
#include <string_view>
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

// ── SGD / SGD with momentum (reference compute_optimizer.hpp:153-216) ─────
//   SGD: axpy_inplace(p, -lr, g)
//   momentum: scale_inplace(v, beta); axpy_inplace(v, 1-beta, g); axpy_inplace(p, -lr, v)
class SGD final : public Optimizer
{
public:
    SGD(ComputeEngine& engine, std::vector<TensorRef> params, std::vector<TensorRef> grads, Scalar lr)
        : Optimizer(engine, std::move(params), std::move(grads)), lr_(lr)
    {
    }
    void set_lr(Scalar lr) override { lr_ = lr; }
    Result<void> step() override
    {
        NN_CHECK(validate_sizes_());
        for (std::size_t i = 0; i < params_.size(); ++i)
            NN_CHECK(engine_.axpy_inplace(params_[i].get(), -lr_, grads_[i].get()));
        return {};
    }

private:
    Scalar lr_;
};

class SGDWithMomentum final : public Optimizer
{
public:
    SGDWithMomentum(ComputeEngine& engine, std::vector<TensorRef> params, std::vector<TensorRef> grads, Scalar lr,
                    Scalar beta = Scalar{0.9f})
        : Optimizer(engine, std::move(params), std::move(grads)), lr_(lr), beta_(beta)
    {
        v_ = zero_buffers_();
    }
    void set_lr(Scalar lr) override { lr_ = lr; }
    Result<void> step() override
    {
        NN_CHECK(validate_sizes_());
        for (std::size_t i = 0; i < params_.size(); ++i)
        {
            NN_CHECK(engine_.scale_inplace(v_[i], beta_));
            NN_CHECK(engine_.axpy_inplace(v_[i], Scalar{1} - beta_, grads_[i].get()));
            NN_CHECK(engine_.axpy_inplace(params_[i].get(), -lr_, v_[i]));
        }
        return {};
    }

private:
    Scalar lr_, beta_;
    std::vector<Tensor> v_;
};

// ── Newton-Schulz orthogonalisation (reference compute_optimizer.hpp:430-497) ─
// X = G / sqrt(||G||_F^2 + eps^2) (the squared norm reduced on the device,
// then downloaded), then `steps` times: A = X X^T, A2 = A A, A = b A + c A2,
// X = A X + a X, with the quintic coefficients (a, b, c) = (3.4445, -4.7750,
// 2.0315). The iteration keeps G's singular vectors and maps each normalised
// singular value s to phi(s) = a s + b s^3 + c s^5.
[[nodiscard]] inline Result<Tensor> newton_schulz_orthogonalize(ComputeEngine& engine, const Tensor& G,
                                                                std::size_t steps = 5, Scalar eps = Scalar{1e-7f})
{
    constexpr Scalar a = 3.4445f, b = -4.7750f, c = 2.0315f;
    NN_TRY(sq, engine.elementwise_binary(BinaryOp::Mul, G, G));
    NN_TRY(rs, engine.row_reduce_sum(sq));
    NN_TRY(total, engine.col_reduce_sum(rs));
    NN_TRY(host, engine.to_matrix(total));
    const Scalar inv_norm = Scalar{1} / std::sqrt(host.at(0, 0) + eps * eps);
    NN_TRY(X0, engine.clone(G));
    Tensor X = X0;
    NN_CHECK(engine.scale_inplace(X, inv_norm));
    for (std::size_t t = 0; t < steps; ++t)
    {
        NN_TRY(A, engine.matmul(X, X, false, true));
        NN_TRY(A2, engine.matmul(A, A, false, false));
        NN_CHECK(engine.scale_inplace(A2, c));
        NN_CHECK(engine.scale_inplace(A, b));
        NN_CHECK(engine.add_inplace(A, A2));
        NN_TRY(BX, engine.matmul(A, X, false, false));
        NN_CHECK(engine.axpy_inplace(BX, a, X));
        X = BX;
    }
    return X;
}

// ── Muon (reference compute_optimizer.hpp:499-590) ─────────────────────────
// Per parameter: v = mu v + g (scale_inplace, add_inplace); the update is
// g + mu v (clone g, axpy_inplace) with Nesterov, else v; 2-D parameters
// (rows > 1 and cols > 1) take p -= lr NS(update), the others p -= lr update.
class Muon final : public Optimizer
{
public:
    Muon(ComputeEngine& engine, std::vector<TensorRef> params, std::vector<TensorRef> grads, Scalar lr,
         Scalar momentum = Scalar{0.95f}, bool nesterov = true, std::size_t ns_steps = 5,
         Scalar ns_eps = Scalar{1e-7f})
        : Optimizer(engine, std::move(params), std::move(grads)), lr_(lr), momentum_(momentum), nesterov_(nesterov),
          ns_steps_(ns_steps), ns_eps_(ns_eps)
    {
        v_ = zero_buffers_();
    }
    void set_lr(Scalar lr) override { lr_ = lr; }
    Result<void> step() override
    {
        NN_CHECK(validate_sizes_());
        for (std::size_t i = 0; i < params_.size(); ++i)
        {
            const Tensor& g = grads_[i].get();
            NN_CHECK(engine_.scale_inplace(v_[i], momentum_));
            NN_CHECK(engine_.add_inplace(v_[i], g));
            Tensor update = v_[i];
            if (nesterov_)
            {
                NN_TRY(buf, engine_.clone(g));
                NN_CHECK(engine_.axpy_inplace(buf, momentum_, v_[i]));
                update = buf;
            }
            Tensor& p = params_[i].get();
            if (p.rows() > 1 && p.cols() > 1)
            {
                NN_TRY(ortho, newton_schulz_orthogonalize(engine_, update, ns_steps_, ns_eps_));
                NN_CHECK(engine_.axpy_inplace(p, -lr_, ortho));
            }
            else
                NN_CHECK(engine_.axpy_inplace(p, -lr_, update));
        }
        return {};
    }

private:
    Scalar lr_, momentum_;
    bool nesterov_;
    std::size_t ns_steps_;
    Scalar ns_eps_;
    std::vector<Tensor> v_;
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

// Optimizer by name (reference compute_optimizer.hpp:594-615): "sgd",
// "sgd_momentum", "adam", "adamw", "muon"; an unknown name gives nullptr.
[[nodiscard]] inline std::unique_ptr<Optimizer> create_optimizer(std::string_view name, ComputeEngine& engine,
                                                                 std::vector<TensorRef> params,
                                                                 std::vector<TensorRef> grads, Scalar lr,
                                                                 Scalar weight_decay = 0)
{
    if (name == "sgd") return std::make_unique<SGD>(engine, std::move(params), std::move(grads), lr);
    if (name == "sgd_momentum")
        return std::make_unique<SGDWithMomentum>(engine, std::move(params), std::move(grads), lr);
    if (name == "adam") return std::make_unique<Adam>(engine, std::move(params), std::move(grads), lr);
    if (name == "adamw")
        return std::make_unique<AdamW>(engine, std::move(params), std::move(grads), lr, Scalar{0.9f}, Scalar{0.999f},
                                       Scalar{1e-8f}, weight_decay);
    if (name == "muon") return std::make_unique<Muon>(engine, std::move(params), std::move(grads), lr);
    return nullptr;
}

} // namespace nn
