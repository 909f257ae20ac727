// compute_layer.hpp — the GPT layers, written once against ComputeEngine&.
//
// These are the callers of the hot path. Each forward/backward issues the
// same primitive sequence as the reference's layer (file:line cited per
// class), so any engine that implements the primitives reproduces the
// reference's model. Layout conventions (reference compute_layer.hpp:2788-2792,
// docs/08-pitfalls-and-lessons.md:39-51):
//   * activations are (features, tokens), token column i = b*T + t (batch-major);
//   * Linear: out = W (out,in) x X (in,N) + b (out,1);
//   * attention heads: rearrange_3d(Q (H*dk, B*T), H*dk, B, T) -> (B*H*dk, T),
//     so the batch index of every batched primitive is b*H + h.
// Covered: Linear, SwiGLU, QuickGeLU, RMSNorm, LayerNorm, Softmax, attention
// (two-pass fused path for a pure causal mask, materialised path for ALiBi /
// document masks, RoPE on Q / K), FeedForward, GPTBlock, learned / sinusoidal /
// no position encoders, GPTModel, and incremental inference (forward_step with
// per-layer KV caches, generate).
#pragma once

#include <cmath>
#include <cstddef>
#include <limits>
#include <memory>
#include <random>
#include <span>
#include <vector>

#include "compute_engine.hpp"
#include "expr_dsl.hpp"
#include "layer_exprs.hpp"
#include "model_spec.hpp"
#include "tensor.hpp"

namespace nn
{

[[noreturn]] inline void layer_fatal_(const Error& e)
{
    std::fprintf(stderr, "nn layer construction failed: %s\n", e.message.c_str());
    std::abort();
}
template <class T>
T layer_take_(Result<T> r)
{
    if (!r) layer_fatal_(r.error());
    return std::move(*r);
}
inline void layer_take_(Result<void> r)
{
    if (!r) layer_fatal_(r.error());
}

// Reference compute_layer.hpp:41-80.
class Layer
{
public:
    virtual ~Layer() = default;
    [[nodiscard]] virtual Result<Tensor> forward(ComputeEngine& engine, const Tensor& input) = 0;
    [[nodiscard]] virtual Result<Tensor> backward(ComputeEngine& engine, const Tensor& grad_output) = 0;
    [[nodiscard]] virtual std::vector<TensorRef> parameters() { return {}; }
    [[nodiscard]] virtual std::vector<TensorRef> param_gradients() { return {}; }
    [[nodiscard]] virtual Result<void> zero_grad(ComputeEngine& engine)
    {
        for (auto& g : param_gradients())
            NN_CHECK(engine.zero(g));
        return {};
    }
    virtual void set_flush_interval(std::size_t) {}
    virtual void set_doc_ids(std::span<const std::size_t>) {}
    virtual void set_training(bool) {}
};

template <class... Ts>
void append_refs_(std::vector<TensorRef>& out, Ts&&... lists)
{
    (out.insert(out.end(), lists.begin(), lists.end()), ...);
}

// ── Linear (reference compute_layer.hpp:99-196) ───────────────────────────
//   fwd: out = matmul(W, x); broadcast_row_inplace(out, b, Add)
//   bwd: dx = matmul(W, g, transA); dW += matmul(g, x, transB); db += row_reduce_sum(g)
class Linear final : public Layer
{
public:
    Linear(ComputeEngine& engine, std::size_t in_features, std::size_t out_features)
    {
        // Xavier-uniform from a per-thread generator, as the reference; every
        // harness overwrites the parameters with copy_from.
        static thread_local std::mt19937_64 rng{std::random_device{}()};
        Matrix w(out_features, in_features);
        const Scalar limit = std::sqrt(6.0f / static_cast<Scalar>(in_features + out_features));
        std::uniform_real_distribution<Scalar> dist(-limit, limit);
        for (auto& v : w.span())
            v = dist(rng);
        w_ = layer_take_(engine.from_matrix(w));
        b_ = layer_take_(engine.from_matrix(Matrix(out_features, 1)));
        grad_w_ = engine.create_tensor(out_features, in_features);
        grad_b_ = engine.create_tensor(out_features, 1);
        layer_take_(engine.zero(grad_w_));
        layer_take_(engine.zero(grad_b_));
    }

    std::vector<TensorRef> parameters() override { return {w_, b_}; }
    std::vector<TensorRef> param_gradients() override { return {grad_w_, grad_b_}; }

    Result<Tensor> forward(ComputeEngine& engine, const Tensor& input) override
    {
        if (input.rows() != w_.cols())
            return fail("linear forward: input shape mismatch");
        input_cache_ = input;
        NN_TRY(out, engine.matmul(w_, input, false, false));
        NN_CHECK(engine.broadcast_row_inplace(out, b_, BinaryOp::Add));
        return out;
    }

    Result<Tensor> backward(ComputeEngine& engine, const Tensor& grad_output) override
    {
        if (grad_output.rows() != w_.rows())
            return fail("linear backward: grad_output shape mismatch");
        NN_TRY(grad_input, engine.matmul(w_, grad_output, true, false));
        NN_TRY(gw, engine.matmul(grad_output, input_cache_, false, true));
        NN_CHECK(engine.add_inplace(grad_w_, gw));
        NN_TRY(gb, engine.row_reduce_sum(grad_output));
        NN_CHECK(engine.add_inplace(grad_b_, gb));
        return grad_input;
    }

private:
    Tensor w_, b_, grad_w_, grad_b_, input_cache_;
};

// ── SwiGLU (reference compute_layer.hpp:360-458) ──────────────────────────
//   input (2*d_ff, N) = [gate; up]; out = gate * sigmoid(gate) * up.
//   fwd: slice x2, Neg, Exp, Add 1, Div (1/., scalar first), Mul, Mul.
//   bwd: grad_gate = g*up*(s*(1 + gate*(1-s))), grad_up = g*gate*s, then
//        create_tensor + zero + insert_rows x2.
class SwiGLU final : public Layer
{
public:
    SwiGLU() = default;
    explicit SwiGLU(std::size_t d_ff) : d_ff_(d_ff) {}

    Result<Tensor> forward(ComputeEngine& engine, const Tensor& input) override
    {
        NN_TRY(gate, engine.slice_rows(input, 0, d_ff_));
        NN_TRY(up, engine.slice_rows(input, d_ff_, d_ff_));
        NN_TRY(t1, engine.elementwise_unary(UnaryOp::Neg, gate));
        NN_TRY(t2, engine.elementwise_unary(UnaryOp::Exp, t1));
        NN_TRY(t3, engine.elementwise_binary_scalar(BinaryOp::Add, t2, Scalar{1}));
        NN_TRY(s, engine.elementwise_binary_scalar(BinaryOp::Div, t3, Scalar{1}, true));
        gate_cache_ = gate;
        sigmoid_cache_ = s;
        up_cache_ = up;
        NN_TRY(sw, engine.elementwise_binary(BinaryOp::Mul, gate, s));
        return engine.elementwise_binary(BinaryOp::Mul, sw, up);
    }

    Result<Tensor> backward(ComputeEngine& engine, const Tensor& grad_output) override
    {
        const std::size_t rows = d_ff_, cols = grad_output.cols();
        NN_TRY(grad_gate, dsl::compute(engine,
                                       layer_exprs::swiglu_grad_gate(grad_output, up_cache_, sigmoid_cache_,
                                                                     gate_cache_),
                                       rows, cols));
        NN_TRY(grad_up, dsl::compute(engine, layer_exprs::swiglu_grad_up(grad_output, gate_cache_, sigmoid_cache_),
                                     rows, cols));
        Tensor grad_input = engine.create_tensor(2 * d_ff_, cols);
        NN_CHECK(engine.zero(grad_input));
        NN_CHECK(engine.insert_rows(grad_input, 0, grad_gate));
        NN_CHECK(engine.insert_rows(grad_input, d_ff_, grad_up));
        return grad_input;
    }

private:
    std::size_t d_ff_ = 0;
    Tensor gate_cache_, sigmoid_cache_, up_cache_;
};

// ── RMSNorm (reference compute_layer.hpp:674-801), eps = 1e-5 ─────────────
//   fwd: s = col_reduce_sum(x*x) (1,N); rms_inv = rsqrt(s*(1/F) + eps);
//        normed = x * colbcast(rms_inv); out = normed * rowbcast(gamma)
//   bwd: m = col_reduce_sum(g*gamma*normed) * (1/F);
//        dx = (g*gamma - colbcast(m)*normed) * colbcast(rms_inv);
//        dgamma += row_reduce_sum(g*gamma*normed)
class RMSNorm final : public Layer
{
public:
    explicit RMSNorm(ComputeEngine& engine, std::size_t features, Scalar epsilon = Scalar{1e-5f})
        : features_(features), epsilon_(epsilon)
    {
        gamma_ = layer_take_(engine.from_matrix(Matrix(features, 1, Scalar{1})));
        grad_gamma_ = engine.create_tensor(features, 1);
        layer_take_(engine.zero(grad_gamma_));
    }

    std::vector<TensorRef> parameters() override { return {gamma_}; }
    std::vector<TensorRef> param_gradients() override { return {grad_gamma_}; }

    Result<Tensor> forward(ComputeEngine& engine, const Tensor& input) override
    {
        if (input.rows() != features_)
            return fail("rmsnorm forward: input shape mismatch");
        const Scalar inv_f = Scalar{1} / static_cast<Scalar>(features_);
        const std::size_t F = features_, N = input.cols();
        NN_TRY(s_raw, dsl::compute_reduce(engine, layer_exprs::rms_sum_sq(input), F, N));
        NN_TRY(scaled, engine.elementwise_binary_scalar(BinaryOp::Mul, s_raw, inv_f));
        NN_TRY(var_eps, engine.elementwise_binary_scalar(BinaryOp::Add, scaled, epsilon_));
        NN_TRY(rms_inv, engine.elementwise_unary(UnaryOp::Rsqrt, var_eps));
        rms_inv_cache_ = rms_inv;
        NN_TRY(normed, dsl::compute(engine, layer_exprs::rms_normalize(input, rms_inv_cache_), F, N));
        normed_cache_ = normed;
        return dsl::compute(engine, layer_exprs::rms_scale(normed_cache_, gamma_), F, N);
    }

    Result<Tensor> backward(ComputeEngine& engine, const Tensor& grad_output) override
    {
        const Scalar inv_f = Scalar{1} / static_cast<Scalar>(features_);
        const std::size_t F = features_, N = grad_output.cols();
        NN_TRY(m_raw, dsl::compute_reduce(engine, layer_exprs::rms_bwd_colsum(grad_output, gamma_, normed_cache_),
                                          F, N));
        NN_TRY(m, engine.elementwise_binary_scalar(BinaryOp::Mul, m_raw, inv_f));
        NN_TRY(grad_x, dsl::compute(engine,
                                    layer_exprs::rms_bwd_dx(grad_output, gamma_, m, normed_cache_, rms_inv_cache_),
                                    F, N));
        NN_TRY(gg, dsl::compute_reduce(engine, layer_exprs::rms_bwd_rowsum(grad_output, gamma_, normed_cache_), F, N));
        NN_CHECK(engine.add_inplace(grad_gamma_, gg));
        return grad_x;
    }

private:
    std::size_t features_;
    Scalar epsilon_;
    Tensor gamma_, grad_gamma_, normed_cache_, rms_inv_cache_;
};

// ── QuickGeLU (reference compute_layer.hpp:256-336), beta = 1.702 ─────────
//   fwd: t1 = x*beta; t2 = -t1; t3 = exp(t2); t4 = t3 + 1; s = 1 / t4; out = x*s
//   bwd: 1 - s; beta*x; (beta*x)*(1-s); + 1; s*(.); grad*(.)
class GeLU final : public Layer
{
public:
    static constexpr Scalar kBeta = 1.702f;
    Result<Tensor> forward(ComputeEngine& engine, const Tensor& input) override
    {
        input_cache_ = input;
        NN_TRY(t1, engine.elementwise_binary_scalar(BinaryOp::Mul, input, kBeta));
        NN_TRY(t2, engine.elementwise_unary(UnaryOp::Neg, t1));
        NN_TRY(t3, engine.elementwise_unary(UnaryOp::Exp, t2));
        NN_TRY(t4, engine.elementwise_binary_scalar(BinaryOp::Add, t3, Scalar{1}));
        NN_TRY(sg, engine.elementwise_binary_scalar(BinaryOp::Div, t4, Scalar{1}, true));
        sigmoid_cache_ = sg;
        return engine.elementwise_binary(BinaryOp::Mul, input, sigmoid_cache_);
    }
    Result<Tensor> backward(ComputeEngine& engine, const Tensor& grad_output) override
    {
        if (input_cache_.rows() != grad_output.rows() || input_cache_.cols() != grad_output.cols())
            return fail("gelu backward: shape mismatch");
        NN_TRY(one_minus_s, engine.elementwise_binary_scalar(BinaryOp::Sub, sigmoid_cache_, Scalar{1}, true));
        NN_TRY(bx, engine.elementwise_binary_scalar(BinaryOp::Mul, input_cache_, kBeta));
        NN_TRY(inner, engine.elementwise_binary(BinaryOp::Mul, bx, one_minus_s));
        NN_TRY(paren, engine.elementwise_binary_scalar(BinaryOp::Add, inner, Scalar{1}));
        NN_TRY(factor, engine.elementwise_binary(BinaryOp::Mul, sigmoid_cache_, paren));
        return engine.elementwise_binary(BinaryOp::Mul, grad_output, factor);
    }

private:
    Tensor input_cache_, sigmoid_cache_;
};

// ── LayerNorm (reference compute_layer.hpp:479-662), eps = 1e-5 ───────────
//   fwd: mean = ColSum(x)*(1/F); diff = x - colbcast(mean); var = ColSum(diff^2)*(1/F);
//        std_inv = rsqrt(var + eps); normed = diff*colbcast(std_inv);
//        out = normed*rowbcast(gamma) + rowbcast(beta)
//   bwd: mean_g = ColSum(g*gamma)/F; mean_gn = ColSum(g*gamma*normed)/F;
//        dx = (g*gamma - mean_g - normed*mean_gn)*std_inv;
//        dgamma += RowSum(g*gamma*normed) (gamma times the true gradient, as the
//        reference accumulates it); dbeta += RowSum(g)
class LayerNorm final : public Layer
{
public:
    explicit LayerNorm(ComputeEngine& engine, std::size_t features, Scalar epsilon = Scalar{1e-5f})
        : features_(features), epsilon_(epsilon)
    {
        gamma_ = layer_take_(engine.from_matrix(Matrix(features, 1, Scalar{1})));
        beta_ = layer_take_(engine.from_matrix(Matrix(features, 1, Scalar{0})));
        grad_gamma_ = engine.create_tensor(features, 1);
        grad_beta_ = engine.create_tensor(features, 1);
        layer_take_(engine.zero(grad_gamma_));
        layer_take_(engine.zero(grad_beta_));
    }

    std::vector<TensorRef> parameters() override { return {gamma_, beta_}; }
    std::vector<TensorRef> param_gradients() override { return {grad_gamma_, grad_beta_}; }

    Result<Tensor> forward(ComputeEngine& engine, const Tensor& input) override
    {
        if (input.rows() != features_)
            return fail("layernorm forward: input shape mismatch");
        const Scalar inv_f = Scalar{1} / static_cast<Scalar>(features_);
        const std::size_t F = features_, N = input.cols();
        NN_TRY(mean_raw, dsl::compute_reduce(engine, layer_exprs::ln_col_sum(input), F, N));
        NN_TRY(mean, engine.elementwise_binary_scalar(BinaryOp::Mul, mean_raw, inv_f));
        NN_TRY(diff, dsl::compute(engine, layer_exprs::ln_center(input, mean), F, N));
        NN_TRY(var_raw, dsl::compute_reduce(engine, layer_exprs::ln_sum_sq(diff), F, N));
        NN_TRY(var, engine.elementwise_binary_scalar(BinaryOp::Mul, var_raw, inv_f));
        NN_TRY(var_eps, engine.elementwise_binary_scalar(BinaryOp::Add, var, epsilon_));
        NN_TRY(std_inv, engine.elementwise_unary(UnaryOp::Rsqrt, var_eps));
        std_cache_ = std_inv;
        NN_TRY(normed, dsl::compute(engine, layer_exprs::ln_normalize(diff, std_cache_), F, N));
        normed_cache_ = normed;
        return dsl::compute(engine, layer_exprs::ln_affine(normed_cache_, gamma_, beta_), F, N);
    }

    Result<Tensor> backward(ComputeEngine& engine, const Tensor& grad_output) override
    {
        const Scalar inv_f = Scalar{1} / static_cast<Scalar>(features_);
        const std::size_t F = features_, N = grad_output.cols();
        NN_TRY(mg_raw, dsl::compute_reduce(engine, layer_exprs::ln_bwd_colsum_g(grad_output, gamma_), F, N));
        NN_TRY(mean_g, engine.elementwise_binary_scalar(BinaryOp::Mul, mg_raw, inv_f));
        NN_TRY(mgn_raw, dsl::compute_reduce(engine, layer_exprs::ln_bwd_colsum_gn(grad_output, gamma_, normed_cache_),
                                            F, N));
        NN_TRY(mean_gn, engine.elementwise_binary_scalar(BinaryOp::Mul, mgn_raw, inv_f));
        NN_TRY(grad_x, dsl::compute(engine,
                                    layer_exprs::ln_bwd_dx(grad_output, gamma_, mean_g, normed_cache_, mean_gn,
                                                           std_cache_),
                                    F, N));
        NN_TRY(gg, dsl::compute_reduce(engine, layer_exprs::ln_bwd_rowsum_gn(grad_output, gamma_, normed_cache_), F,
                                       N));
        NN_CHECK(engine.add_inplace(grad_gamma_, gg));
        NN_TRY(gb, dsl::compute_reduce(engine, layer_exprs::ln_bwd_rowsum(grad_output), F, N));
        NN_CHECK(engine.add_inplace(grad_beta_, gb));
        return grad_x;
    }

private:
    std::size_t features_;
    Scalar epsilon_;
    Tensor gamma_, beta_, grad_gamma_, grad_beta_, normed_cache_, std_cache_;
};

// Reference compute_layer.hpp:804-810.
[[nodiscard]] inline std::unique_ptr<Layer> make_norm_layer(ComputeEngine& engine, std::size_t d_model,
                                                            NormType norm_type)
{
    if (norm_type == NormType::RMSNorm)
        return std::make_unique<RMSNorm>(engine, d_model);
    return std::make_unique<LayerNorm>(engine, d_model);
}

// ── Softmax over rows (reference compute_layer.hpp:824-863) ───────────────
//   fwd: exp(x - rowmax(x)) / RowSum(exp(x - rowmax(x)))
//   bwd: out * (g - RowSum(out * g))
class Softmax final : public Layer
{
public:
    Result<Tensor> forward(ComputeEngine& engine, const Tensor& input) override
    {
        NN_TRY(out, dsl::compute(engine, layer_exprs::softmax_rows(input), input.rows(), input.cols()));
        output_cache_ = out;
        return out;
    }
    Result<Tensor> backward(ComputeEngine& engine, const Tensor& grad_output) override
    {
        return dsl::compute(engine, layer_exprs::softmax_rows_backward(output_cache_, grad_output),
                            output_cache_.rows(), output_cache_.cols());
    }

private:
    Tensor output_cache_;
};

// ── RotaryEmbedding (reference compute_layer.hpp:884-984) ─────────────────
// Half-swap convention: q_rot = q*cos + rotate_half(q)*sin, rotate_half(x) =
// [-x_second_half, x_first_half] per d_k block; cos[j] = cos[j + d_k/2] =
// cos(pos * theta_j), theta_j = 10000^(-2j/d_k). The tables are (d_k, seq) and
// read with RowMod(d_k) by the (B*H*d_k, seq) heads; backward rotates by the
// opposite angle (the rotation is orthogonal).
class RotaryEmbedding
{
public:
    RotaryEmbedding() = default;
    explicit RotaryEmbedding(std::size_t d_k) : d_k_(d_k) {}

    Result<Tensor> apply(ComputeEngine& engine, const Tensor& q, std::size_t seq, bool backward)
    {
        if (d_k_ == 0 || d_k_ % 2 != 0)
            return fail("RotaryEmbedding::apply: d_k must be positive and even");
        if (seq != seq_cached_)
        {
            Matrix c(d_k_, seq), sn(d_k_, seq);
            for (std::size_t pos = 0; pos < seq; ++pos)
                fill_column_(c, sn, pos, pos);
            NN_TRY(ct, engine.from_matrix(c));
            NN_TRY(st, engine.from_matrix(sn));
            cos_ = ct;
            sin_ = st;
            seq_cached_ = seq;
        }
        return rotate_(engine, q, cos_, sin_, backward);
    }

    // One position (incremental inference): q is (H*d_k, 1).
    Result<Tensor> apply_step(ComputeEngine& engine, const Tensor& q, std::size_t pos, bool backward)
    {
        if (d_k_ == 0 || d_k_ % 2 != 0)
            return fail("RotaryEmbedding::apply_step: d_k must be positive and even");
        Matrix c(d_k_, 1), sn(d_k_, 1);
        fill_column_(c, sn, pos, 0);
        NN_TRY(ct, engine.from_matrix(c));
        NN_TRY(st, engine.from_matrix(sn));
        return rotate_(engine, q, ct, st, backward);
    }

private:
    void fill_column_(Matrix& c, Matrix& sn, std::size_t pos, std::size_t col) const
    {
        const std::size_t half = d_k_ / 2;
        for (std::size_t j = 0; j < half; ++j)
        {
            const Scalar theta = static_cast<Scalar>(pos) /
                                 std::pow(Scalar{10000}, static_cast<Scalar>(2 * j) / static_cast<Scalar>(d_k_));
            const Scalar cv = std::cos(theta), sv = std::sin(theta);
            c.set_value_unchecked(j, col, cv);
            c.set_value_unchecked(half + j, col, cv);
            sn.set_value_unchecked(j, col, sv);
            sn.set_value_unchecked(half + j, col, sv);
        }
    }
    Result<Tensor> rotate_(ComputeEngine& engine, const Tensor& q, const Tensor& c, const Tensor& sn, bool backward)
    {
        const auto dk = static_cast<std::uint32_t>(d_k_);
        if (backward)
            return dsl::compute(engine, layer_exprs::rope_backward(q, c, sn, dk), q.rows(), q.cols());
        return dsl::compute(engine, layer_exprs::rope_forward(q, c, sn, dk), q.rows(), q.cols());
    }

    std::size_t d_k_ = 0, seq_cached_ = 0;
    Tensor cos_, sin_;
};

// ── multi-head attention core (reference compute_layer.hpp:1016-1412) ─────
class AttentionBase : public Layer
{
public:
    AttentionBase(ComputeEngine& engine, std::size_t d_model, std::size_t num_heads, std::size_t seq_len,
                  PosEncodingType pos_enc = PosEncodingType::Learned)
        : d_model_(d_model), num_heads_(num_heads), d_k_(d_model / num_heads), seq_len_(seq_len),
          scale_(Scalar{1} / std::sqrt(static_cast<Scalar>(d_model / num_heads))),
          w_q_(engine, d_model, d_model), w_k_(engine, d_model, d_model), w_v_(engine, d_model, d_model),
          w_o_(engine, d_model, d_model), use_rope_(pos_enc == PosEncodingType::RoPE), rope_(d_model / num_heads)
    {
    }

    std::vector<TensorRef> parameters() override
    {
        std::vector<TensorRef> p;
        append_refs_(p, w_q_.parameters(), w_k_.parameters(), w_v_.parameters(), w_o_.parameters());
        return p;
    }
    std::vector<TensorRef> param_gradients() override
    {
        std::vector<TensorRef> g;
        append_refs_(g, w_q_.param_gradients(), w_k_.param_gradients(), w_v_.param_gradients(),
                     w_o_.param_gradients());
        return g;
    }

    Result<Tensor> forward(ComputeEngine& engine, const Tensor& input) override
    {
        if (input.rows() != d_model_)
            return fail("attention forward: input shape mismatch");
        const std::size_t total = input.cols();
        const std::size_t seq = seq_len_ > 0 ? seq_len_ : total;
        const std::size_t batch = seq_len_ > 0 ? total / seq_len_ : 1;
        if (total != batch * seq)
            return fail("attention forward: cols not divisible by seq_len");
        const std::size_t H_dk = num_heads_ * d_k_, BH = batch * num_heads_;

        NN_TRY(q, w_q_.forward(engine, input));
        NN_TRY(k, w_k_.forward(engine, input));
        NN_TRY(v, w_v_.forward(engine, input));
        if (batch > 1)
        {
            NN_TRY(qr, engine.rearrange_3d(q, H_dk, batch, seq, false));
            NN_TRY(kr, engine.rearrange_3d(k, H_dk, batch, seq, false));
            NN_TRY(vr, engine.rearrange_3d(v, H_dk, batch, seq, false));
            Q_ = qr;
            K_ = kr;
            V_ = vr;
        }
        else
        {
            Q_ = q;
            K_ = k;
            V_ = v;
        }
        if (use_rope_)   // reference :1176-1186, on the (B*H*d_k, seq) heads
        {
            NN_TRY(qr2, rope_.apply(engine, Q_, seq, false));
            Q_ = qr2;
            NN_TRY(kr2, rope_.apply(engine, K_, seq, false));
            K_ = kr2;
        }

        NN_TRY(tpm, two_pass_mask_(engine, batch, seq));
        Tensor heads_out;   // (BH*dk, seq)
        if (tpm.use_two_pass)
        {
            // Two-pass path (reference :1193-1229): m, l, then O = softmax-weighted V.
            shared_mask_ = tpm.mask;
            const Tensor* mask = shared_mask_.rows() > 0 ? &shared_mask_ : nullptr;
            NN_TRY(m, engine.batched_matmul_reduce(Q_, K_, BH, ReduceOp::Max, true, false, scale_, true, mask));
            NN_TRY(l, engine.batched_matmul_softmax_denom(Q_, K_, m, BH, true, false, scale_, mask));
            NN_TRY(vt_full, engine.transpose(V_));                         // (seq, BH*dk)
            NN_TRY(vt, engine.rearrange_3d(vt_full, seq, BH, d_k_, false));  // (BH*seq, dk)
            NN_TRY(ot, engine.batched_matmul_softmax_apply(Q_, K_, vt, m, l, BH, true, false, scale_, mask));
            NN_TRY(ot_full, engine.transpose(ot));                         // (dk, BH*seq)
            NN_TRY(co, engine.rearrange_3d(ot_full, d_k_, BH, seq, false));  // (BH*dk, seq)
            heads_out = co;
            m_ = m;
            l_ = l;
            two_pass_ = true;
        }
        else
        {
            // Materialised path (reference :1230-1252).
            two_pass_ = false;
            NN_TRY(scores, engine.batched_matmul(Q_, K_, BH, true, false, scale_));
            NN_TRY(masked, apply_mask_(engine, std::move(scores), batch, seq));
            NN_TRY(attn, softmax_.forward(engine, masked));
            attn_ = attn;
            NN_TRY(co, engine.batched_matmul(V_, attn_, BH, false, true));
            heads_out = co;
        }

        Tensor concat = heads_out;
        if (batch > 1)
        {
            NN_TRY(cb, engine.rearrange_3d(heads_out, H_dk, batch, seq, true));
            concat = cb;
        }
        return w_o_.forward(engine, concat);
    }

    Result<Tensor> backward(ComputeEngine& engine, const Tensor& grad_output) override
    {
        const std::size_t total = grad_output.cols();
        const std::size_t seq = seq_len_ > 0 ? seq_len_ : total;
        const std::size_t batch = seq_len_ > 0 ? total / seq_len_ : 1;
        const std::size_t H_dk = num_heads_ * d_k_, BH = batch * num_heads_;

        NN_TRY(gc, w_o_.backward(engine, grad_output));
        Tensor gre = gc;
        if (batch > 1)
        {
            NN_TRY(r, engine.rearrange_3d(gc, H_dk, batch, seq, false));
            gre = r;
        }

        Tensor gQ, gK, gV;   // (BH*dk, seq)
        if (two_pass_)
        {
            // Reference :1300-1330.
            const Tensor* mask = shared_mask_.rows() > 0 ? &shared_mask_ : nullptr;
            NN_TRY(P, engine.batched_matmul(gre, V_, BH, true, false));              // (BH*seq, seq)
            NN_TRY(gt_full, engine.transpose(gre));
            NN_TRY(G, engine.rearrange_3d(gt_full, seq, BH, d_k_, false));           // (BH*seq, dk)
            Tensor R;
            NN_TRY(gq, engine.batched_matmul_softmax_backward_q(Q_, K_, P, m_, l_, BH, true, false, scale_, R, mask));
            NN_TRY(gk, engine.batched_matmul_softmax_backward_kv(Q_, K_, P, G, R, m_, l_, BH, true, false, scale_, gV,
                                                                 mask));
            gQ = gq;
            gK = gk;
        }
        else
        {
            // Reference :1331-1361.
            NN_TRY(gv, engine.batched_matmul(gre, attn_, BH, false, false));
            gV = gv;
            NN_TRY(gA, engine.batched_matmul(gre, V_, BH, true, false));
            NN_TRY(gS, softmax_.backward(engine, gA));
            NN_TRY(gq, engine.batched_matmul(K_, gS, BH, false, true, scale_));
            NN_TRY(gk, engine.batched_matmul(Q_, gS, BH, false, false, scale_));
            gQ = gq;
            gK = gk;
        }
        if (use_rope_)   // reference :1363-1372: the inverse rotation of the Q / K gradients
        {
            NN_TRY(gq2, rope_.apply(engine, gQ, seq, true));
            gQ = gq2;
            NN_TRY(gk2, rope_.apply(engine, gK, seq, true));
            gK = gk2;
        }

        if (batch > 1)
        {
            NN_TRY(a, engine.rearrange_3d(gQ, H_dk, batch, seq, true));
            NN_TRY(b, engine.rearrange_3d(gK, H_dk, batch, seq, true));
            NN_TRY(c, engine.rearrange_3d(gV, H_dk, batch, seq, true));
            gQ = a;
            gK = b;
            gV = c;
        }

        NN_TRY(dx, w_q_.backward(engine, gQ));
        NN_TRY(dxk, w_k_.backward(engine, gK));
        NN_CHECK(engine.add_inplace(dx, dxk));
        NN_TRY(dxv, w_v_.backward(engine, gV));
        NN_CHECK(engine.add_inplace(dx, dxv));
        return dx;
    }

    // Incremental inference, one token (reference compute_layer.hpp:1426-1511):
    // x_new (d_model, 1); the caches are (seq_len, d_model) with rows [0, cur_len)
    // holding the earlier tokens' K / V. Writes row cur_len, attends over rows
    // [0, cur_len] (no causal mask needed: the cache holds only earlier tokens).
    Result<Tensor> forward_step(ComputeEngine& engine, const Tensor& x_new, Tensor& k_cache, Tensor& v_cache,
                                std::size_t cur_len)
    {
        if (x_new.rows() != d_model_ || x_new.cols() != 1)
            return fail("AttentionBase forward_step: x_new must be (d_model, 1)");
        NN_TRY(q0, w_q_.forward(engine, x_new));
        NN_TRY(k0, w_k_.forward(engine, x_new));
        NN_TRY(v_new, w_v_.forward(engine, x_new));
        Tensor q = q0, k_new = k0;
        if (use_rope_)
        {
            NN_TRY(qr, rope_.apply_step(engine, q, cur_len, false));
            q = qr;
            NN_TRY(kr, rope_.apply_step(engine, k_new, cur_len, false));
            k_new = kr;
        }
        NN_TRY(k_new_T, engine.transpose(k_new));   // (1, H*d_k), the cache's row layout
        NN_TRY(v_new_T, engine.transpose(v_new));
        NN_CHECK(engine.insert_rows(k_cache, cur_len, k_new_T));
        NN_CHECK(engine.insert_rows(v_cache, cur_len, v_new_T));
        const std::size_t new_len = cur_len + 1;
        NN_TRY(k_valid, engine.slice_rows(k_cache, 0, new_len));
        NN_TRY(v_valid, engine.slice_rows(v_cache, 0, new_len));
        NN_TRY(K_T, engine.transpose(k_valid));     // (H*d_k, new_len)
        NN_TRY(V_T, engine.transpose(v_valid));
        NN_TRY(scores, engine.batched_matmul(q, K_T, num_heads_, true, false, scale_));   // (H, new_len)
        NN_TRY(masked, apply_mask_step_(engine, std::move(scores), cur_len));
        NN_TRY(attn, softmax_.forward(engine, masked));
        NN_TRY(attn_out, engine.batched_matmul(V_T, attn, num_heads_, false, true));   // (H*d_k, 1)
        return w_o_.forward(engine, attn_out);
    }

protected:
    struct TwoPassMask
    {
        bool use_two_pass = true;
        Tensor mask;
    };
    // Incremental-inference mask hook (reference :1076-1081): none by default.
    virtual Result<Tensor> apply_mask_step_(ComputeEngine&, Tensor&& scores, std::size_t) { return std::move(scores); }
    virtual Result<TwoPassMask> two_pass_mask_(ComputeEngine&, std::size_t, std::size_t)
    {
        return TwoPassMask{true, {}};
    }
    virtual Result<Tensor> apply_mask_(ComputeEngine&, Tensor&& scores, std::size_t, std::size_t)
    {
        return std::move(scores);
    }

    std::size_t d_model_, num_heads_, d_k_, seq_len_;
    Scalar scale_;
    Linear w_q_, w_k_, w_v_, w_o_;
    Softmax softmax_;
    Tensor Q_, K_, V_;           // (BH*dk, seq)
    Tensor attn_;                // (BH*seq, seq), materialised path
    Tensor m_, l_, shared_mask_; // two-pass path
    bool two_pass_ = false;
    bool use_rope_ = false;
    RotaryEmbedding rope_;
};

// ── build_attention_mask (reference compute_layer.hpp:2081-2128) ──────────
// (BH*seq, seq): row (b*H + h)*seq + i, column j. Allowed iff j <= i and, with
// document ids, doc[b*seq+i] == doc[b*seq+j]; the value is -slope_h*(i-j)
// with ALiBi, 0 otherwise; excluded entries are -inf.
[[nodiscard]] inline Matrix build_attention_mask(std::size_t batch, std::size_t seq, std::size_t heads,
                                                 bool use_alibi, std::span<const Scalar> slopes,
                                                 std::span<const std::size_t> doc_ids = {})
{
    const Scalar neg_inf = -std::numeric_limits<Scalar>::infinity();
    Matrix mask(batch * heads * seq, seq);
    for (std::size_t b = 0; b < batch; ++b)
        for (std::size_t h = 0; h < heads; ++h)
        {
            const Scalar slope = use_alibi ? slopes[h] : Scalar{0};
            const std::size_t base = (b * heads + h) * seq;
            for (std::size_t i = 0; i < seq; ++i)
                for (std::size_t j = 0; j < seq; ++j)
                {
                    bool ok = j <= i;
                    if (ok && !doc_ids.empty())
                        ok = doc_ids[b * seq + i] == doc_ids[b * seq + j];
                    mask.set_value_unchecked(base + i, j,
                                             ok ? (use_alibi ? -slope * static_cast<Scalar>(i - j) : Scalar{0})
                                                : neg_inf);
                }
        }
    return mask;
}

// ALiBi slopes m_h = 2^(-8h/H), h = 0..H-1 (reference compute_layer.hpp:2179-2187;
// note head 0 has slope 1).
[[nodiscard]] inline std::vector<Scalar> alibi_slopes(std::size_t heads)
{
    std::vector<Scalar> s(heads);
    for (std::size_t h = 0; h < heads; ++h)
        s[h] = std::pow(Scalar{2}, -Scalar{8} * static_cast<Scalar>(h) / static_cast<Scalar>(heads));
    return s;
}

// The ALiBi bias of one incremental-inference position (H, new_len), uploaded
// once and read by every attention layer of a model that shares the cache:
// the layers' slopes are equal (they depend on the head count only), so at one
// position their biases are equal too and one upload serves them all.
struct StepBiasCache
{
    std::size_t heads = 0, len = 0;
    Tensor bias;
};

// ── CausalSelfAttention (reference compute_layer.hpp:2156-2304) ───────────
// Pure causal -> two-pass path with a shared (seq,seq) mask; ALiBi or
// document ids -> materialised path with a (BH*seq, seq) mask added to S.
class CausalSelfAttention final : public AttentionBase
{
public:
    CausalSelfAttention(ComputeEngine& engine, std::size_t d_model, std::size_t num_heads, std::size_t seq_len,
                        PosEncodingType pos_enc)
        : AttentionBase(engine, d_model, num_heads, seq_len, pos_enc), use_alibi_(pos_enc == PosEncodingType::ALiBi)
    {
        if (use_alibi_)
            slopes_ = alibi_slopes(num_heads);
    }

    void set_doc_ids(std::span<const std::size_t> ids) override { doc_ids_.assign(ids.begin(), ids.end()); }

protected:
    Result<Tensor> apply_mask_(ComputeEngine& engine, Tensor&& scores, std::size_t batch, std::size_t seq) override
    {
        if (!doc_ids_.empty())
        {
            // Document masks change every step: rebuilt, never cached.
            NN_TRY(mt, engine.from_matrix(build_attention_mask(batch, seq, num_heads_, use_alibi_, slopes_, doc_ids_)));
            return engine.elementwise_binary(BinaryOp::Add, scores, mt);
        }
        if (mask_batch_ != batch || mask_seq_ != seq)
        {
            NN_TRY(mt, engine.from_matrix(build_attention_mask(batch, seq, num_heads_, use_alibi_, slopes_)));
            mask_ = mt;
            mask_batch_ = batch;
            mask_seq_ = seq;
        }
        return engine.elementwise_binary(BinaryOp::Add, scores, mask_);
    }

    // ALiBi at inference (reference :2267-2290): scores (H, cur_len + 1) +=
    // -slope_h * (cur_len - j), the query at position cur_len.
    Result<Tensor> apply_mask_step_(ComputeEngine& engine, Tensor&& scores, std::size_t cur_len) override
    {
        if (!use_alibi_) return std::move(scores);
        const std::size_t new_len = cur_len + 1;
        StepBiasCache& c = *step_bias_;
        if (c.heads != num_heads_ || c.len != new_len || c.bias.size() != num_heads_ * new_len)
        {
            Matrix bias(num_heads_, new_len);
            for (std::size_t h = 0; h < num_heads_; ++h)
                for (std::size_t j = 0; j < new_len; ++j)
                    bias.set_value_unchecked(h, j, -slopes_[h] * static_cast<Scalar>(cur_len - j));
            NN_TRY(bt, engine.from_matrix(bias));
            c = StepBiasCache{num_heads_, new_len, bt};
        }
        return engine.elementwise_binary(BinaryOp::Add, scores, c.bias);
    }

public:
    // Layers of one model (same engine, same head count) share one cache.
    void share_step_bias(std::shared_ptr<StepBiasCache> c) { step_bias_ = std::move(c); }

protected:

    Result<TwoPassMask> two_pass_mask_(ComputeEngine& engine, std::size_t, std::size_t seq) override
    {
        if (use_alibi_ || !doc_ids_.empty())
            return TwoPassMask{false, {}};
        if (causal_seq_ != seq)
        {
            Matrix m(seq, seq, Scalar{0});
            for (std::size_t i = 0; i < seq; ++i)
                for (std::size_t j = i + 1; j < seq; ++j)
                    m.set_value_unchecked(i, j, -std::numeric_limits<Scalar>::infinity());
            NN_TRY(t, engine.from_matrix(m));
            causal_ = t;
            causal_seq_ = seq;
        }
        return TwoPassMask{true, causal_};
    }

private:
    bool use_alibi_;
    std::vector<Scalar> slopes_;
    std::shared_ptr<StepBiasCache> step_bias_ = std::make_shared<StepBiasCache>();
    std::vector<std::size_t> doc_ids_;
    Tensor mask_;
    std::size_t mask_batch_ = 0, mask_seq_ = 0;
    Tensor causal_;
    std::size_t causal_seq_ = 0;
};

// ── FeedForward with SwiGLU (reference compute_layer.hpp:1623-1689) ───────
// QuickGeLU FFN: fc1 d_model -> d_ff; SwiGLU FFN: fc1 d_model -> 2*d_ff.
class FeedForward final : public Layer
{
public:
    FeedForward(ComputeEngine& engine, std::size_t d_model, std::size_t d_ff,
                ActivationType activation = ActivationType::SwiGLU)
        : fc1_(engine, d_model, activation == ActivationType::SwiGLU ? 2 * d_ff : d_ff), fc2_(engine, d_ff, d_model),
          act_(d_ff), use_swiglu_(activation == ActivationType::SwiGLU)
    {
    }
    std::vector<TensorRef> parameters() override
    {
        std::vector<TensorRef> p;
        append_refs_(p, fc1_.parameters(), fc2_.parameters());
        return p;
    }
    std::vector<TensorRef> param_gradients() override
    {
        std::vector<TensorRef> g;
        append_refs_(g, fc1_.param_gradients(), fc2_.param_gradients());
        return g;
    }
    Result<Tensor> forward(ComputeEngine& engine, const Tensor& input) override
    {
        NN_TRY(h1, fc1_.forward(engine, input));
        Tensor h2;
        if (use_swiglu_)
        {
            NN_TRY(a, act_.forward(engine, h1));
            h2 = a;
        }
        else
        {
            NN_TRY(a, gelu_.forward(engine, h1));
            h2 = a;
        }
        return fc2_.forward(engine, h2);
    }
    Result<Tensor> backward(ComputeEngine& engine, const Tensor& grad_output) override
    {
        NN_TRY(b2, fc2_.backward(engine, grad_output));
        Tensor bg;
        if (use_swiglu_)
        {
            NN_TRY(g, act_.backward(engine, b2));
            bg = g;
        }
        else
        {
            NN_TRY(g, gelu_.backward(engine, b2));
            bg = g;
        }
        return fc1_.backward(engine, bg);
    }

private:
    Linear fc1_, fc2_;
    SwiGLU act_;
    GeLU gelu_;
    bool use_swiglu_;
};

// ── GPTBlock, pre-norm (reference compute_layer.hpp:2313-2405) ────────────
//   x1 = x + Attn(N1(x)); out = x1 + FFN(N2(x1))
class GPTBlock final : public Layer
{
public:
    GPTBlock(ComputeEngine& engine, std::size_t d_model, std::size_t heads, std::size_t d_ff, std::size_t seq_len,
             PosEncodingType pos_enc, ActivationType activation = ActivationType::SwiGLU,
             NormType norm_type = NormType::RMSNorm)
        : attn_(engine, d_model, heads, seq_len, pos_enc), norm1_(make_norm_layer(engine, d_model, norm_type)),
          ff_(engine, d_model, d_ff, activation), norm2_(make_norm_layer(engine, d_model, norm_type))
    {
    }
    std::vector<TensorRef> parameters() override
    {
        std::vector<TensorRef> p;
        append_refs_(p, attn_.parameters(), norm1_->parameters(), ff_.parameters(), norm2_->parameters());
        return p;
    }
    std::vector<TensorRef> param_gradients() override
    {
        std::vector<TensorRef> g;
        append_refs_(g, attn_.param_gradients(), norm1_->param_gradients(), ff_.param_gradients(),
                     norm2_->param_gradients());
        return g;
    }
    void set_doc_ids(std::span<const std::size_t> ids) override { attn_.set_doc_ids(ids); }

    Result<Tensor> forward(ComputeEngine& engine, const Tensor& input) override
    {
        NN_TRY(n1, norm1_->forward(engine, input));
        NN_TRY(a, attn_.forward(engine, n1));
        NN_TRY(r2, engine.elementwise_binary(BinaryOp::Add, input, a));
        residual_ = r2;
        NN_TRY(n2, norm2_->forward(engine, residual_));
        NN_TRY(f, ff_.forward(engine, n2));
        return engine.elementwise_binary(BinaryOp::Add, residual_, f);
    }
    Result<Tensor> backward(ComputeEngine& engine, const Tensor& grad_output) override
    {
        NN_TRY(gff, ff_.backward(engine, grad_output));
        NN_TRY(gn2, norm2_->backward(engine, gff));
        NN_TRY(gr1, engine.elementwise_binary(BinaryOp::Add, grad_output, gn2));
        NN_TRY(gsa, attn_.backward(engine, gr1));
        NN_TRY(gn1, norm1_->backward(engine, gsa));
        return engine.elementwise_binary(BinaryOp::Add, gr1, gn1);
    }

    // One token through the block with the layer's KV cache (reference :2413-2437).
    Result<Tensor> forward_step(ComputeEngine& engine, const Tensor& x_new, Tensor& k_cache, Tensor& v_cache,
                                std::size_t cur_len)
    {
        NN_TRY(n1, norm1_->forward(engine, x_new));
        NN_TRY(a, attn_.forward_step(engine, n1, k_cache, v_cache, cur_len));
        NN_TRY(r2, engine.elementwise_binary(BinaryOp::Add, x_new, a));
        NN_TRY(n2, norm2_->forward(engine, r2));
        NN_TRY(f, ff_.forward(engine, n2));
        return engine.elementwise_binary(BinaryOp::Add, r2, f);
    }

    void share_step_bias(std::shared_ptr<StepBiasCache> c) { attn_.share_step_bias(std::move(c)); }

private:
    CausalSelfAttention attn_;
    std::unique_ptr<Layer> norm1_;
    FeedForward ff_;
    std::unique_ptr<Layer> norm2_;
    Tensor residual_;
};

// ── position encoders (reference compute_layer.hpp:2458-2644) ─────────────
class PositionEncoder
{
public:
    virtual ~PositionEncoder() = default;
    virtual Result<Tensor> apply(ComputeEngine& engine, const Tensor& emb_T, std::size_t batch, std::size_t seq) = 0;
    // One position at inference (reference :2467-2468): x (d_model, 1).
    virtual Result<Tensor> apply_step(ComputeEngine& engine, const Tensor& x, std::size_t pos) = 0;
    virtual Result<void> backward(ComputeEngine& engine, const Tensor& grad_T) = 0;
    virtual std::vector<TensorRef> parameters() { return {}; }
    virtual std::vector<TensorRef> param_gradients() { return {}; }
};

// Additive table (learned or sinusoidal): x + transpose(gather_rows(pos_emb, pos_idx)),
// pos_idx[b*seq + t] = t; backward scatter_add_rows into the table gradient.
class AdditivePositionEncoder final : public PositionEncoder
{
public:
    AdditivePositionEncoder(ComputeEngine& engine, Matrix table, bool learnable) : learnable_(learnable)
    {
        const std::size_t r = table.rows(), c = table.cols();
        table_ = layer_take_(engine.from_matrix(table));
        if (learnable_)
        {
            grad_ = engine.create_tensor(r, c);
            layer_take_(engine.zero(grad_));
        }
    }
    Result<Tensor> apply(ComputeEngine& engine, const Tensor& emb_T, std::size_t batch, std::size_t seq) override
    {
        if (idx_batch_ != batch || idx_seq_ != seq)
        {
            Matrix idx(batch * seq, 1);
            for (std::size_t b = 0; b < batch; ++b)
                for (std::size_t t = 0; t < seq; ++t)
                    idx.set_value_unchecked(b * seq + t, 0, static_cast<Scalar>(t));
            NN_TRY(it, engine.from_matrix(idx));
            idx_ = it;
            idx_batch_ = batch;
            idx_seq_ = seq;
        }
        NN_TRY(g, engine.gather_rows(table_, idx_));
        NN_TRY(gT, engine.transpose(g));
        return engine.elementwise_binary(BinaryOp::Add, emb_T, gT);
    }
    // Reference :2550-2565: x + transpose(gather_rows(table, [pos])).
    Result<Tensor> apply_step(ComputeEngine& engine, const Tensor& x, std::size_t pos) override
    {
        NN_TRY(pt, engine.from_matrix(Matrix(1, 1, static_cast<Scalar>(pos))));
        NN_TRY(g, engine.gather_rows(table_, pt));
        NN_TRY(gT, engine.transpose(g));
        return engine.elementwise_binary(BinaryOp::Add, x, gT);
    }
    Result<void> backward(ComputeEngine& engine, const Tensor& grad_T) override
    {
        if (!learnable_)
            return {};
        return engine.scatter_add_rows(grad_, idx_, grad_T);
    }
    std::vector<TensorRef> parameters() override
    {
        if (!learnable_) return {};
        return {table_};
    }
    std::vector<TensorRef> param_gradients() override
    {
        if (!learnable_) return {};
        return {grad_};
    }

private:
    bool learnable_;
    Tensor table_, grad_, idx_;
    std::size_t idx_batch_ = 0, idx_seq_ = 0;
};

class NoPositionEncoder final : public PositionEncoder
{
public:
    Result<Tensor> apply(ComputeEngine&, const Tensor& emb_T, std::size_t, std::size_t) override { return emb_T; }
    Result<Tensor> apply_step(ComputeEngine&, const Tensor& x, std::size_t) override { return x; }
    Result<void> backward(ComputeEngine&, const Tensor&) override { return {}; }
};

// Sinusoidal table PE(pos, i) = sin/cos(pos / 10000^(2*(i/2)/d)) (reference :2605-2622).
[[nodiscard]] inline Matrix sinusoidal_table(std::size_t seq, std::size_t d)
{
    Matrix pe(seq, d);
    for (std::size_t pos = 0; pos < seq; ++pos)
        for (std::size_t i = 0; i < d; ++i)
        {
            const Scalar angle = static_cast<Scalar>(pos) /
                                 std::pow(Scalar{10000}, static_cast<Scalar>(2 * (i / 2)) / static_cast<Scalar>(d));
            pe.set_value_unchecked(pos, i, (i % 2 == 0) ? std::sin(angle) : std::cos(angle));
        }
    return pe;
}

// ── GPTModel (reference compute_layer.hpp:2662-2904) ──────────────────────
// Input: (seq, batch) float token ids. Output: logits (vocab, batch*seq),
// batch-major columns. parameters() order: token_emb, [pos_emb], per block
// {Wq,bq,Wk,bk,Wv,bv,Wo,bo,gamma1,W1,b1,W2,b2,gamma2}, gamma_f, W_lm, b_lm.
class GPTModel final : public Layer
{
public:
    GPTModel(ComputeEngine& engine, std::size_t vocab, std::size_t d_model, std::size_t seq_len, std::size_t heads,
             std::size_t d_ff, std::size_t layers, PosEncodingType pos_enc,
             ActivationType activation = ActivationType::SwiGLU, NormType norm_type = NormType::RMSNorm)
        : vocab_(vocab), d_model_(d_model), seq_len_(seq_len), ln_f_(make_norm_layer(engine, d_model, norm_type)),
          lm_head_(engine, d_model, vocab)
    {
        // Embeddings ~ N(0, 0.02) from mt19937_64{42}, as the reference; the
        // learned position table continues the same generator.
        std::mt19937_64 rng{42};
        std::normal_distribution<Scalar> dist(Scalar{0}, Scalar{0.02f});
        Matrix te(vocab, d_model);
        for (auto& v : te.span())
            v = dist(rng);
        token_emb_ = layer_take_(engine.from_matrix(te));
        grad_token_emb_ = engine.create_tensor(vocab, d_model);
        layer_take_(engine.zero(grad_token_emb_));
        if (pos_enc == PosEncodingType::Learned)
        {
            Matrix pe(seq_len, d_model);
            for (auto& v : pe.span())
                v = dist(rng);
            pos_ = std::make_unique<AdditivePositionEncoder>(engine, std::move(pe), true);
        }
        else if (pos_enc == PosEncodingType::Sinusoidal)
            pos_ = std::make_unique<AdditivePositionEncoder>(engine, sinusoidal_table(seq_len, d_model), false);
        else
            pos_ = std::make_unique<NoPositionEncoder>();
        blocks_.reserve(layers);
        auto step_bias = std::make_shared<StepBiasCache>();
        for (std::size_t i = 0; i < layers; ++i)
        {
            blocks_.push_back(
                std::make_unique<GPTBlock>(engine, d_model, heads, d_ff, seq_len, pos_enc, activation, norm_type));
            blocks_.back()->share_step_bias(step_bias);
        }
    }

    std::vector<TensorRef> parameters() override
    {
        std::vector<TensorRef> p{token_emb_};
        append_refs_(p, pos_->parameters());
        for (auto& b : blocks_)
            append_refs_(p, b->parameters());
        append_refs_(p, ln_f_->parameters(), lm_head_.parameters());
        return p;
    }
    std::vector<TensorRef> param_gradients() override
    {
        std::vector<TensorRef> g{grad_token_emb_};
        append_refs_(g, pos_->param_gradients());
        for (auto& b : blocks_)
            append_refs_(g, b->param_gradients());
        append_refs_(g, ln_f_->param_gradients(), lm_head_.param_gradients());
        return g;
    }
    void set_doc_ids(std::span<const std::size_t> ids) override { doc_ids_.assign(ids.begin(), ids.end()); }
    void set_flush_interval(std::size_t n) override { flush_interval_ = n; }

    Result<Tensor> forward(ComputeEngine& engine, const Tensor& input) override
    {
        const std::size_t seq = input.rows();
        batch_ = input.cols();
        NN_TRY(ids_T, engine.transpose(input));              // (batch, seq): flat order b*seq+t
        NN_TRY(emb, engine.gather_rows(token_emb_, ids_T));  // (N, D)
        NN_TRY(stored, engine.clone(ids_T));
        tokens_ = stored;
        NN_TRY(emb_T, engine.transpose(emb));                // (D, N)
        NN_TRY(x0, pos_->apply(engine, emb_T, batch_, seq));
        Tensor x = x0;
        for (std::size_t bi = 0; bi < blocks_.size(); ++bi)
        {
            blocks_[bi]->set_doc_ids(doc_ids_);
            NN_TRY(y, blocks_[bi]->forward(engine, x));
            x = y;
            if (flush_interval_ > 0 && (bi + 1) % flush_interval_ == 0 && bi + 1 < blocks_.size())
                NN_CHECK(engine.flush_batch());
        }
        NN_TRY(xn, ln_f_->forward(engine, x));
        return lm_head_.forward(engine, xn);
    }

    Result<Tensor> backward(ComputeEngine& engine, const Tensor& grad_output) override
    {
        NN_TRY(g0, lm_head_.backward(engine, grad_output));
        NN_TRY(g1, ln_f_->backward(engine, g0));
        Tensor g = g1;
        const std::size_t n = blocks_.size();
        for (std::size_t bi = 0; bi < n; ++bi)
        {
            NN_TRY(y, blocks_[n - 1 - bi]->backward(engine, g));
            g = y;
            if (flush_interval_ > 0 && (bi + 1) % flush_interval_ == 0 && bi + 1 < n)
                NN_CHECK(engine.flush_batch());
        }
        NN_TRY(gT, engine.transpose(g));   // (N, D)
        NN_CHECK(pos_->backward(engine, gT));
        NN_CHECK(engine.scatter_add_rows(grad_token_emb_, tokens_, gT));
        return engine.from_matrix(Matrix(seq_len_, batch_, Scalar{0}));
    }

    [[nodiscard]] std::size_t vocab_size() const noexcept { return vocab_; }
    [[nodiscard]] std::size_t num_blocks() const noexcept { return blocks_.size(); }
    [[nodiscard]] std::size_t seq_len() const noexcept { return seq_len_; }
    [[nodiscard]] std::size_t d_model() const noexcept { return d_model_; }

    // One token with per-layer KV caches (reference compute_layer.hpp:2906-2950):
    // token_emb[token] (gather + transpose), the position at `pos`, every block's
    // forward_step, the final norm and the LM head. Returns logits (vocab, 1).
    Result<Tensor> forward_step(ComputeEngine& engine, std::size_t token_id, std::size_t pos,
                                std::vector<Tensor>& k_caches, std::vector<Tensor>& v_caches, std::size_t cur_len)
    {
        if (k_caches.size() != blocks_.size() || v_caches.size() != blocks_.size())
            return fail("GPTModel forward_step: one K and one V cache per block required");
        if (cur_len >= seq_len_)
            return fail("GPTModel forward_step: cur_len must be below seq_len (the caches' rows)");
        NN_TRY(id_t, engine.from_matrix(Matrix(1, 1, static_cast<Scalar>(token_id))));
        NN_TRY(emb, engine.gather_rows(token_emb_, id_t));
        NN_TRY(x0, engine.transpose(emb));
        NN_TRY(xp, pos_->apply_step(engine, x0, pos));
        Tensor x = xp;
        for (std::size_t i = 0; i < blocks_.size(); ++i)
        {
            NN_TRY(y, blocks_[i]->forward_step(engine, x, k_caches[i], v_caches[i], cur_len));
            x = y;
            if (flush_interval_ > 0 && (i + 1) % flush_interval_ == 0 && i + 1 < blocks_.size())
                NN_CHECK(engine.flush_batch());
        }
        NN_TRY(ln, ln_f_->forward(engine, x));
        return lm_head_.forward(engine, ln);
    }

    // Sampling with KV caches (reference compute_layer.hpp:2963-3096): the
    // caches are (seq_len, d_model) per block; the prompt (its last seq_len
    // tokens) fills them token by token; each new token is drawn from the last
    // logits (temperature scaling, softmax, inverse-CDF draw from one uniform;
    // temperature 0 = argmax) and fed back; when the caches are full they are
    // zeroed and refilled with the last seq_len - 1 tokens (sliding window).
    // Generation stops after max_new_tokens, or at eos once min_new_tokens are
    // out (eos itself is not returned). The reference seeds its generator from
    // std::random_device; here the caller passes the seed of the same
    // std::mt19937_64 / uniform_real_distribution draw.
    Result<std::vector<std::size_t>> generate(ComputeEngine& engine, const std::vector<std::size_t>& prompt,
                                              std::size_t max_new_tokens, Scalar temperature,
                                              std::size_t eos_token_id, std::size_t min_new_tokens,
                                              std::uint64_t seed)
    {
        if (prompt.empty()) return fail("GPTModel generate: empty prompt");
        std::vector<std::size_t> context(prompt), generated;
        std::mt19937_64 rng{seed};
        std::uniform_real_distribution<Scalar> dist(Scalar{0}, Scalar{1});
        std::vector<Tensor> kc, vc;
        for (std::size_t i = 0; i < blocks_.size(); ++i)
        {
            kc.push_back(engine.create_tensor(seq_len_, d_model_));
            vc.push_back(engine.create_tensor(seq_len_, d_model_));
        }
        std::size_t cur_len = 0;
        Tensor last;
        auto fill = [&](std::size_t start) -> Result<void> {
            for (std::size_t i = start; i < context.size(); ++i)
            {
                NN_TRY(r, forward_step(engine, context[i], cur_len, kc, vc, cur_len));
                last = r;
                ++cur_len;
            }
            return {};
        };
        NN_CHECK(fill(context.size() > seq_len_ ? context.size() - seq_len_ : 0));
        for (std::size_t step = 0; step < max_new_tokens; ++step)
        {
            if (cur_len >= seq_len_)
            {
                for (auto& t : kc) NN_CHECK(engine.zero(t));
                for (auto& t : vc) NN_CHECK(engine.zero(t));
                cur_len = 0;
                const std::size_t keep = seq_len_ - 1;
                NN_CHECK(fill(context.size() > keep ? context.size() - keep : 0));
            }
            NN_TRY(lm, engine.to_matrix(last));
            std::vector<Scalar> p(vocab_);
            for (std::size_t v = 0; v < vocab_; ++v) p[v] = lm.at(v, 0);
            if (temperature > 0 && temperature != Scalar{1})
                for (auto& v : p) v /= temperature;
            Scalar mx = p[0];
            for (std::size_t v = 1; v < vocab_; ++v) mx = std::max(mx, p[v]);
            Scalar sum = 0;
            for (auto& v : p)
            {
                v = std::exp(v - mx);
                sum += v;
            }
            for (auto& v : p) v /= sum;
            std::size_t next = 0;
            if (temperature > 0)
            {
                const Scalar r = dist(rng);
                Scalar cum = 0;
                next = vocab_ - 1;
                for (std::size_t v = 0; v < vocab_; ++v)
                {
                    cum += p[v];
                    if (r <= cum)
                    {
                        next = v;
                        break;
                    }
                }
            }
            else
            {
                Scalar best = p[0];
                for (std::size_t v = 1; v < vocab_; ++v)
                    if (p[v] > best)
                    {
                        best = p[v];
                        next = v;
                    }
            }
            context.push_back(next);
            if (step >= min_new_tokens && next == eos_token_id) break;
            generated.push_back(next);
            NN_CHECK(engine.begin_batch());
            NN_TRY(r, forward_step(engine, next, cur_len, kc, vc, cur_len));
            NN_CHECK(engine.end_batch());
            last = r;
            ++cur_len;
        }
        return generated;
    }

private:
    std::size_t vocab_, d_model_, seq_len_;
    Tensor token_emb_, grad_token_emb_, tokens_;
    std::unique_ptr<PositionEncoder> pos_;
    std::vector<std::unique_ptr<GPTBlock>> blocks_;
    std::unique_ptr<Layer> ln_f_;
    Linear lm_head_;
    std::size_t batch_ = 0;
    std::vector<std::size_t> doc_ids_;
    std::size_t flush_interval_ = 0;
};

} // namespace nn
