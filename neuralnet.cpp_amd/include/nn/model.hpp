// model.hpp — layer container and GPT construction.
//
// Model follows include/neuralnet.cpp/model_container.hpp:31-188 (ordered
// layers, forward in order, backward in reverse, concatenated parameters);
// GptConfig / build_gpt_model follow include/neuralnet.cpp/domain_gpt.hpp:32-63:
// GeLU or SwiGLU feed-forward, LayerNorm or RMSNorm, learned / sinusoidal /
// ALiBi / RoPE positions.
#pragma once

#include <memory>
#include <vector>

#include "compute_layer.hpp"

namespace nn
{

class Model
{
public:
    Model() = default;
    explicit Model(ComputeEngine& engine) : engine_(&engine) {}
    Model(Model&&) noexcept = default;
    Model& operator=(Model&&) noexcept = default;

    Model& add_layer(std::unique_ptr<Layer> layer)
    {
        layers_.push_back(std::move(layer));
        return *this;
    }
    [[nodiscard]] std::size_t num_layers() const noexcept { return layers_.size(); }
    [[nodiscard]] Layer& layer_at(std::size_t i) { return *layers_.at(i); }
    [[nodiscard]] ComputeEngine& engine() const { return *engine_; }

    void set_flush_interval(std::size_t n)
    {
        for (auto& l : layers_) l->set_flush_interval(n);
    }
    void set_doc_ids(std::span<const std::size_t> ids)
    {
        for (auto& l : layers_) l->set_doc_ids(ids);
    }

    Result<Tensor> forward(const Tensor& input)
    {
        if (layers_.empty()) return fail("Model::forward: no layers");
        if (!engine_) return fail("Model::forward: engine not bound");
        Tensor x = input;
        for (auto& l : layers_)
        {
            NN_TRY(y, l->forward(*engine_, x));
            x = y;
        }
        return x;
    }
    Result<Tensor> backward(const Tensor& grad_output)
    {
        if (layers_.empty()) return fail("Model::backward: no layers");
        if (!engine_) return fail("Model::backward: engine not bound");
        Tensor g = grad_output;
        for (std::size_t i = layers_.size(); i-- > 0;)
        {
            NN_TRY(y, layers_[i]->backward(*engine_, g));
            g = y;
        }
        return g;
    }
    std::vector<TensorRef> parameters()
    {
        std::vector<TensorRef> p;
        for (auto& l : layers_) append_refs_(p, l->parameters());
        return p;
    }
    std::vector<TensorRef> param_gradients()
    {
        std::vector<TensorRef> g;
        for (auto& l : layers_) append_refs_(g, l->param_gradients());
        return g;
    }
    Result<void> zero_grad()
    {
        for (auto& l : layers_) NN_CHECK(l->zero_grad(*engine_));
        return {};
    }

private:
    ComputeEngine* engine_ = nullptr;
    std::vector<std::unique_ptr<Layer>> layers_;
};

struct GptConfig
{
    std::size_t vocab_size = 1024;
    std::size_t d_model = 128;
    std::size_t seq_len = 128;
    std::size_t num_heads = 4;
    std::size_t d_ff = 512;
    std::size_t num_layers = 2;
    PosEncodingType pos_enc = PosEncodingType::Learned;
    ActivationType activation = ActivationType::SwiGLU;
    NormType norm_type = NormType::RMSNorm;
};

[[nodiscard]] inline Result<Model> build_gpt_model(ComputeEngine& engine, const GptConfig& c)
{
    if (c.d_model == 0 || c.num_heads == 0 || c.seq_len == 0 || c.vocab_size == 0)
        return fail("GPT model parameters must be positive");
    if (c.d_ff == 0 || c.num_layers == 0)
        return fail("GPT d_ff and num_layers must be positive");
    if (c.d_model % c.num_heads != 0)
        return fail("GPT d_model must be divisible by num_heads");
    if (c.activation != ActivationType::SwiGLU && c.activation != ActivationType::GeLU)
        return fail("build_gpt_model: activation must be GeLU or SwiGLU");
    if (c.norm_type != NormType::RMSNorm && c.norm_type != NormType::LayerNorm)
        return fail("build_gpt_model: norm must be LayerNorm or RMSNorm");
    if (static_cast<std::uint32_t>(c.pos_enc) > static_cast<std::uint32_t>(PosEncodingType::RoPE))
        return fail("build_gpt_model: unknown position encoding");
    if (c.pos_enc == PosEncodingType::RoPE && (c.d_model / c.num_heads) % 2 != 0)
        return fail("build_gpt_model: RoPE needs an even head dimension");
    Model m(engine);
    m.add_layer(std::make_unique<GPTModel>(engine, c.vocab_size, c.d_model, c.seq_len, c.num_heads, c.d_ff,
                                           c.num_layers, c.pos_enc, c.activation, c.norm_type));
    return m;
}

} // namespace nn
