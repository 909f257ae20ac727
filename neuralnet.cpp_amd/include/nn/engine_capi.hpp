// engine_capi.hpp — implementation of the flat C-ABI (include/nnhip_engine.h)
// over any nn::ComputeEngine. A library instantiates it once with its
// engine type and symbol prefix via NN_DEFINE_ENGINE_CAPI(prefix, make_engine).
#pragma once

#include <cstring>
#include <iterator>
#include <memory>
#include <optional>
#include <string>
#include <vector>

#include "compute_engine.hpp"
#include "compute_loss.hpp"
#include "compute_optimizer.hpp"
#include "model_file.hpp"
#include "layer_exprs.hpp"
#include "model.hpp"

namespace nn::capi
{

inline std::string& last_error()
{
    static thread_local std::string e;
    return e;
}
inline int set_error(const std::string& m)
{
    last_error() = m;
    return 1;
}

struct EngineHandle
{
    std::unique_ptr<ComputeEngine> eng;
};

inline Tensor* T(void* h) { return static_cast<Tensor*>(h); }
inline const Tensor* T(const void* h) { return static_cast<const Tensor*>(h); }

inline void* new_tensor(Tensor t) { return new Tensor(std::move(t)); }

inline void* tensor_create(EngineHandle* e, std::size_t r, std::size_t c)
{
    return new_tensor(e->eng->create_tensor(r, c));
}

inline void* tensor_from_host(EngineHandle* e, const float* data, std::size_t r, std::size_t c)
{
    Matrix m(r, c);
    if (r * c != 0) std::memcpy(m.data(), data, r * c * sizeof(float));
    auto t = e->eng->from_matrix(m);
    if (!t)
    {
        set_error(t.error().message);
        return nullptr;
    }
    return new_tensor(*t);
}

inline int tensor_to_host(EngineHandle* e, const void* h, float* out)
{
    auto m = e->eng->to_matrix(*T(h));
    if (!m) return set_error(m.error().message);
    if (m->size()) std::memcpy(out, m->data(), m->size() * sizeof(float));
    return 0;
}

inline int tensor_copy_from_host(EngineHandle* e, void* h, const float* data)
{
    Tensor* t = T(h);
    Matrix m(t->rows(), t->cols());
    if (m.size()) std::memcpy(m.data(), data, m.size() * sizeof(float));
    auto r = e->eng->copy_from(*t, m);
    return r ? 0 : set_error(r.error().message);
}

inline void* tensor_data_ptr(const void* h)
{
    const Tensor* t = T(h);
    if (t->is_cpu()) return const_cast<float*>(t->cpu_matrix().data());
    return t->dev_ptr();
}

// The pointer for a raw reader, once the engine has queued what t's values depend on.
inline int tensor_device_ptr(EngineHandle* e, const void* h, void** out)
{
    if (!e || !h || !out) return set_error("tensor_device_ptr: null argument");
    auto r = e->eng->settle_for_read(*T(h));
    if (!r) return set_error(r.error().message);
    *out = tensor_data_ptr(h);
    return 0;
}

inline int engine_op(EngineHandle* e, int op, void* const* in, std::size_t n_in, void** out, std::size_t n_out,
                     const double* a, std::size_t n_args)
{
    ComputeEngine& E = *e->eng;
    auto need = [&](std::size_t ni, std::size_t no, std::size_t na) -> bool {
        if (n_in < ni || n_out < no || n_args < na)
        {
            set_error("engine_op: too few inputs/outputs/args for op " + std::to_string(op));
            return false;
        }
        return true;
    };
    auto in_t = [&](std::size_t i) -> Tensor& { return *T(in[i]); };
    auto flag = [&](std::size_t i) { return a[i] != 0.0; };
    auto sz = [&](std::size_t i) { return static_cast<std::size_t>(a[i]); };
    auto sc = [&](std::size_t i) { return static_cast<Scalar>(a[i]); };
    auto put = [&](std::size_t i, Result<Tensor>& r) -> int {
        if (!r) return set_error(r.error().message);
        out[i] = new_tensor(*r);
        return 0;
    };
    auto done = [&](const Result<void>& r) -> int { return r ? 0 : set_error(r.error().message); };
    auto opt_mask = [&](std::size_t idx) -> const Tensor* { return n_in > idx ? T(in[idx]) : nullptr; };

    switch (op)
    {
    case 1: { if (!need(1, 1, 0)) return 1; auto r = E.clone(in_t(0)); return put(0, r); }
    case 2: { if (!need(1, 1, 2)) return 1; auto r = E.slice_rows(in_t(0), sz(0), sz(1)); return put(0, r); }
    case 3: { if (!need(2, 0, 1)) return 1; return done(E.insert_rows(in_t(0), sz(0), in_t(1))); }
    case 4: { if (!need(2, 1, 0)) return 1; auto r = E.gather_rows(in_t(0), in_t(1)); return put(0, r); }
    case 5: { if (!need(3, 0, 0)) return 1; return done(E.scatter_add_rows(in_t(0), in_t(1), in_t(2))); }
    case 6: { if (!need(1, 1, 4)) return 1; auto r = E.rearrange_3d(in_t(0), sz(0), sz(1), sz(2), flag(3)); return put(0, r); }
    case 7: { if (!need(1, 1, 0)) return 1; auto r = E.transpose(in_t(0)); return put(0, r); }
    case 8: { if (!need(2, 1, 2)) return 1; auto r = E.matmul(in_t(0), in_t(1), flag(0), flag(1)); return put(0, r); }
    case 9: { if (!need(2, 1, 4)) return 1; auto r = E.batched_matmul(in_t(0), in_t(1), sz(0), flag(1), flag(2), sc(3)); return put(0, r); }
    case 10:
    {
        if (!need(2, 1, 6)) return 1;
        auto r = E.batched_matmul_reduce(in_t(0), in_t(1), sz(0), static_cast<ReduceOp>(sz(1)), flag(2), flag(3), sc(4),
                                         flag(5), opt_mask(2));
        return put(0, r);
    }
    case 11:
    {
        if (!need(3, 1, 4)) return 1;
        auto r = E.batched_matmul_softmax_denom(in_t(0), in_t(1), in_t(2), sz(0), flag(1), flag(2), sc(3), opt_mask(3));
        return put(0, r);
    }
    case 12:
    {
        if (!need(5, 1, 4)) return 1;
        auto r = E.batched_matmul_softmax_apply(in_t(0), in_t(1), in_t(2), in_t(3), in_t(4), sz(0), flag(1), flag(2),
                                                sc(3), opt_mask(5));
        return put(0, r);
    }
    case 13:
    {
        if (!need(5, 2, 4)) return 1;
        Tensor R;
        auto r = E.batched_matmul_softmax_backward_q(in_t(0), in_t(1), in_t(2), in_t(3), in_t(4), sz(0), flag(1),
                                                     flag(2), sc(3), R, opt_mask(5));
        if (put(0, r)) return 1;
        out[1] = new_tensor(R);
        return 0;
    }
    case 14:
    {
        if (!need(7, 2, 4)) return 1;
        Tensor gv;
        auto r = E.batched_matmul_softmax_backward_kv(in_t(0), in_t(1), in_t(2), in_t(3), in_t(4), in_t(5), in_t(6),
                                                      sz(0), flag(1), flag(2), sc(3), gv, opt_mask(7));
        if (put(0, r)) return 1;
        out[1] = new_tensor(gv);
        return 0;
    }
    case 15: { if (!need(2, 1, 0)) return 1; auto r = E.col_softmax_denom(in_t(0), in_t(1)); return put(0, r); }
    case 16:
    {
        if (!need(2, 2, 2)) return 1;
        Tensor lv;
        auto r = E.col_softmax_sparse_forward(in_t(0), in_t(1), opt_mask(2), sz(0), sc(1), lv);
        if (put(0, r)) return 1;
        out[1] = new_tensor(lv);
        return 0;
    }
    case 17: { if (!need(2, 0, 0)) return 1; return done(E.add_inplace(in_t(0), in_t(1))); }
    case 18: { if (!need(1, 0, 1)) return 1; return done(E.scale_inplace(in_t(0), sc(0))); }
    case 19: { if (!need(2, 0, 1)) return 1; return done(E.axpy_inplace(in_t(0), sc(0), in_t(1))); }
    case 20: { if (!need(1, 0, 0)) return 1; return done(E.zero(in_t(0))); }
    case 21: { if (!need(1, 1, 0)) return 1; auto r = E.row_reduce_sum(in_t(0)); return put(0, r); }
    case 22: { if (!need(1, 1, 0)) return 1; auto r = E.col_reduce_sum(in_t(0)); return put(0, r); }
    case 23: { if (!need(1, 1, 0)) return 1; auto r = E.row_reduce_max(in_t(0)); return put(0, r); }
    case 24: { if (!need(1, 1, 0)) return 1; auto r = E.col_reduce_max(in_t(0)); return put(0, r); }
    case 25: { if (!need(2, 0, 1)) return 1; return done(E.broadcast_row_inplace(in_t(0), in_t(1), static_cast<BinaryOp>(sz(0)))); }
    case 26: { if (!need(2, 0, 1)) return 1; return done(E.broadcast_col_inplace(in_t(0), in_t(1), static_cast<BinaryOp>(sz(0)))); }
    case 27: { if (!need(1, 1, 1)) return 1; auto r = E.elementwise_unary(static_cast<UnaryOp>(sz(0)), in_t(0)); return put(0, r); }
    case 28: { if (!need(2, 1, 1)) return 1; auto r = E.elementwise_binary(static_cast<BinaryOp>(sz(0)), in_t(0), in_t(1)); return put(0, r); }
    case 29:
    {
        if (!need(1, 1, 3)) return 1;
        auto r = E.elementwise_binary_scalar(static_cast<BinaryOp>(sz(0)), in_t(0), sc(1), flag(2));
        return put(0, r);
    }
    case 30:
    {
        if (!need(2, 1, 3)) return 1;
        auto r = E.elementwise_select_scalar_cond(static_cast<CompareOp>(sz(0)), in_t(0), sc(1), in_t(1), sc(2));
        return put(0, r);
    }
    default:
        return set_error("engine_op: unknown op " + std::to_string(op));
    }
}

inline int eval_expr(EngineHandle* e, const std::uint8_t* instrs, std::size_t n_instrs, const std::uint8_t* vk,
                     const std::uint32_t* vp, std::size_t n_views, const float* consts, std::size_t n_consts,
                     std::uint32_t num_regs, void* const* inputs, std::size_t n_inputs, std::size_t rows,
                     std::size_t cols, int vector_out, void** out)
{
    ExprSpec s;
    for (std::size_t i = 0; i < n_instrs; ++i)
    {
        const std::uint8_t* p = instrs + 8 * i;
        ExprInstr in;
        in.op = p[0];
        in.dst = p[1];
        in.a = {p[2], p[3]};
        in.b = {p[4], p[5]};
        in.c = {p[6], p[7]};
        s.instrs.push_back(in);
    }
    for (std::size_t i = 0; i < n_views; ++i)
        s.views.push_back(ExprView{vk[2 * i], vk[2 * i + 1], vp[i]});
    s.consts.assign(consts, consts + n_consts);
    s.num_regs = num_regs;
    std::vector<Tensor> ins;
    for (std::size_t i = 0; i < n_inputs; ++i)
        ins.push_back(*T(inputs[i]));
    auto r = vector_out ? e->eng->eval_expr_reduce(s, ins, rows, cols) : e->eng->eval_expr(s, ins, rows, cols);
    if (!r) return set_error(r.error().message);
    *out = new_tensor(*r);
    return 0;
}

struct GptConfigC
{
    std::size_t vocab_size, d_model, seq_len, num_heads, d_ff, num_layers;
    std::uint32_t pos_enc;
    float lr, beta1, beta2, eps, weight_decay;
    std::uint32_t activation, norm_type, optimizer;
};

// Optimizer codes of GptConfigC::optimizer, the names create_optimizer takes
// (reference compute_optimizer.hpp:594-615).
constexpr const char* kOptimizerNames[] = {"adamw", "adam", "sgd", "sgd_momentum", "muon"};

// One training session: GPTModel + CrossEntropyLoss + AdamW on one engine,
// issuing the reference train-step sequence (src/text_train.cpp:1181-1330):
// begin_batch, forward, sparse CE (loss download), backward, end_batch,
// begin_batch, AdamW step, zero_grad, end_batch.
struct GptSession
{
    ComputeEngine* eng = nullptr;
    Model model;
    std::vector<TensorRef> params, grads;
    std::unique_ptr<Optimizer> opt;
    std::vector<Tensor> k_cache, v_cache;   // incremental inference, one pair per block
    CrossEntropyLoss ce;
    std::size_t vocab = 0, seq = 0, batch = 0, num_valid = 0;
    Tensor tokens, labels, mask, logits;
    bool has_batch = false, has_mask = false;
    GptConfigC cfg{};
};

// The session's optimizer over its parameters: AdamW with the session's
// betas / eps / weight decay, else create_optimizer by name with lr (and the
// weight decay), as text_train creates it (text_train.cpp:966-969).
inline Result<std::unique_ptr<Optimizer>> make_optimizer(ComputeEngine& eng, const GptConfigC& c,
                                                         std::vector<TensorRef> params, std::vector<TensorRef> grads)
{
    if (c.optimizer == 0)
        return std::unique_ptr<Optimizer>(std::make_unique<AdamW>(eng, std::move(params), std::move(grads), c.lr,
                                                                  c.beta1, c.beta2, c.eps, c.weight_decay));
    if (c.optimizer >= std::size(kOptimizerNames)) return fail("gpt: unknown optimizer code");
    auto o = create_optimizer(kOptimizerNames[c.optimizer], eng, std::move(params), std::move(grads), c.lr,
                              c.weight_decay);
    if (!o) return fail("gpt: unknown optimizer");
    return o;
}

inline int gpt_create(EngineHandle* e, const GptConfigC* c, GptSession** out)
{
    GptConfig cfg;
    cfg.vocab_size = c->vocab_size;
    cfg.d_model = c->d_model;
    cfg.seq_len = c->seq_len;
    cfg.num_heads = c->num_heads;
    cfg.d_ff = c->d_ff;
    cfg.num_layers = c->num_layers;
    cfg.pos_enc = static_cast<PosEncodingType>(c->pos_enc);
    cfg.activation = static_cast<ActivationType>(c->activation);
    cfg.norm_type = static_cast<NormType>(c->norm_type);
    auto m = build_gpt_model(*e->eng, cfg);
    if (!m) return set_error(m.error().message);
    auto s = std::make_unique<GptSession>();
    s->eng = e->eng.get();
    s->model = std::move(*m);
    s->params = s->model.parameters();
    s->grads = s->model.param_gradients();
    auto o = make_optimizer(*s->eng, *c, s->params, s->grads);
    if (!o) return set_error(o.error().message);
    s->opt = std::move(*o);
    s->vocab = c->vocab_size;
    s->cfg = *c;
    if (auto r = s->eng->end_batch(); !r) return set_error(r.error().message);
    *out = s.release();
    return 0;
}

inline int gpt_param_shape(const GptSession* g, std::size_t i, std::size_t* r, std::size_t* c)
{
    if (i >= g->params.size()) return set_error("gpt: parameter index out of range");
    *r = g->params[i].get().rows();
    *c = g->params[i].get().cols();
    return 0;
}

inline int gpt_set_param(GptSession* g, std::size_t i, const float* data)
{
    if (i >= g->params.size()) return set_error("gpt: parameter index out of range");
    Tensor& p = g->params[i].get();
    Matrix m(p.rows(), p.cols());
    std::memcpy(m.data(), data, m.size() * sizeof(float));
    auto r = g->eng->copy_from(p, m);
    return r ? 0 : set_error(r.error().message);
}

inline int gpt_read(GptSession* g, const Tensor& t, float* out)
{
    auto m = g->eng->to_matrix(t);
    if (!m) return set_error(m.error().message);
    std::memcpy(out, m->data(), m->size() * sizeof(float));
    return 0;
}

inline int gpt_set_doc_ids(GptSession* g, const std::uint64_t* ids, std::size_t n)
{
    std::vector<std::size_t> v(ids, ids + n);
    g->model.set_doc_ids(v);
    return 0;
}

inline int gpt_load_batch(GptSession* g, const float* tokens, std::size_t seq, std::size_t batch,
                          const std::uint64_t* labels, const float* loss_mask)
{
    const std::size_t n = seq * batch;
    Matrix tk(seq, batch);
    std::memcpy(tk.data(), tokens, n * sizeof(float));
    auto t = g->eng->from_matrix(tk);
    if (!t) return set_error(t.error().message);
    Matrix lb(1, n);
    std::vector<std::size_t> lab(labels, labels + n);
    for (std::size_t i = 0; i < n; ++i) lb.data()[i] = static_cast<Scalar>(lab[i]);
    auto l = g->eng->from_matrix(lb);
    if (!l) return set_error(l.error().message);
    std::vector<Scalar> mvec;
    g->has_mask = loss_mask != nullptr;
    if (g->has_mask)
    {
        mvec.assign(loss_mask, loss_mask + n);
        Matrix mm(1, n);
        for (std::size_t i = 0; i < n; ++i) mm.data()[i] = loss_mask[i] >= 0.5f ? 1.0f : 0.0f;
        auto mt = g->eng->from_matrix(mm);
        if (!mt) return set_error(mt.error().message);
        g->mask = *mt;
    }
    g->tokens = *t;
    g->labels = *l;
    g->num_valid = CrossEntropyLoss::count_valid(lab, mvec, g->vocab);
    g->seq = seq;
    g->batch = batch;
    g->has_batch = true;
    return 0;
}

// Forward + CE of the loaded batch with the loss left on the device (the
// (1,1) sum of loss_vec); flush_batch submits the work without waiting.
inline int gpt_forward_total(GptSession* g, Tensor& total)
{
    if (!g->has_batch) return set_error("gpt: no batch loaded");
    if (auto r = g->eng->begin_batch(); !r) return set_error(r.error().message);
    auto lg = g->model.forward(g->tokens);
    if (!lg) return set_error(lg.error().message);
    g->logits = *lg;
    auto t = g->ce.forward_sparse_total(*g->eng, g->logits, g->labels, g->has_mask ? &g->mask : nullptr, g->vocab,
                                        g->num_valid);
    if (!t) return set_error(t.error().message);
    total = *t;
    if (auto r = g->eng->flush_batch(); !r) return set_error(r.error().message);
    return 0;
}

inline int gpt_read_loss(GptSession* g, const Tensor& total, float* loss)
{
    auto h = g->eng->to_matrix(total);
    if (!h) return set_error(h.error().message);
    *loss = CrossEntropyLoss::loss_of_total(*h, g->num_valid);
    return 0;
}

inline int gpt_forward_loss(GptSession* g, float* loss)
{
    Tensor total;
    if (int rc = gpt_forward_total(g, total)) return rc;
    return gpt_read_loss(g, total, loss);
}

// Backward of one micro-batch, submitted without waiting. When gradients are
// accumulated over several (src/text_train.cpp:1242-1253) the loss gradient
// is scaled in place by grad_scale (1 / accum_steps there) before the model
// backward, so the accumulated gradients are the mean over the micro-batches.
inline int gpt_backward_queued(GptSession* g, float grad_scale)
{
    auto gr = g->ce.backward();
    if (!gr) return set_error(gr.error().message);
    if (grad_scale != 1.0f)
        if (auto r = g->eng->scale_inplace(*gr, grad_scale); !r) return set_error(r.error().message);
    auto b = g->model.backward(*gr);
    if (!b) return set_error(b.error().message);
    if (auto r = g->eng->flush_batch(); !r) return set_error(r.error().message);
    return 0;
}

inline int gpt_backward_scaled(GptSession* g, float grad_scale)
{
    if (int rc = gpt_backward_queued(g, grad_scale)) return rc;
    if (auto r = g->eng->end_batch(); !r) return set_error(r.error().message);
    return 0;
}

inline int gpt_backward(GptSession* g) { return gpt_backward_scaled(g, 1.0f); }

// Global L2-norm gradient clipping (Optimizer::clip_grad_norm,
// compute_optimizer.hpp:90-140); max_norm <= 0 leaves the gradients alone.
inline int gpt_clip_grad_norm(GptSession* g, float max_norm)
{
    if (auto r = g->opt->clip_grad_norm(max_norm); !r) return set_error(r.error().message);
    return 0;
}

// One iteration of the reference training loop (src/text_train.cpp:1181-1330):
// forward + CE (flush), backward with the loss gradient scaled by
// 1 / accum_steps when accum_steps > 1; then, when do_update,
// clip_grad_norm(max_norm) if max_norm > 0, and begin_batch, AdamW step,
// zero_grad, end_batch. The work is submitted phase by phase and waited for
// once, at the end, where the loss is read: the host records the backward
// and the update while the GPU still runs the forward.
inline int gpt_train_step_ex(GptSession* g, std::size_t accum_steps, float max_norm, int do_update, float* loss)
{
    if (accum_steps == 0) return set_error("gpt: accum_steps must be at least 1");
    Tensor total;
    if (int rc = gpt_forward_total(g, total)) return rc;
    const float scale = accum_steps > 1 ? 1.0f / static_cast<float>(accum_steps) : 1.0f;
    if (int rc = gpt_backward_queued(g, scale)) return rc;
    if (do_update)
    {
        if (max_norm > 0)
            if (int rc = gpt_clip_grad_norm(g, max_norm)) return rc;
        if (auto r = g->eng->begin_batch(); !r) return set_error(r.error().message);
        if (auto r = g->opt->step(); !r) return set_error(r.error().message);
        if (auto r = g->opt->zero_grad(); !r) return set_error(r.error().message);
    }
    if (auto r = g->eng->end_batch(); !r) return set_error(r.error().message);
    return gpt_read_loss(g, total, loss);
}

// The ModelSpec this session's model is built from (model_spec.hpp:58-77).
inline model_file::GptSpec session_spec(const GptSession& g)
{
    model_file::GptSpec s;
    s.d_model = g.cfg.d_model;
    s.num_heads = g.cfg.num_heads;
    s.d_ff = g.cfg.d_ff;
    s.num_layers = g.cfg.num_layers;
    s.vocab_size = g.cfg.vocab_size;
    s.seq_len = g.cfg.seq_len;
    s.pos_encoding = g.cfg.pos_enc;
    s.activation = g.cfg.activation;
    s.norm_type = g.cfg.norm_type;
    return s;
}

// The reference's model file (format v4; model_file.hpp): save_model /
// load_model (model_serialization.hpp:380-503) for this session's GPT.
inline int gpt_save(GptSession* g, const char* path, const char* tokenizer, std::size_t tok_len)
{
    if (!path) return set_error("gpt_save: null path");
    std::vector<Matrix> ms;
    for (auto& p : g->params)
    {
        auto m = g->eng->to_matrix(p.get());
        if (!m) return set_error(m.error().message);
        ms.push_back(std::move(*m));
    }
    auto r = model_file::save(path, session_spec(*g), ms,
                              std::string_view(tokenizer ? tokenizer : "", tokenizer ? tok_len : 0));
    return r ? 0 : set_error(r.error().message);
}

// Loads a model file into this session. The reference builds its model from
// the file's spec and then creates the optimizer (text_train.cpp:940-966);
// a session's model already exists, so the file's spec must describe it field
// for field (a file of another head count, context or position encoding has
// the same matrix shapes but another model), and the AdamW state (moments and
// step count) starts afresh, as a newly created optimizer's does. The type
// check is build_gpt_model_from_spec's (domain_gpt.hpp:87-99). The embedded
// tokenizer's length goes to *tok_len and up to tok_cap of its bytes to
// tok_out (a tokenizer is never longer than the file that holds it).
inline int gpt_load(GptSession* g, const char* path, char* tok_out, std::size_t tok_cap, std::size_t* tok_len)
{
    if (!path) return set_error("gpt_load: null path");
    std::vector<Matrix> ms;
    for (auto& p : g->params) ms.emplace_back(p.get().rows(), p.get().cols());
    std::string tok;
    auto spec = model_file::load(path, ms, tok);
    if (!spec) return set_error(spec.error().message);
    if (spec->type != model_file::kTypeGpt && spec->pos_encoding != model_file::kPosALiBi)
        return set_error("Invalid ModelSpec type for GPT: expected GPT or ALiBi_GPT");
    const model_file::GptSpec want = session_spec(*g);
    const std::pair<const char*, std::pair<std::uint64_t, std::uint64_t>> fields[] = {
        {"d_model", {spec->d_model, want.d_model}},          {"num_heads", {spec->num_heads, want.num_heads}},
        {"d_ff", {spec->d_ff, want.d_ff}},                   {"num_layers", {spec->num_layers, want.num_layers}},
        {"vocab_size", {spec->vocab_size, want.vocab_size}}, {"seq_len", {spec->seq_len, want.seq_len}},
        {"pos_encoding", {spec->pos_encoding, want.pos_encoding}},
        {"activation", {spec->activation, want.activation}}, {"norm_type", {spec->norm_type, want.norm_type}}};
    for (const auto& [key, v] : fields)
        if (v.first != v.second)
            return set_error("gpt_load: the file's " + std::string(key) + " is " + std::to_string(v.first) +
                             ", this session's model has " + std::to_string(v.second));
    for (std::size_t i = 0; i < ms.size(); ++i)
        if (auto r = g->eng->copy_from(g->params[i].get(), ms[i]); !r) return set_error(r.error().message);
    auto o = make_optimizer(*g->eng, g->cfg, g->params, g->grads);
    if (!o) return set_error(o.error().message);
    g->opt = std::move(*o);
    if (auto r = g->eng->end_batch(); !r) return set_error(r.error().message);
    if (tok_len) *tok_len = tok.size();
    if (tok_out && tok_cap) std::memcpy(tok_out, tok.data(), std::min(tok_cap, tok.size()));
    return 0;
}

// ── incremental inference (reference compute_layer.hpp:2906-3096) ─────────
inline GPTModel* gpt_model(GptSession* g) { return dynamic_cast<GPTModel*>(&g->model.layer_at(0)); }

// One token through the model with the session's per-block KV caches
// ((seq_len, d_model) each, created on first use): GPTModel::forward_step.
// logits_out: vocab floats.
inline int gpt_forward_step(GptSession* g, std::uint64_t token, std::size_t pos, std::size_t cur_len,
                            float* logits_out)
{
    GPTModel* m = gpt_model(g);
    if (!m) return set_error("gpt_forward_step: the session holds no GPT model");
    if (token >= m->vocab_size()) return set_error("gpt_forward_step: token id out of range");
    if (pos >= m->seq_len()) return set_error("gpt_forward_step: position out of range");
    if (g->k_cache.size() != m->num_blocks())
    {
        g->k_cache.clear();
        g->v_cache.clear();
        for (std::size_t i = 0; i < m->num_blocks(); ++i)
        {
            g->k_cache.push_back(g->eng->create_tensor(m->seq_len(), m->d_model()));
            g->v_cache.push_back(g->eng->create_tensor(m->seq_len(), m->d_model()));
            if (auto r = g->eng->zero(g->k_cache.back()); !r) return set_error(r.error().message);
            if (auto r = g->eng->zero(g->v_cache.back()); !r) return set_error(r.error().message);
        }
    }
    if (auto r = g->eng->begin_batch(); !r) return set_error(r.error().message);
    auto y = m->forward_step(*g->eng, static_cast<std::size_t>(token), pos, g->k_cache, g->v_cache, cur_len);
    if (!y) return set_error(y.error().message);
    if (auto r = g->eng->end_batch(); !r) return set_error(r.error().message);
    return logits_out ? gpt_read(g, *y, logits_out) : 0;
}

inline int gpt_reset_cache(GptSession* g)
{
    g->k_cache.clear();
    g->v_cache.clear();
    return 0;
}

// GPTModel::generate with the caller's seed; *n_out tokens (at most out_cap are copied).
inline int gpt_generate(GptSession* g, const std::uint64_t* prompt, std::size_t n_prompt, std::size_t max_new,
                        float temperature, std::uint64_t eos, std::size_t min_new, std::uint64_t seed,
                        std::uint64_t* out, std::size_t out_cap, std::size_t* n_out)
{
    GPTModel* m = gpt_model(g);
    if (!m) return set_error("gpt_generate: the session holds no GPT model");
    if (!prompt || n_prompt == 0) return set_error("gpt_generate: empty prompt");
    std::vector<std::size_t> pr(n_prompt);
    for (std::size_t i = 0; i < n_prompt; ++i)
    {
        if (prompt[i] >= m->vocab_size()) return set_error("gpt_generate: prompt token out of range");
        pr[i] = static_cast<std::size_t>(prompt[i]);
    }
    if (auto r = g->eng->begin_batch(); !r) return set_error(r.error().message);
    auto toks = m->generate(*g->eng, pr, max_new, temperature, static_cast<std::size_t>(eos), min_new, seed);
    if (!toks) return set_error(toks.error().message);
    if (auto r = g->eng->end_batch(); !r) return set_error(r.error().message);
    if (n_out) *n_out = toks->size();
    for (std::size_t i = 0; i < toks->size() && i < out_cap && out; ++i) out[i] = (*toks)[i];
    return 0;
}

inline int gpt_step(GptSession* g)
{
    if (auto r = g->eng->begin_batch(); !r) return set_error(r.error().message);
    if (auto r = g->opt->step(); !r) return set_error(r.error().message);
    if (auto r = g->eng->end_batch(); !r) return set_error(r.error().message);
    return 0;
}

inline int gpt_zero_grad(GptSession* g)
{
    if (auto r = g->opt->zero_grad(); !r) return set_error(r.error().message);
    if (auto r = g->eng->end_batch(); !r) return set_error(r.error().message);
    return 0;
}

inline int gpt_train_step(GptSession* g, float* loss) { return gpt_train_step_ex(g, 1, 0.0f, 1, loss); }

// One training batch cut from a token flow, as src/text_train.cpp:1137-1172
// builds it: window b starts at flow offset starts[b] and holds
// win_len = min(seq, n_flow - start) tokens; x[t] = flow[start + t] and
// y[t] = flow[start + t + 1] inside the window, pad_id past it; position t
// takes part in the loss iff t + 1 < win_len. doc_ids (optional; flow_doc
// null leaves them untouched) are flow_doc[start + t] inside the window and
// 0 past it. tokens (seq, batch) column per window; labels, loss_mask and
// doc_ids batch-major (b * seq + t). Returns the participating positions.
inline int window_batch(const std::uint64_t* flow, const std::uint64_t* flow_doc, std::size_t n_flow,
                        const std::uint64_t* starts, std::size_t batch, std::size_t seq, std::uint64_t pad_id,
                        float* tokens, std::uint64_t* labels, float* loss_mask, std::uint64_t* doc_ids,
                        std::size_t* valid)
{
    if (!flow || !starts || !tokens || !labels || !loss_mask || !valid || seq == 0)
        return set_error("window_batch: null argument or seq 0");
    std::size_t n_valid = 0;
    for (std::size_t b = 0; b < batch; ++b)
    {
        if (starts[b] >= n_flow) return set_error("window_batch: window start past the flow");
        const std::size_t pos = starts[b], len = std::min(seq, n_flow - pos);
        for (std::size_t t = 0; t < seq; ++t)
        {
            const std::uint64_t x = t < len ? flow[pos + t] : pad_id;
            const std::uint64_t y = t + 1 < len ? flow[pos + t + 1] : pad_id;
            const bool take = t + 1 < len;
            tokens[t * batch + b] = static_cast<float>(x);
            labels[b * seq + t] = y;
            loss_mask[b * seq + t] = take ? 1.0f : 0.0f;
            n_valid += take ? 1 : 0;
            if (flow_doc && doc_ids) doc_ids[b * seq + t] = t < len ? flow_doc[pos + t] : 0;
        }
    }
    *valid = n_valid;
    return 0;
}

inline int attention_mask(std::size_t batch, std::size_t seq, std::size_t heads, int alibi, const float* slopes,
                          const std::uint64_t* doc_ids, std::size_t n_doc, float* out)
{
    if (n_doc != 0 && n_doc < batch * seq) return set_error("build_attention_mask: doc_ids too small for batch*seq");
    if (!out || (alibi && !slopes) || (n_doc != 0 && !doc_ids))
        return set_error("build_attention_mask: null output, slopes (ALiBi needs one per head) or doc_ids");
    std::vector<Scalar> sl;
    if (alibi) sl.assign(slopes, slopes + heads);
    std::vector<std::size_t> d(doc_ids, doc_ids + n_doc);
    Matrix m = build_attention_mask(batch, seq, heads, alibi != 0, sl, d);
    std::memcpy(out, m.data(), m.size() * sizeof(float));
    return 0;
}

// The programs of layer_exprs.hpp by name (param: RoPE's head dim d_k),
// serialised as eval_expr takes them, with the argument each input slot reads
// (its position in the C++ builder's parameter list). Hosts that build the
// same programs check theirs against these.
inline int layer_program(const char* name, std::uint32_t param, std::uint8_t* instrs, std::size_t* n_instrs,
                         std::uint8_t* vk, std::uint32_t* vp, std::size_t* n_views, float* consts,
                         std::size_t* n_consts, std::uint32_t* num_regs, std::int32_t* slot_args, std::size_t* n_slots)
{
    namespace le = layer_exprs;
    if (!name || !instrs || !n_instrs || !vk || !vp || !n_views || !consts || !n_consts || !num_regs || !slot_args ||
        !n_slots)
        return set_error("layer_program: null argument");
    std::vector<Tensor> a;   // argument i is a placeholder with i + 1 rows
    for (std::size_t i = 0; i < 6; ++i) a.push_back(Tensor::cpu(i + 1, 1));
    const std::string n(name);
    std::optional<std::pair<ExprSpec, std::vector<Tensor>>> r;
    auto take = [&r](const auto& e) { r = dsl::to_expr_spec(e); };
    if (n == "rms_sum_sq") take(le::rms_sum_sq(a[0]));
    else if (n == "rms_normalize") take(le::rms_normalize(a[0], a[1]));
    else if (n == "rms_scale") take(le::rms_scale(a[0], a[1]));
    else if (n == "rms_bwd_colsum") take(le::rms_bwd_colsum(a[0], a[1], a[2]));
    else if (n == "rms_bwd_dx") take(le::rms_bwd_dx(a[0], a[1], a[2], a[3], a[4]));
    else if (n == "rms_bwd_rowsum") take(le::rms_bwd_rowsum(a[0], a[1], a[2]));
    else if (n == "softmax_rows") take(le::softmax_rows(a[0]));
    else if (n == "softmax_rows_backward") take(le::softmax_rows_backward(a[0], a[1]));
    else if (n == "swiglu_grad_gate") take(le::swiglu_grad_gate(a[0], a[1], a[2], a[3]));
    else if (n == "swiglu_grad_up") take(le::swiglu_grad_up(a[0], a[1], a[2]));
    else if (n == "rope_forward") take(le::rope_forward(a[0], a[1], a[2], param));
    else if (n == "rope_backward") take(le::rope_backward(a[0], a[1], a[2], param));
    if (!r) return set_error("layer_program: unknown program " + n);
    const ExprSpec& sp = r->first;
    if (sp.instrs.size() > EXPR_MAX_INSTRS || sp.views.size() > EXPR_MAX_INPUTS || sp.consts.size() > EXPR_MAX_CONSTS)
        return set_error("layer_program: program exceeds the ExprSpec limits");
    for (std::size_t i = 0; i < sp.instrs.size(); ++i)
    {
        const ExprInstr& in = sp.instrs[i];
        const std::uint8_t b[8] = {in.op, in.dst, in.a.kind, in.a.idx, in.b.kind, in.b.idx, in.c.kind, in.c.idx};
        std::memcpy(instrs + 8 * i, b, 8);
    }
    for (std::size_t i = 0; i < sp.views.size(); ++i)
    {
        vk[2 * i] = sp.views[i].kind;
        vk[2 * i + 1] = sp.views[i].negate_first_half;
        vp[i] = sp.views[i].param;
    }
    for (std::size_t i = 0; i < sp.consts.size(); ++i) consts[i] = sp.consts[i];
    for (std::size_t i = 0; i < r->second.size(); ++i) slot_args[i] = static_cast<std::int32_t>(r->second[i].rows()) - 1;
    *n_instrs = sp.instrs.size();
    *n_views = sp.views.size();
    *n_consts = sp.consts.size();
    *num_regs = sp.num_regs;
    *n_slots = r->second.size();
    return 0;
}

} // namespace nn::capi

// Defines every symbol of include/nnhip_engine.h with the given prefix.
// MAKE_ENGINE must be an expression yielding std::unique_ptr<nn::ComputeEngine>
// or returning an error string through `err` (a std::string).
// Libraries are built with hidden visibility; only these entry points are
// exported, so two libraries defining the same inline C++ code (the product
// and the test oracle) never bind to each other's copies in one process.
#define NN_CAPI_EXPORT __attribute__((visibility("default")))
#define NN_CAPI_CAT2(a, b) a##b
#define NN_CAPI_CAT(a, b) NN_CAPI_CAT2(a, b)
#define NN_DEFINE_ENGINE_CAPI(P, MAKE_ENGINE)                                                                       \
    _Pragma("GCC visibility push(default)")                                                                         \
    extern "C" {                                                                                                    \
    const char* NN_CAPI_CAT(P, last_error)(void) { return nn::capi::last_error().c_str(); }                        \
    int NN_CAPI_CAT(P, engine_create)(void** out)                                                                  \
    {                                                                                                               \
        std::string err;                                                                                            \
        std::unique_ptr<nn::ComputeEngine> eng = MAKE_ENGINE;                                                       \
        if (!eng) return nn::capi::set_error(err.empty() ? "engine creation failed" : err);                        \
        *out = new nn::capi::EngineHandle{std::move(eng)};                                                          \
        return 0;                                                                                                   \
    }                                                                                                               \
    void NN_CAPI_CAT(P, engine_destroy)(void* e) { delete static_cast<nn::capi::EngineHandle*>(e); }             \
    int NN_CAPI_CAT(P, engine_sync)(void* e)                                                                       \
    {                                                                                                               \
        auto r = static_cast<nn::capi::EngineHandle*>(e)->eng->end_batch();                                        \
        return r ? 0 : nn::capi::set_error(r.error().message);                                                      \
    }                                                                                                               \
    void* NN_CAPI_CAT(P, tensor_create)(void* e, size_t r, size_t c)                                               \
    {                                                                                                               \
        return nn::capi::tensor_create(static_cast<nn::capi::EngineHandle*>(e), r, c);                             \
    }                                                                                                               \
    void* NN_CAPI_CAT(P, tensor_from_host)(void* e, const float* d, size_t r, size_t c)                            \
    {                                                                                                               \
        return nn::capi::tensor_from_host(static_cast<nn::capi::EngineHandle*>(e), d, r, c);                       \
    }                                                                                                               \
    int NN_CAPI_CAT(P, tensor_to_host)(void* e, const void* t, float* out)                                        \
    {                                                                                                               \
        return nn::capi::tensor_to_host(static_cast<nn::capi::EngineHandle*>(e), t, out);                          \
    }                                                                                                               \
    int NN_CAPI_CAT(P, tensor_copy_from_host)(void* e, void* t, const float* d)                                    \
    {                                                                                                               \
        return nn::capi::tensor_copy_from_host(static_cast<nn::capi::EngineHandle*>(e), t, d);                     \
    }                                                                                                               \
    size_t NN_CAPI_CAT(P, tensor_rows)(const void* t) { return nn::capi::T(t)->rows(); }                          \
    size_t NN_CAPI_CAT(P, tensor_cols)(const void* t) { return nn::capi::T(t)->cols(); }                          \
    void* NN_CAPI_CAT(P, tensor_data_ptr)(const void* t) { return nn::capi::tensor_data_ptr(t); }                 \
    int NN_CAPI_CAT(P, tensor_device_ptr)(void* e, const void* t, void** out)                                      \
    {                                                                                                               \
        return nn::capi::tensor_device_ptr(static_cast<nn::capi::EngineHandle*>(e), t, out);                      \
    }                                                                                                               \
    void NN_CAPI_CAT(P, tensor_release)(void* t) { delete nn::capi::T(t); }                                        \
    int NN_CAPI_CAT(P, engine_op)(void* e, int op, void* const* in, size_t n_in, void** out, size_t n_out,        \
                                  const double* args, size_t n_args)                                                \
    {                                                                                                               \
        return nn::capi::engine_op(static_cast<nn::capi::EngineHandle*>(e), op, in, n_in, out, n_out, args,       \
                                   n_args);                                                                         \
    }                                                                                                               \
    int NN_CAPI_CAT(P, engine_eval_expr)(void* e, const uint8_t* ins, size_t ni, const uint8_t* vk,               \
                                         const uint32_t* vp, size_t nv, const float* cs, size_t nc, uint32_t nr,   \
                                         void* const* inputs, size_t nin, size_t rows, size_t cols, int vec,       \
                                         void** out)                                                                \
    {                                                                                                               \
        return nn::capi::eval_expr(static_cast<nn::capi::EngineHandle*>(e), ins, ni, vk, vp, nv, cs, nc, nr,      \
                                   inputs, nin, rows, cols, vec, out);                                              \
    }                                                                                                               \
    int NN_CAPI_CAT(P, gpt_create)(void* e, const void* cfg, void** out)                                           \
    {                                                                                                               \
        nn::capi::GptSession* s = nullptr;                                                                          \
        int rc = nn::capi::gpt_create(static_cast<nn::capi::EngineHandle*>(e),                                     \
                                      static_cast<const nn::capi::GptConfigC*>(cfg), &s);                          \
        *out = s;                                                                                                   \
        return rc;                                                                                                  \
    }                                                                                                               \
    void NN_CAPI_CAT(P, gpt_destroy)(void* g) { delete static_cast<nn::capi::GptSession*>(g); }                   \
    size_t NN_CAPI_CAT(P, gpt_num_params)(const void* g)                                                           \
    {                                                                                                               \
        return static_cast<const nn::capi::GptSession*>(g)->params.size();                                        \
    }                                                                                                               \
    int NN_CAPI_CAT(P, gpt_param_shape)(const void* g, size_t i, size_t* r, size_t* c)                             \
    {                                                                                                               \
        return nn::capi::gpt_param_shape(static_cast<const nn::capi::GptSession*>(g), i, r, c);                    \
    }                                                                                                               \
    int NN_CAPI_CAT(P, gpt_set_param)(void* g, size_t i, const float* d)                                           \
    {                                                                                                               \
        return nn::capi::gpt_set_param(static_cast<nn::capi::GptSession*>(g), i, d);                               \
    }                                                                                                               \
    int NN_CAPI_CAT(P, gpt_get_param)(void* g, size_t i, float* out)                                               \
    {                                                                                                               \
        auto* s = static_cast<nn::capi::GptSession*>(g);                                                            \
        if (i >= s->params.size()) return nn::capi::set_error("gpt: parameter index out of range");                \
        return nn::capi::gpt_read(s, s->params[i].get(), out);                                                      \
    }                                                                                                               \
    int NN_CAPI_CAT(P, gpt_get_grad)(void* g, size_t i, float* out)                                                \
    {                                                                                                               \
        auto* s = static_cast<nn::capi::GptSession*>(g);                                                            \
        if (i >= s->grads.size()) return nn::capi::set_error("gpt: parameter index out of range");                 \
        return nn::capi::gpt_read(s, s->grads[i].get(), out);                                                       \
    }                                                                                                               \
    int NN_CAPI_CAT(P, gpt_set_doc_ids)(void* g, const uint64_t* ids, size_t n)                                    \
    {                                                                                                               \
        return nn::capi::gpt_set_doc_ids(static_cast<nn::capi::GptSession*>(g), ids, n);                           \
    }                                                                                                               \
    int NN_CAPI_CAT(P, gpt_load_batch)(void* g, const float* tk, size_t seq, size_t batch, const uint64_t* lb,    \
                                       const float* mask)                                                           \
    {                                                                                                               \
        return nn::capi::gpt_load_batch(static_cast<nn::capi::GptSession*>(g), tk, seq, batch, lb, mask);          \
    }                                                                                                               \
    int NN_CAPI_CAT(P, gpt_forward_loss)(void* g, float* loss)                                                     \
    {                                                                                                               \
        return nn::capi::gpt_forward_loss(static_cast<nn::capi::GptSession*>(g), loss);                            \
    }                                                                                                               \
    int NN_CAPI_CAT(P, gpt_logits)(void* g, float* out)                                                            \
    {                                                                                                               \
        auto* s = static_cast<nn::capi::GptSession*>(g);                                                            \
        if (!s->logits.valid()) return nn::capi::set_error("gpt: no forward pass yet");                            \
        return nn::capi::gpt_read(s, s->logits, out);                                                               \
    }                                                                                                               \
    int NN_CAPI_CAT(P, gpt_backward)(void* g) { return nn::capi::gpt_backward(static_cast<nn::capi::GptSession*>(g)); } \
    int NN_CAPI_CAT(P, gpt_optimizer_step)(void* g) { return nn::capi::gpt_step(static_cast<nn::capi::GptSession*>(g)); } \
    int NN_CAPI_CAT(P, gpt_zero_grad)(void* g) { return nn::capi::gpt_zero_grad(static_cast<nn::capi::GptSession*>(g)); } \
    int NN_CAPI_CAT(P, layer_program)(const char* name, uint32_t param, uint8_t* ins, size_t* ni, uint8_t* vk,     \
                                      uint32_t* vp, size_t* nv, float* cs, size_t* nc, uint32_t* nr,               \
                                      int32_t* slot_args, size_t* ns)                                               \
    {                                                                                                               \
        return nn::capi::layer_program(name, param, ins, ni, vk, vp, nv, cs, nc, nr, slot_args, ns);              \
    }                                                                                                               \
    int NN_CAPI_CAT(P, build_attention_mask)(size_t batch, size_t seq, size_t heads, int alibi, const float* slopes, \
                                             const uint64_t* doc_ids, size_t n_doc, float* out)                     \
    {                                                                                                               \
        return nn::capi::attention_mask(batch, seq, heads, alibi, slopes, doc_ids, n_doc, out);                    \
    }                                                                                                               \
    int NN_CAPI_CAT(P, gpt_train_step)(void* g, float* loss)                                                       \
    {                                                                                                               \
        return nn::capi::gpt_train_step(static_cast<nn::capi::GptSession*>(g), loss);                              \
    }                                                                                                               \
    int NN_CAPI_CAT(P, window_batch)(const uint64_t* flow, const uint64_t* flow_doc, size_t n_flow,                 \
                                     const uint64_t* starts, size_t batch, size_t seq, uint64_t pad_id, float* tokens, \
                                     uint64_t* labels, float* loss_mask, uint64_t* doc_ids, size_t* valid)          \
    {                                                                                                               \
        return nn::capi::window_batch(flow, flow_doc, n_flow, starts, batch, seq, pad_id, tokens, labels, loss_mask, \
                                      doc_ids, valid);                                                              \
    }                                                                                                               \
    int NN_CAPI_CAT(P, gpt_save)(void* g, const char* path, const char* tok, size_t tok_len)                      \
    {                                                                                                               \
        return nn::capi::gpt_save(static_cast<nn::capi::GptSession*>(g), path, tok, tok_len);                      \
    }                                                                                                               \
    int NN_CAPI_CAT(P, gpt_load)(void* g, const char* path, char* tok_out, size_t tok_cap, size_t* tok_len)        \
    {                                                                                                               \
        return nn::capi::gpt_load(static_cast<nn::capi::GptSession*>(g), path, tok_out, tok_cap, tok_len);         \
    }                                                                                                               \
    int NN_CAPI_CAT(P, gpt_backward_scaled)(void* g, float s)                                                      \
    {                                                                                                               \
        return nn::capi::gpt_backward_scaled(static_cast<nn::capi::GptSession*>(g), s);                            \
    }                                                                                                               \
    int NN_CAPI_CAT(P, gpt_clip_grad_norm)(void* g, float max_norm)                                                \
    {                                                                                                               \
        return nn::capi::gpt_clip_grad_norm(static_cast<nn::capi::GptSession*>(g), max_norm);                      \
    }                                                                                                               \
    int NN_CAPI_CAT(P, gpt_train_step_ex)(void* g, size_t accum_steps, float max_norm, int do_update, float* loss) \
    {                                                                                                               \
        return nn::capi::gpt_train_step_ex(static_cast<nn::capi::GptSession*>(g), accum_steps, max_norm,            \
                                           do_update, loss);                                                        \
    }                                                                                                               \
    int NN_CAPI_CAT(P, gpt_forward_step)(void* g, uint64_t token, size_t pos, size_t cur_len, float* logits)       \
    {                                                                                                               \
        return nn::capi::gpt_forward_step(static_cast<nn::capi::GptSession*>(g), token, pos, cur_len, logits);     \
    }                                                                                                               \
    int NN_CAPI_CAT(P, gpt_reset_cache)(void* g) { return nn::capi::gpt_reset_cache(static_cast<nn::capi::GptSession*>(g)); } \
    int NN_CAPI_CAT(P, gpt_generate)(void* g, const uint64_t* prompt, size_t n_prompt, size_t max_new,             \
                                     float temperature, uint64_t eos, size_t min_new, uint64_t seed, uint64_t* out,  \
                                     size_t out_cap, size_t* n_out)                                                 \
    {                                                                                                               \
        return nn::capi::gpt_generate(static_cast<nn::capi::GptSession*>(g), prompt, n_prompt, max_new,            \
                                      temperature, eos, min_new, seed, out, out_cap, n_out);                        \
    }                                                                                                               \
    }                                                                                                               \
    _Pragma("GCC visibility pop")
