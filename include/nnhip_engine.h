/* nnhip_engine.h — C-ABI of the HIP compute engine, for FFI hosts.
 *
 * The reference's boundary is the C++ virtual interface nn::ComputeEngine
 * (/root/reference/include/neuralnet.cpp/compute_engine.hpp:87-410); its Python
 * front end (gui.py, cli_controllers.py) drives compiled binaries only, so it
 * has no FFI binding of its own. This header flattens the engine for
 * ctypes/cgo-style hosts: opaque engine and tensor handles, one dispatcher
 * for the op-level primitives (op codes below, each naming the
 * ComputeEngine method it forwards to), eval_expr over a serialised
 * ExprSpec, and a GPT training session that runs the reference's
 * GPTModel + CrossEntropyLoss::forward_sparse + AdamW step
 * (/root/reference/src/text_train.cpp:1181-1330) on the engine.
 *
 * Conventions (same as the kernel ABI in nnhip_kernels.h):
 *   - every int-returning call returns 0 on success, non-zero on error, and
 *     the message is available from nnhip_last_error() (thread-local);
 *   - tensors are row-major float32; index tensors hold integers as floats;
 *   - handles are never shared between threads; one engine owns one HIP stream.
 *
 * libnnhip.so exports these symbols with the prefix `nnhip_`. The CPU
 * restatement used as the test oracle exports the identical set with the
 * prefix `nnoracle_` (tests only; it is not part of the product).
 */
#ifndef NNHIP_ENGINE_H
#define NNHIP_ENGINE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct nnhip_engine nnhip_engine;
typedef struct nnhip_tensor nnhip_tensor;
typedef struct nnhip_gpt nnhip_gpt;

/* Op codes of nnhip_engine_op. in[] / out[] / args[] per op:              */
enum nnhip_op {
    NNHIP_OP_CLONE = 1,            /* in A                 out C              compute_engine.hpp:131 */
    NNHIP_OP_SLICE_ROWS = 2,       /* in A; args start,count  out C           :136-137 */
    NNHIP_OP_INSERT_ROWS = 3,      /* in dst,src; args start (in place)        :142-143 */
    NNHIP_OP_GATHER_ROWS = 4,      /* in table,idx         out C              :151-152 */
    NNHIP_OP_SCATTER_ADD_ROWS = 5, /* in dst,idx,grad (in place)               :160-161 */
    NNHIP_OP_REARRANGE_3D = 6,     /* in X; args M,B,N,inverse  out C          :170-172 */
    NNHIP_OP_TRANSPOSE = 7,        /* in A                 out C              :175 */
    NNHIP_OP_MATMUL = 8,           /* in A,B; args tA,tB   out C              :182-184 */
    NNHIP_OP_BATCHED_MATMUL = 9,   /* in A,B; args batch,tA,tB,alpha  out C   :195-199 */
    NNHIP_OP_BMM_REDUCE = 10,      /* in A,B[,mask]; args batch,op,tA,tB,alpha,reduce_cols  out C  :217-221 */
    NNHIP_OP_BMM_DENOM = 11,       /* in A,B,m[,mask]; args batch,tA,tB,alpha  out l  :226-229 */
    NNHIP_OP_BMM_APPLY = 12,       /* in A,B,V,m,l[,mask]; args batch,tA,tB,alpha  out O  :236-240 */
    NNHIP_OP_BMM_BWD_Q = 13,       /* in A,B,P,m,l[,mask]; args batch,tA,tB,alpha  out dQ,R  :264-268 */
    NNHIP_OP_BMM_BWD_KV = 14,      /* in A,B,P,G,R,m,l[,mask]; args batch,tA,tB,alpha  out dK,dV  :271-276 */
    NNHIP_OP_COL_SOFTMAX_DENOM = 15,  /* in L,colmax  out denom               :289-290 */
    NNHIP_OP_COL_SOFTMAX_SPARSE = 16, /* in L,labels[,mask]; args vocab,inv  out grad,loss_vec  :301-303 */
    NNHIP_OP_ADD_INPLACE = 17,     /* in A,B                                   :306 */
    NNHIP_OP_SCALE_INPLACE = 18,   /* in A; args s                             :309 */
    NNHIP_OP_AXPY_INPLACE = 19,    /* in A,B; args s                           :313 */
    NNHIP_OP_ZERO = 20,            /* in A                                     :316 */
    NNHIP_OP_ROW_REDUCE_SUM = 21,  /* in A  out (rows,1)                       :324 */
    NNHIP_OP_COL_REDUCE_SUM = 22,  /* in A  out (1,cols)                       :328 */
    NNHIP_OP_ROW_REDUCE_MAX = 23,  /*                                          :332 */
    NNHIP_OP_COL_REDUCE_MAX = 24,  /*                                          :336 */
    NNHIP_OP_BROADCAST_ROW = 25,   /* in A,v; args op (in place)               :344-346 */
    NNHIP_OP_BROADCAST_COL = 26,   /* in A,v; args op (in place)               :349-350 */
    NNHIP_OP_UNARY = 27,           /* in A; args op         out C              :357-358 */
    NNHIP_OP_BINARY = 28,          /* in A,B; args op       out C              :361-362 */
    NNHIP_OP_BINARY_SCALAR = 29,   /* in A; args op,s,scalar_first  out C      :366-367 */
    NNHIP_OP_SELECT_SCALAR_COND = 30 /* in A,then; args cmp,scalar_b,scalar_else  out C  :376-378 */
};

const char* nnhip_last_error(void);

/* Engine on the current HIP device (its own stream, its own caching pool). */
int nnhip_engine_create(nnhip_engine** out);
/* Engine selection as the reference's cli::create_engine (include/neuralnet.cpp/cli/engine_factory.hpp:45-88)
 * with a use_hip flag first in priority (HIP > CUDA > Vulkan > CPU): the requested backend, or an error
 * and *out = NULL, never a fallback to another engine. This library holds the HIP engine only, so a CUDA or
 * Vulkan request, or none (the reference's CpuEngine), is an error naming the engine to use. verbose: one
 * line on stderr naming the engine. */
int nnhip_engine_select(int use_hip, int use_cuda, int use_gpu, int verbose, nnhip_engine** out);
void nnhip_engine_destroy(nnhip_engine* e);
int nnhip_engine_sync(nnhip_engine* e);   /* end_batch: waits for all queued work */

nnhip_tensor* nnhip_tensor_create(nnhip_engine* e, size_t rows, size_t cols);   /* uninitialised */
nnhip_tensor* nnhip_tensor_from_host(nnhip_engine* e, const float* data, size_t rows, size_t cols);
int nnhip_tensor_to_host(nnhip_engine* e, const nnhip_tensor* t, float* out);   /* rows*cols floats */
int nnhip_tensor_copy_from_host(nnhip_engine* e, nnhip_tensor* t, const float* data);
size_t nnhip_tensor_rows(const nnhip_tensor* t);
size_t nnhip_tensor_cols(const nnhip_tensor* t);
/* Device pointer (host pointer for the CPU oracle), as it is: results of deferred calls may not be queued
 * yet, and the materialised attention's probability tensor holds score blocks until it is read through the
 * engine. A raw reader takes nnhip_tensor_device_ptr below instead. */
void* nnhip_tensor_data_ptr(const nnhip_tensor* t);
void nnhip_tensor_release(nnhip_tensor* t);

/* One ComputeEngine primitive; new tensors are returned in out[] and must be released. */
int nnhip_engine_op(nnhip_engine* e, int op, nnhip_tensor* const* in, size_t n_in, nnhip_tensor** out,
                    size_t n_out, const double* args, size_t n_args);

/* eval_expr / eval_expr_reduce (compute_engine.hpp:392-409) on a serialised ExprSpec:
 *   instrs: 8 bytes per instruction {op, dst, a.kind, a.idx, b.kind, b.idx, c.kind, c.idx}
 *   views:  n_views records {kind, negate_first_half} in view_kinds[2*i..] and param in view_params[i]. */
int nnhip_engine_eval_expr(nnhip_engine* e, const uint8_t* instrs, size_t n_instrs, const uint8_t* view_kinds,
                           const uint32_t* view_params, size_t n_views, const float* consts, size_t n_consts,
                           uint32_t num_regs, nnhip_tensor* const* inputs, size_t n_inputs, size_t rows, size_t cols,
                           int vector_out, nnhip_tensor** out);

/* The ExprSpec programs the GPT layers issue (include/nn/layer_exprs.hpp; reference compute_layer.hpp
 * RMSNorm :733-795, SwiGLU backward :436-444, Softmax :840-860, RoPE :884-984), which HipEngine recognises
 * structurally and runs as fused kernels, serialised as nnhip_engine_eval_expr takes them, so a host that
 * builds the same programs can check that its copies match. name: rms_sum_sq, rms_normalize, rms_scale,
 * rms_bwd_colsum, rms_bwd_dx, rms_bwd_rowsum, softmax_rows, softmax_rows_backward, swiglu_grad_gate,
 * swiglu_grad_up, rope_forward, rope_backward (param: d_k). Capacities: instrs 8*64 bytes, view_kinds 2*8,
 * view_params 8, consts 16, slot_args 8; slot_args[i] is the builder argument input slot i reads.
 * Host-only. */
int nnhip_layer_program(const char* name, uint32_t param, uint8_t* instrs, size_t* n_instrs, uint8_t* view_kinds,
                        uint32_t* view_params, size_t* n_views, float* consts, size_t* n_consts, uint32_t* num_regs,
                        int32_t* slot_args, size_t* n_slots);

/* build_attention_mask (compute_layer.hpp:2081-2128): writes the (batch*heads*seq, seq) mask.
 * slopes: heads floats when alibi != 0; doc_ids: batch*seq ids or n_doc = 0. Host-only, no device use. */
int nnhip_build_attention_mask(size_t batch, size_t seq, size_t heads, int alibi, const float* slopes,
                               const uint64_t* doc_ids, size_t n_doc, float* out);

/* One training batch cut from a token flow (src/text_train.cpp:1137-1172). Window b starts at
 * starts[b] < n_flow and holds win_len = min(seq, n_flow - starts[b]) tokens: x[t] = flow[start+t],
 * y[t] = flow[start+t+1] inside it, pad_id past it; position t is in the loss iff t+1 < win_len.
 * tokens (seq, batch) column per window; labels, loss_mask, doc_ids batch-major (b*seq + t);
 * doc_ids = flow_doc[start+t] inside the window, 0 past it (skipped when flow_doc or doc_ids is
 * NULL). *valid = positions in the loss. Host-only, no device use. */
int nnhip_window_batch(const uint64_t* flow, const uint64_t* flow_doc, size_t n_flow, const uint64_t* starts,
                       size_t batch, size_t seq, uint64_t pad_id, float* tokens, uint64_t* labels, float* loss_mask,
                       uint64_t* doc_ids, size_t* valid);

/* GPT training session (GPTModel + sparse CE + an optimizer; compute_layer.hpp:2662-3096, domain_gpt.hpp:48-63). */
typedef struct nnhip_gpt_config {
    size_t vocab_size, d_model, seq_len, num_heads, d_ff, num_layers;
    uint32_t pos_enc; /* 0 learned, 1 sinusoidal, 2 ALiBi, 3 RoPE (model_spec.hpp:24-30) */
    float lr, beta1, beta2, eps, weight_decay;   /* beta1 / beta2 / eps: AdamW only */
    uint32_t activation;  /* 0 QuickGeLU, 1 SwiGLU (model_spec.hpp:33-37) */
    uint32_t norm_type;   /* 0 LayerNorm, 1 RMSNorm (model_spec.hpp:40-45) */
    uint32_t optimizer;   /* 0 adamw, 1 adam, 2 sgd, 3 sgd_momentum, 4 muon (compute_optimizer.hpp:594-615) */
} nnhip_gpt_config;

int nnhip_gpt_create(nnhip_engine* e, const nnhip_gpt_config* cfg, nnhip_gpt** out);
void nnhip_gpt_destroy(nnhip_gpt* g);
size_t nnhip_gpt_num_params(const nnhip_gpt* g);   /* parameter tensors, parameters() order */
int nnhip_gpt_param_shape(const nnhip_gpt* g, size_t i, size_t* rows, size_t* cols);
int nnhip_gpt_set_param(nnhip_gpt* g, size_t i, const float* data);
int nnhip_gpt_get_param(nnhip_gpt* g, size_t i, float* out);
int nnhip_gpt_get_grad(nnhip_gpt* g, size_t i, float* out);
/* Per-token document ids, batch-major (b*seq + t), n = batch*seq; n = 0 clears. */
int nnhip_gpt_set_doc_ids(nnhip_gpt* g, const uint64_t* ids, size_t n);
/* Upload one batch: tokens (seq, batch) column per sequence, labels (batch*seq) batch-major,
 * loss_mask optional (NULL = all valid). The batch stays resident until replaced. */
int nnhip_gpt_load_batch(nnhip_gpt* g, const float* tokens, size_t seq, size_t batch, const uint64_t* labels,
                         const float* loss_mask);
int nnhip_gpt_forward_loss(nnhip_gpt* g, float* loss_out);   /* forward + sparse CE on the resident batch */
int nnhip_gpt_logits(nnhip_gpt* g, float* out);              /* (vocab, batch*seq) of the last forward */
int nnhip_gpt_backward(nnhip_gpt* g);
int nnhip_gpt_optimizer_step(nnhip_gpt* g);                  /* the session's optimizer (cfg.optimizer) */
int nnhip_gpt_zero_grad(nnhip_gpt* g);
/* forward + CE + backward + AdamW + zero_grad on the resident batch. */
int nnhip_gpt_train_step(nnhip_gpt* g, float* loss_out);
/* The reference's model file, format v4 ("NNNN": header, ModelSpec record, parameter matrices
 * in parameters() order, embedded tokenizer; model_serialization.hpp:36-52,380-503).
 * _save writes the session's parameters (tokenizer may be NULL with tok_len 0); _load reads a
 * file whose matrices match this session's shapes, *tok_len = embedded tokenizer length and up
 * to tok_cap of its bytes are copied to tok_out. */
int nnhip_gpt_save(nnhip_gpt* g, const char* path, const char* tokenizer, size_t tok_len);
int nnhip_gpt_load(nnhip_gpt* g, const char* path, char* tok_out, size_t tok_cap, size_t* tok_len);
/* Backward with the loss gradient scaled in place by grad_scale first: one micro-batch of
 * gradient accumulation, 1 / accum_steps in src/text_train.cpp:1242-1253. */
int nnhip_gpt_backward_scaled(nnhip_gpt* g, float grad_scale);
/* Optimizer::clip_grad_norm (compute_optimizer.hpp:90-140): scales every gradient by
 * max_norm / ||g||_2 when the global norm exceeds max_norm; max_norm <= 0 does nothing. */
int nnhip_gpt_clip_grad_norm(nnhip_gpt* g, float max_norm);
/* One iteration of the reference training loop (src/text_train.cpp:1181-1330): forward + CE,
 * backward scaled by 1 / accum_steps (accum_steps >= 1); when do_update != 0 also
 * clip_grad_norm(max_norm) if max_norm > 0, AdamW step and zero_grad. */
int nnhip_gpt_train_step_ex(nnhip_gpt* g, size_t accum_steps, float max_norm, int do_update, float* loss_out);
/* Incremental inference with KV caches (GPTModel::forward_step / generate, compute_layer.hpp:2906-3096).
 * _forward_step runs one token (id `token` at position `pos`) through the model with the session's
 * per-block K / V caches ((seq_len, d_model) each, created on first use), writing cache row cur_len and
 * attending over rows [0, cur_len]; logits_out (vocab floats) may be NULL. _reset_cache drops the caches.
 * _generate fills fresh caches from the prompt (its last seq_len tokens), then samples up to max_new
 * tokens (temperature 0: argmax; else softmax(logits / temperature) and one uniform draw of
 * std::mt19937_64(seed) per token; caches refilled with the last seq_len - 1 tokens when full) and stops
 * early at eos once min_new tokens are out; *n_out = tokens generated, up to out_cap copied to out. The
 * reference seeds its generator from std::random_device; the seed argument makes runs repeatable. */
int nnhip_gpt_forward_step(nnhip_gpt* g, uint64_t token, size_t pos, size_t cur_len, float* logits_out);
int nnhip_gpt_reset_cache(nnhip_gpt* g);
int nnhip_gpt_generate(nnhip_gpt* g, const uint64_t* prompt, size_t n_prompt, size_t max_new, float temperature,
                       uint64_t eos, size_t min_new, uint64_t seed, uint64_t* out, size_t out_cap, size_t* n_out);

/* Measurement hooks (no reference counterpart). While enabled, every GEMM launch of the
 * engine is bracketed by HIP events on the engine's stream; _read waits for the stream and
 * returns launches, algorithmic FLOPs (2*M*N*K per batch) and summed kernel milliseconds,
 * then clears the record. nnhip_engine_stream returns the engine's hipStream_t. */
int nnhip_engine_profile_gemm(nnhip_engine* e, int enable);
int nnhip_engine_profile_gemm_read(nnhip_engine* e, double* launches, double* flops, double* ms);
/* Per-launch records {M, N, K, batch, transA, transB, ms} (7 doubles each) of the profiled GEMMs,
 * at most max; returns the number written (-1 on error) and clears the record. */
long nnhip_engine_profile_gemm_records(nnhip_engine* e, double* out, size_t max);
void* nnhip_engine_stream(nnhip_engine* e);
/* Bytes of attention score blocks that the two-pass chain's recorded forward outputs may hold for their
 * backward (default 1/8 of the device memory free when the engine was created, at most 8 GiB); 0 keeps
 * none, and every backward forms its scores again. The blocks only save work: results are the same
 * either way, and an allocation that fails leaves them out. No reference counterpart. */
int nnhip_engine_set_score_budget(nnhip_engine* e, size_t bytes);
/* The device pointer of t for a raw reader (an FFI host handing it to its own kernels): everything t's
 * values depend on is queued first, as a read through the engine would (the deferred producers; for the
 * materialised attention's probability tensor, which holds the forward's score blocks across
 * flush_batch, the probabilities), without waiting; t holds its values once nnhip_engine_stream reaches
 * this point (nnhip_engine_sync, or work ordered after it on that stream). 0 or an error code. No
 * reference counterpart (the reference's host reads go through to_matrix, compute_engine.hpp). */
int nnhip_tensor_device_ptr(nnhip_engine* e, const nnhip_tensor* t, void** out);
/* Launches every deferred attention call (HipEngine defers the reference's two-pass attention chains
 * and runs each as one fused launch) whose results are still referenced, without waiting. */
int nnhip_engine_settle(nnhip_engine* e);

#ifdef __cplusplus
}
#endif

#endif /* NNHIP_ENGINE_H */
