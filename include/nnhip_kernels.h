/* nnhip_kernels.h — C-ABI of the gfx950 kernel library (libnnhip.so).
 *
 * Plays the role of the reference's CUDA kernel ABI
 * (/root/reference/cuda/cuda_kernels.h:15-169): flat extern "C" entry points,
 * plain device pointers and sizes, op codes as unsigned, scalars as float, a
 * HIP stream as void* (NULL = default stream), return 0 on success or a
 * hipError_t / negative status. Entry points marked "no CUDA counterpart"
 * cover primitives the CUDA engine leaves unimplemented
 * (/root/reference/include/neuralnet.cpp/cuda_engine.hpp:212-260,461-469);
 * their semantics are those of the CPU engine at the cited lines of
 * /root/reference/include/neuralnet.cpp/cpu_engine.hpp.
 *
 * All tensors are row-major float32 in device memory. Index tensors hold
 * integers as floats (exact up to 2^24). Nothing here allocates device
 * memory: entry points that need scratch take a workspace pointer whose size
 * comes from the matching *_workspace_bytes function.
 */
#ifndef NNHIP_KERNELS_H
#define NNHIP_KERNELS_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif
#if defined(__GNUC__)
#pragma GCC visibility push(default) /* the library is built with hidden visibility */
#endif

/* ── GEMM (fp32 MFMA) ────────────────────────────────────────────────────
 * C (M,N) = alpha * op(A) op(B); A stored (A_rows, A_cols), B stored (B_rows, B_cols).
 * Replaces cuda_matmul / cuda_matmul_with_handle (cuda_kernels.h:24-43). */
int nnhip_matmul(const float* A, const float* B, float* C, size_t A_rows, size_t A_cols, size_t B_rows,
                 size_t B_cols, int transA, int transB, void* stream);

/* General form used by the engine: per batch b, C_b = alpha * op(A_b) op(B_b). With a workspace of
 * nnhip_gemm_workspace_bytes(M, N, K, batch) bytes, output grids too small to fill the GPU split K
 * over workgroups and sum the partial tiles in slice order (deterministic); with workspace NULL the
 * product is computed without splitting. */
size_t nnhip_gemm_workspace_bytes(size_t M, size_t N, size_t K, size_t batch);
int nnhip_gemm(const float* A, const float* B, float* C, size_t A_rows, size_t A_cols, size_t B_rows, size_t B_cols,
               size_t batch, int transA, int transB, float alpha, void* workspace, size_t workspace_bytes,
               void* stream);

/* A Linear output in the attention heads' layout: out (B*M, T) = rearrange_3d(W X (+ row_bias), M, B, T)
 * (compute_layer.hpp AttentionBase::forward's q / k / v projections and head split), i.e. per batch b
 * out[b*M + m][t] = sum_k W[m][k] X[k][b*T + t] (+ row_bias[m]); W (M, K), X (K, B*T). The sums are
 * those of the product then the rearrange when that product is not split over K (K < 1024 for these
 * shapes). No CUDA counterpart. */
int nnhip_gemm_heads(const float* W, const float* X, const float* row_bias, float* out, size_t M, size_t K, size_t B,
                     size_t T, void* stream);

/* nnhip_gemm_heads with W stored (K, M) when transW (out_b = W^T X_b): the attention's output projection
 * backward, grad_concat = matmul(W_o, G, true, false) (compute_layer.hpp:179 in Linear::backward), followed
 * by its head split rearrange_3d(grad_concat, H d_k, B, T) (:1281-1291), written in the heads' layout
 * directly. No CUDA counterpart. */
int nnhip_gemm_heads_ex(const float* W, const float* X, const float* row_bias, float* out, size_t M, size_t K,
                        size_t B, size_t T, int transW, void* stream);

/* Up to three such products of one X in one launch (the q, k and v projections): out[i] as
 * nnhip_gemm_heads(W[i], X, row_bias ? row_bias[i] : NULL, out[i], ...); count in 1..3, count * B <= 65535,
 * row_bias may be NULL (no bias) or hold NULL entries. No CUDA counterpart. */
int nnhip_gemm_heads_group(const float* const* W, const float* X, const float* const* row_bias, float* const* out,
                           size_t count, size_t M, size_t K, size_t B, size_t T, void* stream);

/* An operand stored by sequence, as the attention's heads' layout stores a (rows, B * T) matrix: its
 * contiguous index c (k of an untransposed A, n of an untransposed B, k of a transposed B) lies at
 * (c / len) * step + c % len and its rows len apart; len a multiple of 16 (of 128 for an untransposed B),
 * step a multiple of 4 and >= len. The attention's rearrange_3d(x, H d_k, B, T, inverse) of such rows
 * (compute_layer.hpp:1256-1259, :1377-1386) is then read in place: len = T, step = H d_k T. len 0: an
 * ordinary operand. */
typedef struct nnhip_by_seq
{
    size_t len, step;
} nnhip_by_seq;

/* C_i (M, N) = [C_i +] A_i op(B), i < count (1..4): products sharing B in one launch, split-K over all of
 * them and one reduction; A_i stored (M, K), B (K, N) or (N, K) with transB, every C_i 16-byte aligned and
 * M*N % 4 == 0. The attention's q, k and v Linear backward each add G_i X^T into its weight gradient with
 * the same input X (compute_layer.hpp Linear::backward: grad_w += matmul(G, X, false, true)); this runs the
 * three accumulations together. row_sums (may be NULL): row_sums[i] (M) = [row_sums[i] +] the row sums of
 * A_i over k (Linear::backward's grad_b += row_reduce_sum(G), G being A_i), computed from the A tiles the
 * product stages (within float32 summation tolerance of row_reduce_sum: the order differs). Workspace:
 * nnhip_gemm_workspace_bytes(M, N, K, count). Within the GEMM tolerance of the separate products (the K
 * split differs). No CUDA counterpart. */
int nnhip_gemm_group_acc(const float* const* A, const float* B, float* const* C, size_t count, size_t M, size_t N,
                         size_t K, int transB, int accumulate, float* const* row_sums, int row_sums_accumulate,
                         void* workspace, size_t workspace_bytes, void* stream);

/* nnhip_gemm_group_acc with a B of each member: C_i = [C_i +] A_i op(B_i), i < count (1..4), every B_i of one
 * shape. The attention's four Linears (output, q, k, v) have weight gradients of one shape, d_model x
 * d_model over the batch's tokens (compute_layer.hpp:183-185 in each Linear::backward), the output
 * projection's with its own input; they run as one launch. Same rounding and row sums as
 * nnhip_gemm_group_acc. No CUDA counterpart. */
int nnhip_gemm_group_acc_each(const float* const* A, const float* const* B, float* const* C, size_t count,
                              size_t M, size_t N, size_t K, int transB, int accumulate, float* const* row_sums,
                              int row_sums_accumulate, void* workspace, size_t workspace_bytes, void* stream);

/* nnhip_gemm_group_acc_each with transB, member i's A and / or B stored by sequence (a_seq[i], b_seq[i];
 * either array may be NULL): the q, k and v layers' gradients G_i come from the attention backward as heads'
 * rows (compute_layer.hpp:1377-1386 rearranges them back) and the output projection's input is the
 * attention output as heads' rows (:1256-1259); the weight gradients read them in place. Returns -7 when
 * the shapes do not give whole tiles (the caller rearranges instead). No CUDA counterpart. */
int nnhip_gemm_group_acc_seq(const float* const* A, const float* const* B, float* const* C, size_t count, size_t M,
                             size_t N, size_t K, int transB, int accumulate, float* const* row_sums,
                             int row_sums_accumulate, const nnhip_by_seq* a_seq, const nnhip_by_seq* b_seq,
                             void* workspace, size_t workspace_bytes, void* stream);

/* C (M, N) = alpha * sum_i A_i^T B_i over count (1..3) products of one shape, one accumulator over
 * K = count * K_each in segment order: A_i stored (K_each, M), B_i (K_each, N), all 16-byte aligned, M and N
 * multiples of 4, K_each a multiple of 16. The attention's input gradient is three Linear backward products
 * added in place (compute_layer.hpp:1397-1408: dx = Wq^T gQ; dx += Wk^T gK; dx += Wv^T gV); this computes it
 * as one product, rounded once per output instead of after each add (within the GEMM tolerance of the
 * separate calls, not bit-identical). Workspace as nnhip_gemm at K = count * K_each. No CUDA counterpart. */
int nnhip_gemm_tn_sum(const float* const* A, const float* const* B, size_t count, float* C, size_t M, size_t N,
                      size_t K_each, float alpha, void* workspace, size_t workspace_bytes, void* stream);

/* nnhip_gemm_tn_sum with every B_i stored by sequence along n (b_seq): the attention's input gradient
 * Wq^T gQ + Wk^T gK + Wv^T gV (compute_layer.hpp:1397-1408) from gQ, gK, gV as the backward's heads' rows,
 * without their rearrange (:1377-1386). Returns -7 when the shapes do not give whole tiles. No CUDA
 * counterpart. */
int nnhip_gemm_tn_sum_seq(const float* const* A, const float* const* B, size_t count, float* C, size_t M, size_t N,
                          size_t K_each, float alpha, nnhip_by_seq b_seq, void* workspace, size_t workspace_bytes,
                          void* stream);

/* C (M, N) = [C +] alpha A B [+ row_bias], A (M, K) stored as it is, B (K, N) stored by sequence along n
 * (b_seq), rounded as nnhip_gemm_epilogue: the attention's output projection of its output as heads' rows
 * (compute_layer.hpp:1256-1259 rearranges them, then Linear::forward). Returns -7 when the shapes do not
 * give whole tiles. No CUDA counterpart. */
int nnhip_gemm_epilogue_seq(const float* A, const float* B, float* C, size_t M, size_t N, size_t K, float alpha,
                            const float* row_bias, int accumulate, nnhip_by_seq b_seq, void* workspace,
                            size_t workspace_bytes, void* stream);

/* One product with the epilogue of the call that follows it in the reference's Linear layer
 * (compute_layer.hpp Linear::forward / backward): C = alpha * op(A) op(B), then C[i][j] += row_bias[i]
 * (broadcast_row_inplace(C, bias, Add)) when row_bias is not null, and C = C_old + result
 * (add_inplace(C_old, result)) when accumulate; each addition rounded as the separate call rounds it.
 * Workspace as nnhip_gemm. No CUDA counterpart. */
int nnhip_gemm_epilogue(const float* A, const float* B, float* C, size_t A_rows, size_t A_cols, size_t B_rows,
                        size_t B_cols, int transA, int transB, float alpha, const float* row_bias, int accumulate,
                        void* workspace, size_t workspace_bytes, void* stream);

/* Up to four products v_i (rows) = R_i (rows, K) x (+ bias_i) of one vector x in one launch, count in 1..4:
 * the q, k and v Linear forwards of one token in incremental inference (compute_layer.hpp:1426-1511 calls
 * w_q, w_k, w_v on the same x_new). v_i goes to y_i and, when out_i is set, out_i = add_i + v_i (add_i set:
 * the block's residual add, compute_layer.hpp:2413-2437) or out_i = v_i (a copy, e.g. into the KV cache row
 * of insert_rows). bias, y, add, out: NULL or arrays with NULL entries; each member needs y_i or out_i.
 * Each v_i is bit-identical to nnhip_gemm_epilogue(R_i, x, y_i, rows, K, K, 1, 0, 0, 1.0f, bias_i, 0, ...),
 * and add_i + v_i to the separate add. No CUDA counterpart. */
int nnhip_gemv_group(const float* const* R, const float* x, const float* const* bias, float* const* y,
                     const float* const* add, float* const* out, size_t count, size_t rows, size_t K, void* stream);
/* The same products of y = RMSNorm(x) instead of x (the block's norm before the q, k, v projections,
 * compute_layer.hpp:2413-2437): y is what nnhip_rmsnorm_forward(x, gamma, inv_f, eps, ...) gives for the
 * (K, 1) column x, bit for bit, and the RMSNorm outputs whose pointers are set here are written as that
 * call writes them. K <= 1024. No CUDA counterpart. */
typedef struct nnhip_gemv_rmsnorm
{
    const float* gamma;   /* (K) */
    float inv_f, eps;
    float* s_raw;         /* (1) each of these may be NULL */
    float* scaled;
    float* var_eps;
    float* rinv;
    float* normed;        /* (K) */
    float* out;           /* (K): y */
} nnhip_gemv_rmsnorm;
/* A token's SwiGLU feed-forward input in one launch (incremental inference; no CUDA counterpart): the
 * Linear fc1 of 2*half rows on x, or on RMSNorm(x) when rms is set (K <= 1024; the RMSNorm outputs as
 * nnhip_gemv_group_rmsnorm writes them), v = R x (+ bias), written to y (2*half, may be NULL), then
 * SwiGLU::forward's chain on gate = v[0, half), up = v[half, 2*half) (compute_layer.hpp:143-154 on a
 * (2*d_ff, 1) input; its scalar constants c_add = 1 and c_div = 1 as the chain passes them):
 * s = c_div / (exp(-gate) + c_add) to s_out (may be NULL) and out = (gate * s) * up. Bit-identical to
 * nnhip_gemv_group[_rmsnorm] of the 2*half rows followed by nnhip_swiglu_forward(y, y + half, s_out, out).
 * With rms, K % 4 == 0 and R 16-byte aligned. */
int nnhip_gemv_swiglu(const float* R, const float* x, const nnhip_gemv_rmsnorm* rms, const float* bias, float* y,
                      float* s_out, float* out, size_t half, size_t K, float c_add, float c_div, void* stream);
int nnhip_gemv_group_rmsnorm(const float* const* R, const float* x, const nnhip_gemv_rmsnorm* rms,
                             const float* const* bias, float* const* y, const float* const* add, float* const* out,
                             size_t count, size_t rows, size_t K, void* stream);

/* nnhip_gemm that allocates nothing and takes no workspace. No counterpart in the reference: it is for
 * callers that cannot allocate device memory or hand in a workspace (code under HIP graph capture, tight
 * serving loops, harnesses that forbid allocation). Split-K partial tiles go to a scratch array inside
 * the library, one per GPU, NNHIP_GEMM_NOALLOC_SCRATCH_BYTES (64 MiB) in size and held until the process
 * ends. Same plan, kernels and summation order as nnhip_gemm given nnhip_gemm_workspace_bytes(M, N, K,
 * batch) bytes of workspace, so the results are identical. Returns -6, launching nothing, when that
 * workspace size exceeds NNHIP_GEMM_NOALLOC_SCRATCH_BYTES: products whose output grid fills the GPU need
 * none; among the config-4 step's, the long-K ones into small outputs (768 x 8192 from K = 6144 or
 * 32000, the 6144 x 768 and 768 x 3072 weight gradients) need 72-144 MiB and are rejected. All calls on
 * one GPU share its scratch: calls that may overlap in time on one GPU (other streams, other threads) race
 * and must be ordered by the caller. */
#define NNHIP_GEMM_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int nnhip_gemm_noalloc(const float* A, const float* B, float* C, size_t A_rows, size_t A_cols, size_t B_rows,
                       size_t B_cols, size_t batch, int transA, int transB, float alpha, void* stream);

/* Per batch b: C_b = alpha * op(A_b) op(B_b); A/B split into `batch` row blocks, C stacked (batch*M, N).
 * Replaces cuda_batched_matmul (cuda_kernels.h:49-54); alpha as in ComputeEngine::batched_matmul
 * (compute_engine.hpp:195-199, cpu_engine.hpp:335-419). */
int nnhip_batched_matmul(const float* A, const float* B, float* C, size_t A_rows, size_t A_cols, size_t B_rows,
                         size_t B_cols, size_t batch, int transA, int transB, float alpha, void* stream);

/* ── elementwise (cuda_kernels.h:60-92) ──────────────────────────────────── */
int nnhip_elementwise_unary(const float* A, float* out, size_t count, unsigned op, void* stream);
int nnhip_elementwise_binary(const float* A, const float* B, float* out, size_t count, unsigned op, void* stream);
int nnhip_elementwise_binary_scalar(const float* A, float* out, size_t count, unsigned op, float scalar,
                                    int scalar_first, void* stream);
/* out = A + scalar * B (cuda_axpy, cuda_kernels.h:83-86). */
int nnhip_axpy(const float* A, const float* B, float* out, size_t count, float scalar, void* stream);
int nnhip_elementwise_select_scalar_cond(const float* A, const float* then_v, float* out, size_t count,
                                         unsigned cmp, float scalar_b, float scalar_else, void* stream);
/* One Adam / AdamW update of a parameter tensor in one pass, rounding every step exactly as the
 * reference's chain of engine primitives does (compute_optimizer.hpp:252-304; AdamW's decay
 * scale_inplace(p, 1 - lr*wd), :388-412, when has_decay): m = m*beta1; m = fma(1-beta1, g, m);
 * v = v*beta2 + (g*g)*(1-beta2); p = p*decay + (-lr) * ((m*inv_bc1) / (sqrt(v*inv_bc2) + eps)).
 * p, m, v updated in place; g read only. The CUDA backend has no counterpart (it runs the
 * primitive chain); HipEngine issues this when it recognises that chain among deferred calls. */
int nnhip_adam_update(float* p, float* m, float* v, const float* g, size_t count, int has_decay, float decay,
                      float beta1, float one_minus_beta1, float beta2, float one_minus_beta2, float inv_bc1,
                      float inv_bc2, float eps, float neg_lr, void* stream);
/* The update above for n tensors with one set of scalars (one optimizer step over every parameter,
 * compute_optimizer.hpp:252-304, :388-412), in as few launches as possible (48 tensors per launch):
 * tensor i is p[i], m[i], v[i], g[i] of counts[i] floats. Bit-identical to n nnhip_adam_update calls. */
int nnhip_adam_update_list(float* const* p, float* const* m, float* const* v, const float* const* g,
                           const size_t* counts, size_t n, int has_decay, float decay, float beta1,
                           float one_minus_beta1, float beta2, float one_minus_beta2, float inv_bc1, float inv_bc2,
                           float eps, float neg_lr, void* stream);
/* SwiGLU forward (reference compute_layer.hpp, SwiGLU::forward, a chain of six primitives:
 * Neg, Exp, + c_add, c_div / x, gate * s, * up) in one pass with the same roundings:
 * s = c_div / (exp(-gate) + c_add) (stored when s_out is not null), out = (gate * s) * up.
 * No CUDA counterpart; HipEngine issues it when it recognises that chain among deferred calls. */
int nnhip_swiglu_forward(const float* gate, const float* up, float* s_out, float* out, size_t count, float c_add,
                         float c_div, void* stream);
/* dst[i] = src[i] for count floats (non-overlapping): slice_rows / insert_rows / clone (cpu_engine.hpp:75-114;
 * the CUDA engine uses cudaMemcpy). */
int nnhip_copy(const float* src, float* dst, size_t count, void* stream);
/* Zeroes n device buffers (ptrs[i], counts[i] floats) in as few launches as possible (consecutive
 * ComputeEngine::zero calls, e.g. Optimizer::zero_grad, compute_optimizer.hpp:142-151). */
int nnhip_zero_list(float* const* ptrs, const size_t* counts, size_t n, void* stream);
/* out[i] = value (used for ComputeEngine::zero; no CUDA counterpart, CUDA uses cudaMemset). */
int nnhip_fill(float* out, size_t count, float value, void* stream);

/* ── reductions (cuda_kernels.h:98-109); mode 0 = sum, 1 = max (init lowest()) ── */
int nnhip_reduce_row(const float* A, float* out, size_t rows, size_t cols, unsigned mode, void* stream);
/* out[r] = out[r] + (row sum of A)[r]: the sums added into out as a following add_inplace(out, sums) would
 * add them (a Linear bias gradient, compute_layer.hpp Linear::backward; no CUDA counterpart). */
int nnhip_reduce_row_sum_add(const float* A, float* out, size_t rows, size_t cols, void* stream);
/* Column reduction over row chunks combined in chunk order; workspace from nnhip_reduce_col_workspace_bytes. */
size_t nnhip_reduce_col_workspace_bytes(size_t rows, size_t cols);
int nnhip_reduce_col(const float* A, float* out, size_t rows, size_t cols, unsigned mode, void* workspace,
                     void* stream);

/* ── broadcast (cuda_kernels.h:115-125) ───────────────────────────────────── */
int nnhip_broadcast_row(const float* A, const float* vec, float* out, size_t rows, size_t cols, unsigned op,
                        void* stream);
int nnhip_broadcast_col(const float* A, const float* vec, float* out, size_t rows, size_t cols, unsigned op,
                        void* stream);

/* ── layout (cuda_kernels.h:131-143) ──────────────────────────────────────── */
int nnhip_transpose(const float* A, float* out, size_t R, size_t C, void* stream);
/* Per batch b: out rows [b*C, (b+1)*C) = (A rows [b*R, (b+1)*R))^T, i.e. rearrange_3d(transpose(A), C,
 * batch, R) (cpu_engine.hpp:226-287) in one pass; the reference's two-pass attention makes V and dO
 * (per batch (d_k, seq)) query-major that way (compute_layer.hpp:1211-1214, :1309-1313). No CUDA
 * counterpart. */
int nnhip_transpose_batched(const float* A, float* out, size_t batch, size_t R, size_t C, void* stream);
int nnhip_rearrange_3d(const float* A, float* out, size_t M, size_t B, size_t N, unsigned inverse, void* stream);

/* ── gather / scatter (cuda_kernels.h:151-163) ───────────────────────────
 * gather: out[i] = table[idx[i]] or a zero row when idx[i] is out of range (cpu_engine.hpp:125-179).
 * scatter_add: dst[idx[i]] += grad[i] in increasing i per destination row, bit-identical to the
 * CPU engine's serial loop (cpu_engine.hpp:184-216); the CUDA version uses unordered atomics. */
int nnhip_gather(const float* table, const float* indices, float* out, size_t vocab, size_t D, size_t num,
                 void* stream);
size_t nnhip_scatter_add_workspace_bytes(size_t num);
int nnhip_scatter_add(float* dst, const float* indices, const float* grad, size_t vocab, size_t D, size_t num,
                      void* workspace, void* stream);

/* ── fused attention primitives (no CUDA counterpart) ────────────────────
 * Shapes as ComputeEngine (compute_engine.hpp:217-276): per batch A_b is (M,K), or stored (K,M) when
 * transA; B_b is (K,N), or stored (N,K) when transB; mask (M,N) shared by all batches (-inf excludes,
 * finite values add) or NULL. With a workspace of nnhip_bmm_workspace_bytes(batch, M, N, K, D) bytes
 * (D: value width of softmax_apply, else 1) and head dims K <= 128, the matrix-core kernels run: they
 * skip fully masked 32x32 cells (causal and document masks) and split long rows over several
 * workgroups whose partial results are combined in a fixed order (deterministic). With workspace
 * NULL a general, slower path runs. */
size_t nnhip_bmm_workspace_bytes(size_t batch, size_t M, size_t N, size_t K, size_t D);
/* cpu_engine.hpp:426-532: out[b*M+i] = reduce_j(alpha*dot + mask) (reduce_cols), or out[b*N+j] over i. */
int nnhip_bmm_reduce(const float* A, const float* B, const float* mask, float* out, size_t batch, size_t M,
                     size_t N, size_t K, int transA, int transB, unsigned op, float alpha, int reduce_cols,
                     void* workspace, void* stream);
/* cpu_engine.hpp:535-604: l[b*M+i] = sum_j exp(alpha*dot + mask - row_max[b*M+i]). */
int nnhip_bmm_softmax_denom(const float* A, const float* B, const float* row_max, const float* mask, float* out,
                            size_t batch, size_t M, size_t N, size_t K, int transA, int transB, float alpha,
                            void* workspace, void* stream);
/* cpu_engine.hpp:607-699: O[(b*M+i)*D+k] = sum_j W_ij V[(b*N+j)*D+k]. */
int nnhip_bmm_softmax_apply(const float* A, const float* B, const float* V, const float* row_max,
                            const float* denom, const float* mask, float* out, size_t batch, size_t M, size_t N,
                            size_t K, size_t D, int transA, int transB, float alpha, void* workspace, void* stream);
/* cpu_engine.hpp:702-801: R[b*M+i] = sum_j W P; dQ[(b*K+k)*M+i] = alpha sum_j W (P-R) B_b[k][j]. */
int nnhip_bmm_softmax_backward_q(const float* A, const float* B, const float* P, const float* row_max,
                                 const float* denom, const float* mask, float* dQ, float* R, size_t batch,
                                 size_t M, size_t N, size_t K, int transA, int transB, float alpha, void* workspace,
                                 void* stream);
/* cpu_engine.hpp:804-915: dK[(b*K+k)*N+j] = alpha sum_i W (P-R) A_b[:,i]_k; dV = sum_i W G[b*M+i][k]
 * (G has D >= K columns). */
int nnhip_bmm_softmax_backward_kv(const float* A, const float* B, const float* P, const float* G, const float* R,
                                  const float* row_max, const float* denom, const float* mask, float* dK,
                                  float* dV, size_t batch, size_t M, size_t N, size_t K, size_t D, int transA,
                                  int transB, float alpha, void* workspace, void* stream);

/* ── one-pass attention chains (no CUDA counterpart) ─────────────────────
 * The reference's two-pass attention issues reduce(Max) -> softmax_denom -> softmax_apply forward and
 * batched_matmul(dO, V', transA) -> softmax_backward_q -> softmax_backward_kv backward
 * (compute_layer.hpp:1196-1221, :1304-1327; semantics cpu_engine.hpp:426-915, :335-419). These entry
 * points compute each chain in one pass, for the operand layouts the attention layer passes:
 * Q per batch (K,M) (the transA = 1 operand), K per batch (K,N) (transB = 0), V per batch (N,D),
 * dO per batch (Kd,M) and V' per batch (Kd,N) (P_ij = alpha2 sum_k dO(k,i) V'(k,j), recomputed, never
 * stored), G per batch (M,ldg). Supported when nnhip_flash_supported(batch, M, N, max(K,Kd), D)
 * (K, Kd <= 64; D <= 64, D % 4 == 0); the backward also needs K % 4 == 0, ldg % 4 == 0. Fully masked
 * 32x32 cells are skipped; long rows are split over workgroups and combined in a fixed order. */
int nnhip_flash_supported(size_t batch, size_t M, size_t N, size_t K, size_t D);
/* Mask cell table: one byte per 32x32 cell of the (M,N) mask (0 all -inf, 1 all zero, 2 general), the
 * argument `cells` of the calls below when a mask is given. The caller may keep it while the mask is
 * unchanged. */
size_t nnhip_flash_cells_bytes(size_t M, size_t N);
int nnhip_flash_classify(const float* mask, size_t M, size_t N, void* cells, void* stream);
/* Scratch for the partial results of rows cut into several ranges (0 when none are). */
size_t nnhip_flash_workspace_bytes(size_t batch, size_t M, size_t N, size_t K, size_t D, int backward);
/* m, l (batch*M) as reduce(Max) and softmax_denom; O (batch*M, D) as softmax_apply, or O = V = NULL. */
int nnhip_flash_forward(const float* Q, const float* Kt, const float* V, const float* mask, const void* cells,
                        float* m, float* l, float* O, size_t batch, size_t M, size_t N, size_t K, size_t D,
                        float alpha, void* workspace, void* stream);
/* R (batch*M), dQ (batch*K, M) as softmax_backward_q; dK, dV (batch*K, N) as softmax_backward_kv. */
int nnhip_flash_backward(const float* Q, const float* Kt, const float* dO, const float* Vp, const float* G, size_t ldg,
                         const float* mask, const void* cells, const float* m, const float* l, float* R, float* dQ,
                         float* dK, float* dV, size_t batch, size_t M, size_t N, size_t K, size_t Kd, float alpha,
                         float alpha2, void* workspace, void* stream);

/* Layout options of the one-pass chains for the reference's materialised attention path
 * (compute_layer.hpp:1230-1252 forward, :1331-1361 backward: scores = batched_matmul(Q, K, transA),
 * masked = scores + mask, A = softmax rows, O = batched_matmul(V, A, transB); dV = batched_matmul(dO, A),
 * P = batched_matmul(dO, V, transA), dS = softmax backward, dQ = batched_matmul(K, dS, transB),
 * dK = batched_matmul(Q, dS)), which HipEngine runs here without materialising scores or A:
 *   mask_batch_stride  floats between the batch entries' (M, N) masks (0: one mask for all), e.g. M*N for
 *                      the (batch*M, N) ALiBi / document mask; cells then come from
 *                      nnhip_flash_classify_batched over the same masks;
 *   v_dim_major        V per batch is (D, N) [dim][key] (the layer's (B*H*d, T) heads) instead of (N, D);
 *   o_dim_major        O per batch is written (D, M) [dim][query] instead of (M, D);
 *   g_is_do            G_i is dO's column i (dV_j = sum_i W_ij dO_i, the materialised path's
 *                      batched_matmul(dO, A)); G and ldg are ignored; needs Kd == K.
 * No CUDA counterpart (cuda_engine.hpp leaves the attention primitives to the CPU). */
int nnhip_flash_classify_batched(const float* mask, size_t masks, size_t mask_batch_stride, size_t M, size_t N,
                                 void* cells, void* stream);
int nnhip_flash_forward_layout(const float* Q, const float* Kt, const float* V, const float* mask, const void* cells,
                               float* m, float* l, float* O, size_t batch, size_t M, size_t N, size_t K, size_t D,
                               float alpha, size_t mask_batch_stride, int v_dim_major, int o_dim_major,
                               void* workspace, void* stream);
int nnhip_flash_backward_layout(const float* Q, const float* Kt, const float* dO, const float* Vp, const float* G,
                                size_t ldg, const float* mask, const void* cells, const float* m, const float* l,
                                float* R, float* dQ, float* dK, float* dV, size_t batch, size_t M, size_t N, size_t K,
                                size_t Kd, float alpha, float alpha2, size_t mask_batch_stride, int g_is_do,
                                void* workspace, void* stream);
/* Backward of the materialised path when the forward output O is at hand (per batch (K, M), dim-major,
 * computed from the same V as Vp): R_i = alpha2 dO_i . O_i, then one key-line pass for dK, dV and
 * dS = W (P - R) (stored in the workspace), then dQ = alpha dS K; G is dO's columns (Kd == K). Workspace
 * from nnhip_flash_ds_workspace_bytes (batch*M*N floats of dS included). No CUDA counterpart. */
size_t nnhip_flash_ds_workspace_bytes(size_t batch, size_t M, size_t N, size_t K);
int nnhip_flash_backward_ds(const float* Q, const float* Kt, const float* dO, const float* Vp, const float* O,
                            const float* mask, const void* cells, const float* m, const float* l, float* dQ, float* dK,
                            float* dV, size_t batch, size_t M, size_t N, size_t K, float alpha, float alpha2,
                            size_t mask_batch_stride, void* workspace, void* stream);
/* Work order of the calls above with a mask (no CUDA counterpart). The kernels' time is set by the most
 * loaded CU; an order table (built from a cell table for one (batch, M, N): kind 0 the forward, 1 the
 * backward, 2 the backward from the forward output) sorts the line groups by the cells they visit and
 * spreads heavy and light ones over the CUs. Build it once per cell table and shape and pass it to the
 * _ordered variants, which are the calls above plus `order` (NULL: the calls above). Results do not
 * depend on the order. */
size_t nnhip_flash_order_bytes(size_t batch, size_t M, size_t N, int kind);
int nnhip_flash_build_order(const void* cells, size_t batch, size_t M, size_t N, size_t mask_batch_stride, int kind,
                            void* order, void* stream);
/* scores (forward, may be NULL): each visited 32 x 32 cell's alpha q.k + mask, -inf past N, stored as
 * a block of 1024 floats at ((b*RT + query tile)*CT + key tile)*1024 (RT, CT = M, N in 32-tiles), score
 * (query q, key k) at r*64 + h*32 + q where k = 8*(r/4) + 4*h + r%4; batch*RT*CT*1024 floats. The
 * dS backward reads them back (scores, same cells and shape) instead of computing them again. */
int nnhip_flash_forward_ordered(const float* Q, const float* Kt, const float* V, const float* mask, const void* cells,
                                float* m, float* l, float* O, size_t batch, size_t M, size_t N, size_t K, size_t D,
                                float alpha, size_t mask_batch_stride, int v_dim_major, int o_dim_major,
                                float* scores, const void* order, void* workspace, void* stream);
int nnhip_flash_backward_ordered(const float* Q, const float* Kt, const float* dO, const float* Vp, const float* G,
                                 size_t ldg, const float* mask, const void* cells, const float* m, const float* l,
                                 float* R, float* dQ, float* dK, float* dV, size_t batch, size_t M, size_t N, size_t K,
                                 size_t Kd, float alpha, float alpha2, size_t mask_batch_stride, int g_is_do,
                                 const void* order, void* workspace, void* stream);
/* nnhip_flash_backward_ds_ordered also takes O per batch (M, K) query-major when o_query_major (the
 * two-pass chain's softmax_apply output) and writes R (batch*M) when R is not NULL. */
int nnhip_flash_backward_ds_ordered(const float* Q, const float* Kt, const float* dO, const float* Vp, const float* O,
                                    int o_query_major, const float* mask, const void* cells, const float* m,
                                    const float* l, float* R, float* dQ, float* dK, float* dV, size_t batch, size_t M,
                                    size_t N, size_t K, float alpha, float alpha2, size_t mask_batch_stride,
                                    const float* scores, const void* order, void* workspace, void* stream);
/* Multi-row launches (no CUDA counterpart): nrows (1..NNHIP_FLASH_MAX_ROWS) independent two-pass chains of one shape, hpr
 * batch entries each, as one launch. The reference issues a document-masked batch as one chain per
 * packed row, since each row has its own (M, N) mask (the primitives take one mask shared by the batch:
 * cpu_engine.hpp:426-915); one row alone fills a small part of the GPU. Row r's pointers are those of
 * its own one-row call (nnhip_flash_forward_ordered with mask_batch_stride 0; the dS backward's R may be
 * NULL in every row or in none). Workspaces: nnhip_flash_workspace_bytes / nnhip_flash_ds_workspace_bytes
 * at batch nrows * hpr. order: a table from nnhip_flash_build_rows_order over the rows' cell tables
 * (nnhip_flash_order_bytes at batch nrows * hpr), or NULL. */
#define NNHIP_FLASH_MAX_ROWS 8
typedef struct nnhip_flash_fwd_row
{
    const float* Q;
    const float* Kt;
    const float* V;
    const float* mask;
    const void* cells;
    float* m;
    float* l;
    float* O;
    float* scores;
} nnhip_flash_fwd_row;
typedef struct nnhip_flash_bwd_row
{
    const float* Q;
    const float* Kt;
    const float* dO;
    const float* Vp;
    const float* O;
    const float* mask;
    const void* cells;
    const float* m;
    const float* l;
    const float* scores;
    float* R;
    float* dQ;
    float* dK;
    float* dV;
} nnhip_flash_bwd_row;
int nnhip_flash_forward_rows(const nnhip_flash_fwd_row* rows, size_t nrows, size_t hpr, size_t M, size_t N, size_t K,
                             size_t D, float alpha, int v_dim_major, int o_dim_major, const void* order,
                             void* workspace, void* stream);
int nnhip_flash_backward_ds_rows(const nnhip_flash_bwd_row* rows, size_t nrows, size_t hpr, size_t M, size_t N,
                                 size_t K, float alpha, float alpha2, int o_query_major, const void* order,
                                 void* workspace, void* stream);
int nnhip_flash_build_rows_order(const void* const* cells, size_t nrows, size_t hpr, size_t M, size_t N, int kind,
                                 void* order, void* stream);

/* One query per batch entry (incremental inference, compute_layer.hpp:1426-1511: scores =
 * batched_matmul(q, K_T, transA, scale), + the ALiBi row, softmax, batched_matmul(V_T, attn, transB)),
 * with keys and values read where they lie. For b < batch, j < N:
 *   s_j = alpha * (q_b . k_bj) + mask[b*mask_bs + j]   (no mask term when mask is NULL)
 *   m[b] = max_j s_j, l[b] = sum_j exp(s_j - m[b]), O[b*D + d] = sum_j exp(s_j - m[b]) v_bj[d] / l[b]
 *   P[b*N + j] = exp(s_j - m[b]) / l[b]   (the probabilities, when P is not NULL)
 * (m = lowest(), l = 0, O = 0 when every s_j is -inf, as nnhip_flash_forward leaves such rows), with
 * q_b[k] = Q[b*K + k], k_bj[k] = Kp[b*kb + j*kj + k*kk], v_bj[d] = V[b*vb + j*vj + d*vd]: the rows of
 * a (seq, heads*d) KV cache are read in place with kb = d, kj = heads*d, kk = 1. K, D <= 64. Workspace:
 * nnhip_attn_query_workspace_bytes (0 up to 256 keys; longer rows are split and merged in key order).
 * No CUDA counterpart. */
size_t nnhip_attn_query_workspace_bytes(size_t batch, size_t N, size_t D);
int nnhip_attn_query(const float* Q, const float* Kp, long kb, long kj, long kk, const float* V, long vb, long vj,
                     long vd, const float* mask, long mask_bs, float* m, float* l, float* O, float* P, size_t batch,
                     size_t N, size_t K, size_t D, float alpha, void* workspace, void* stream);

/* ── column softmax / sparse cross-entropy (no CUDA counterpart) ─────────
 * cpu_engine.hpp:922-945 and :948-1006. Workspace from nnhip_col_softmax_workspace_bytes. */
size_t nnhip_col_softmax_workspace_bytes(size_t C, size_t N);
int nnhip_col_softmax_denom(const float* logits, const float* col_max, float* out, size_t C, size_t N,
                            void* workspace, void* stream);
int nnhip_col_softmax_sparse_forward(const float* logits, const float* labels, const float* mask, float* grad,
                                     float* loss_vec, size_t C, size_t N, size_t vocab_size, float inv_num_valid,
                                     void* workspace, void* stream);

/* The sparse cross-entropy of logits produced by nnhip_gemm_colstats (the GPT's lm_head Linear:
 * logits = W x + b, compute_layer.hpp Linear::forward, then CrossEntropyLoss::forward_sparse,
 * compute_loss.hpp:229-309): the product's epilogue leaves, per column and per block of
 * nnhip_gemm_colstats_tiles(M, N, K, transA, transB) rows, the max and the sum of exp(x - max) in
 * stats[(tile) * N + col] and stats[(tiles + tile) * N + col] (2 * tiles * N floats; 0 tiles: the
 * shape has no such epilogue). nnhip_col_softmax_sparse_from_stats merges them in row order and writes
 * the gradient and loss as nnhip_col_softmax_sparse_forward does, reading the logits once instead of
 * twice; workspace 2 * N floats. No CUDA counterpart. */
size_t nnhip_gemm_colstats_tiles(size_t M, size_t N, size_t K, int transA, int transB);
int nnhip_gemm_colstats(const float* A, const float* B, float* C, size_t A_rows, size_t A_cols, size_t B_rows,
                        size_t B_cols, int transA, int transB, const float* row_bias, float* stats, void* stream);
int nnhip_col_softmax_sparse_from_stats(const float* logits, const float* labels, const float* mask,
                                        const float* stats, size_t tiles, float* grad, float* loss_vec, size_t C,
                                        size_t N, size_t vocab_size, float inv_num_valid, void* workspace,
                                        void* stream);

/* ── row softmax (eval_expr fast path of the Softmax layer, compute_layer.hpp:832-862) ──
 * forward: out = exp(x - rowmax) / sum(exp(x - rowmax)); backward: dx = y * (g - sum(y*g)). */
int nnhip_row_softmax(const float* X, float* out, size_t rows, size_t cols, void* stream);
int nnhip_row_softmax_backward(const float* Y, const float* G, float* out, size_t rows, size_t cols, void* stream);

/* ── fused GPT-layer programs (eval_expr fast paths) ─────────────────────
 * One kernel per ExprSpec program the layers issue, the role of the reference's ahead-of-time fused
 * shaders (tools/scan_exprs.cpp, tools/gen_fused.cpp; no CUDA counterpart). Matrices are (F, N) with
 * N % 4 == 0 and 16-byte aligned pointers, else -5 is returned and nothing runs. vectors: gamma and
 * row results (F); m, rinv and column results (N).
 *   RMSNorm forward, compute_layer.hpp:733-754:  sumsq  out[c] = sum_r X[r,c]^2;
 *     colbcast_mul  out = X * v[c];  rowbcast_mul  out = X * v[r].
 *   RMSNorm backward, compute_layer.hpp:772-795:  bwd_colsum  out[c] = sum_r G*gamma[r]*Nrm;
 *     bwd_dx  out = (G*gamma[r] - m[c]*Nrm) * rinv[c];  bwd_rowsum  out[r] = sum_c G*gamma[r]*Nrm.
 *   SwiGLU backward, compute_layer.hpp:436-444 (count % 4 == 0):
 *     grad_gate = G*up*(s*(1 + gate*(1 - s)));  grad_up = G*gate*s.
 * sumsq, colbcast_mul and rmsnorm_forward also take narrow matrices (N % 4 != 0, 1 <= F <= 1024, N <= 65535,
 * any alignment): one token's (F, 1) activations in incremental inference. */
int nnhip_rmsnorm_sumsq(const float* X, float* out, size_t F, size_t N, void* stream);
int nnhip_colbcast_mul(const float* X, const float* v, float* out, size_t F, size_t N, void* stream);
int nnhip_rowbcast_mul(const float* X, const float* v, float* out, size_t F, size_t N, void* stream);
/* RMSNorm::forward's six calls in one pass (compute_layer.hpp:733-754; no CUDA counterpart): s = sumsq(X),
 * scaled = s * inv_f, var_eps = scaled + eps, rinv = 1 / sqrt(var_eps), normed = X * rinv[c],
 * out = normed * gamma[r], equal bit for bit to the separate calls; s_raw, scaled and var_eps (N) may be
 * NULL (not written). 1 <= F <= 1024. */
int nnhip_rmsnorm_forward(const float* X, const float* gamma, float inv_f, float eps, float* s_raw, float* scaled,
                          float* var_eps, float* rinv, float* normed, float* out, size_t F, size_t N, void* stream);
/* nnhip_rmsnorm_forward of X = A + B, X written as well: GPTBlock::forward's residual add followed by the next
 * RMSNorm (compute_layer.hpp:2375-2379 and 2385 with the following block's norm, each add rounded as
 * elementwise_binary(Add)), one pass reading A and B. N % 4 == 0, every matrix 16-byte aligned. Outputs equal
 * elementwise_binary(Add, A, B) followed by nnhip_rmsnorm_forward bit for bit. No CUDA counterpart. */
int nnhip_rmsnorm_forward_sum(const float* A, const float* B, float* X, const float* gamma, float inv_f, float eps,
                              float* s_raw, float* scaled, float* var_eps, float* rinv, float* normed, float* out,
                              size_t F, size_t N, void* stream);
/* RMSNorm::backward's column sum, its scaling and dx in one pass (compute_layer.hpp:772-791; no CUDA
 * counterpart): m_raw = bwd_colsum(G, gamma, Nrm), m = m_raw * inv_f, dx = bwd_dx(G, gamma, m, Nrm, rinv),
 * equal bit for bit to the separate calls; m_raw may be NULL. 1 <= F <= 1024. */
int nnhip_rmsnorm_backward(const float* G, const float* gamma, const float* Nrm, const float* rinv, float inv_f,
                           float* m_raw, float* m, float* dx, size_t F, size_t N, void* stream);
/* nnhip_rmsnorm_backward that also writes out2 = addend + dx: GPTBlock::backward's residual adds of the layer
 * gradients (compute_layer.hpp:2396 and 2404, elementwise_binary(Add, grad, dx)), in the same pass. dx, out2
 * equal the separate calls bit for bit. No CUDA counterpart. */
int nnhip_rmsnorm_backward_add(const float* G, const float* gamma, const float* Nrm, const float* rinv, float inv_f,
                               float* m_raw, float* m, float* dx, const float* addend, float* out2, size_t F,
                               size_t N, void* stream);
int nnhip_rmsnorm_bwd_colsum(const float* G, const float* gamma, const float* Nrm, float* out, size_t F, size_t N,
                             void* stream);
int nnhip_rmsnorm_bwd_dx(const float* G, const float* gamma, const float* m, const float* Nrm, const float* rinv,
                         float* out, size_t F, size_t N, void* stream);
int nnhip_rmsnorm_bwd_rowsum(const float* G, const float* gamma, const float* Nrm, float* out, size_t F, size_t N,
                             void* stream);
/* out[r] = out[r] + bwd_rowsum(...)[r]: the row sums added into out as a following add_inplace(out, sums)
 * would add them (RMSNorm::backward's grad_gamma += gg; no CUDA counterpart). */
int nnhip_rmsnorm_bwd_rowsum_add(const float* G, const float* gamma, const float* Nrm, float* out, size_t F,
                                 size_t N, void* stream);
int nnhip_swiglu_grad_gate(const float* G, const float* up, const float* s, const float* gate, float* out,
                           size_t count, void* stream);
int nnhip_swiglu_grad_up(const float* G, const float* gate, const float* s, float* out, size_t count, void* stream);
/* Both of the above in one pass (SwiGLU::backward's two programs, whose results it inserts into one (2 d_ff, N)
 * gradient): out_gate and out_up may be rows of one tensor. Same roundings as the separate calls. */
int nnhip_swiglu_grad_both(const float* G, const float* up, const float* s, const float* gate, float* out_gate,
                           float* out_up, size_t count, void* stream);

/* ── ExprSpec interpreter (no CUDA counterpart; cpu_engine.hpp:1298-1659) ──
 * The program is the ExprSpec in serialised form (see nnhip_engine.h); inputs[k] are device pointers
 * shaped per view. Workspace from nnhip_eval_expr_workspace_bytes. */
typedef struct nnhip_expr_program {
    unsigned char instrs[64][8]; /* {op, dst, a.kind, a.idx, b.kind, b.idx, c.kind, c.idx} */
    unsigned char view_kind[8];
    unsigned char view_negate[8];
    unsigned int view_param[8];
    float consts[16];
    unsigned int n_instrs, n_views, n_consts, num_regs;
} nnhip_expr_program;
size_t nnhip_eval_expr_workspace_bytes(const nnhip_expr_program* prog, size_t rows, size_t cols);
int nnhip_eval_expr(const nnhip_expr_program* prog, const float* const* inputs, float* out, size_t rows,
                    size_t cols, int vector_out, void* workspace, void* stream);

#if defined(__GNUC__)
#pragma GCC visibility pop
#endif
#ifdef __cplusplus
}
#endif

#endif /* NNHIP_KERNELS_H */
