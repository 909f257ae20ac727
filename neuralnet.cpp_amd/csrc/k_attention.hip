// k_attention.hip — the fused attention primitives of ComputeEngine
// (compute_engine.hpp:217-276), general-shape path.
//
// Semantics follow the CPU engine (cpu_engine.hpp:426-915) term by term:
//   s_ij  = alpha * dot_k(A_b(i,k), B_b(k,j)) + mask(i,j)      (k ascending)
//   W_ij  = exp(s_ij - row_max_i) / denom_i                     (0 where mask = -inf)
// with A_b(i,k) = A[b*M*K + (transA ? k*M + i : i*K + k)] and
// B_b(k,j) = B[b*K*N + (transB ? j*K + k : k*N + j)].
// The matrix-core kernels (k_attn_mfma.hip) take every call with a workspace
// and head dim K <= 128 (value width <= 128), except bmm_reduce with Sum/Min
// or over columns; this file holds the entry points and the general fallback,
// in which one workgroup owns one output row (query i, or key j for backward_kv); its
// fixed operand vector is staged in LDS and the lanes sweep the other index.
// Every sum over j (or i) that produces an output element runs in the CPU's
// order inside one lane; only the row-level reductions (max / denominators
// / R) are tree-combined across lanes.
#include "attn_mfma.hpp"
#include "common.hpp"
#include "nnhip_kernels.h"

namespace nnhip
{
namespace
{

constexpr unsigned kThreads = 256;
constexpr float kNegInf = -__builtin_huge_valf();

struct Dims
{
    const float* A;
    const float* B;
    const float* mask;
    size_t M, N, K;
    int tA, tB;
    float alpha;
};

__device__ __forceinline__ float a_at(const Dims& d, size_t b, size_t i, size_t k)
{
    return d.A[b * d.M * d.K + (d.tA ? k * d.M + i : i * d.K + k)];
}
__device__ __forceinline__ float b_at(const Dims& d, size_t b, size_t k, size_t j)
{
    return d.B[b * d.K * d.N + (d.tB ? j * d.K + k : k * d.N + j)];
}
__device__ __forceinline__ float mask_at(const Dims& d, size_t i, size_t j)
{
    return d.mask ? d.mask[i * d.N + j] : 0.0f;
}
// Score with query vector q (K floats, LDS) against key column j.
__device__ __forceinline__ float score_row(const Dims& d, const float* q, size_t b, size_t j)
{
    float s = 0.0f;
    for (size_t k = 0; k < d.K; ++k) s += q[k] * b_at(d, b, k, j);
    return s;
}
// Score with key vector kv (K floats, LDS) against query row i.
__device__ __forceinline__ float score_col(const Dims& d, const float* kv, size_t b, size_t i)
{
    float s = 0.0f;
    for (size_t k = 0; k < d.K; ++k) s += a_at(d, b, i, k) * kv[k];
    return s;
}

__device__ __forceinline__ float reduce_combine(unsigned op, float acc, float v)
{
    return op == R_MAX ? fmax_std(acc, v) : op == R_MIN ? fmin_std(acc, v) : acc + v;
}

// Workgroup-wide reduction (all lanes must call it); every lane gets the result.
__device__ float block_reduce(float v, unsigned op, float* scratch)
{
    for (int o = 32; o > 0; o >>= 1) v = reduce_combine(op, v, __shfl_xor(v, o, 64));
    const unsigned lane = threadIdx.x % 64, wave = threadIdx.x / 64;
    __syncthreads();
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    float t = scratch[0];
    for (unsigned w = 1; w < kThreads / 64; ++w) t = reduce_combine(op, t, scratch[w]);
    return t;
}

__device__ __forceinline__ float reduce_init(unsigned op) { return op == R_MAX ? kLowest : op == R_MIN ? kMaxF : 0.0f; }

// ── batched_matmul_reduce, reduce_cols = true: one workgroup per (b, i) ───
__global__ __launch_bounds__(kThreads) void k_bmm_reduce_rows(Dims d, float* out, unsigned op)
{
    extern __shared__ float q[];
    __shared__ float scratch[kThreads / 64];
    const size_t b = blockIdx.y, i = blockIdx.x;
    for (size_t k = threadIdx.x; k < d.K; k += kThreads) q[k] = a_at(d, b, i, k);
    __syncthreads();
    const bool skip_masked = op == R_SUM || op == R_MIN;
    float acc = reduce_init(op);
    for (size_t j = threadIdx.x; j < d.N; j += kThreads)
    {
        const float mv = mask_at(d, i, j);
        if (skip_masked && mv == kNegInf) continue;
        acc = reduce_combine(op, acc, d.alpha * score_row(d, q, b, j) + mv);
    }
    acc = block_reduce(acc, op, scratch);
    if (threadIdx.x == 0) out[b * d.M + i] = acc;
}

// ── batched_matmul_reduce, reduce_cols = false: one workgroup per (b, j) ──
__global__ __launch_bounds__(kThreads) void k_bmm_reduce_cols(Dims d, float* out, unsigned op)
{
    extern __shared__ float kv[];
    __shared__ float scratch[kThreads / 64];
    const size_t b = blockIdx.y, j = blockIdx.x;
    for (size_t k = threadIdx.x; k < d.K; k += kThreads) kv[k] = b_at(d, b, k, j);
    __syncthreads();
    const bool skip_masked = op == R_SUM || op == R_MIN;
    float acc = reduce_init(op);
    for (size_t i = threadIdx.x; i < d.M; i += kThreads)
    {
        const float mv = mask_at(d, i, j);
        if (skip_masked && mv == kNegInf) continue;
        acc = reduce_combine(op, acc, d.alpha * score_col(d, kv, b, i) + mv);
    }
    acc = block_reduce(acc, op, scratch);
    if (threadIdx.x == 0) out[b * d.N + j] = acc;
}

// ── batched_matmul_softmax_denom ─────────────────────────────────────────
__global__ __launch_bounds__(kThreads) void k_bmm_denom(Dims d, const float* row_max, float* out)
{
    extern __shared__ float q[];
    __shared__ float scratch[kThreads / 64];
    const size_t b = blockIdx.y, i = blockIdx.x;
    for (size_t k = threadIdx.x; k < d.K; k += kThreads) q[k] = a_at(d, b, i, k);
    __syncthreads();
    const float m = row_max[b * d.M + i];
    float acc = 0.0f;
    for (size_t j = threadIdx.x; j < d.N; j += kThreads)
    {
        const float mv = mask_at(d, i, j);
        if (mv == kNegInf) continue;
        acc += expf(d.alpha * score_row(d, q, b, j) + mv - m);
    }
    acc = block_reduce(acc, R_SUM, scratch);
    if (threadIdx.x == 0) out[b * d.M + i] = acc;
}

constexpr unsigned kChunk = 1024;   // j values staged per pass

// ── batched_matmul_softmax_apply: O_i = sum_j W_ij V_j ────────────────────
__global__ __launch_bounds__(kThreads) void k_bmm_apply(Dims d, const float* V, const float* row_max,
                                                        const float* denom, float* out, size_t D)
{
    extern __shared__ float q[];   // K floats, then kChunk weights
    float* w = q + d.K;
    const size_t b = blockIdx.y, i = blockIdx.x;
    for (size_t k = threadIdx.x; k < d.K; k += kThreads) q[k] = a_at(d, b, i, k);
    const float m = row_max[b * d.M + i], inv_l = 1.0f / denom[b * d.M + i];
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};   // columns threadIdx.x + 256*u, D <= 1024
    for (size_t j0 = 0; j0 < d.N; j0 += kChunk)
    {
        const size_t jn = (d.N - j0 < kChunk) ? d.N - j0 : kChunk;
        __syncthreads();
        for (size_t jj = threadIdx.x; jj < jn; jj += kThreads)
        {
            const size_t j = j0 + jj;
            const float mv = mask_at(d, i, j);
            w[jj] = mv == kNegInf ? 0.0f : expf(d.alpha * score_row(d, q, b, j) + mv - m) * inv_l;
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < 4; ++u)
        {
            const size_t k = threadIdx.x + kThreads * u;
            if (k >= D) break;
            float a = acc[u];
            for (size_t jj = 0; jj < jn; ++jj) a += w[jj] * V[(b * d.N + j0 + jj) * D + k];
            acc[u] = a;
        }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
    {
        const size_t k = threadIdx.x + kThreads * u;
        if (k < D) out[(b * d.M + i) * D + k] = acc[u];
    }
}

// ── batched_matmul_softmax_backward_q ─────────────────────────────────────
//   R_i = sum_j W_ij P_ij;  dQ[k][i] = alpha * sum_j W_ij (P_ij - R_i) B_b(k, j)
__global__ __launch_bounds__(kThreads) void k_bmm_bwd_q(Dims d, const float* P, const float* row_max,
                                                        const float* denom, float* dQ, float* R)
{
    extern __shared__ float q[];   // K floats, then kChunk weights
    __shared__ float scratch[kThreads / 64];
    float* w = q + d.K;
    const size_t b = blockIdx.y, i = blockIdx.x, ri = b * d.M + i;
    for (size_t k = threadIdx.x; k < d.K; k += kThreads) q[k] = a_at(d, b, i, k);
    __syncthreads();
    const float m = row_max[ri], inv_l = 1.0f / denom[ri];
    const float* prow = P + ri * d.N;
    // Pass 1: R.
    float rv = 0.0f;
    for (size_t j = threadIdx.x; j < d.N; j += kThreads)
    {
        const float mv = mask_at(d, i, j);
        if (mv == kNegInf) continue;
        const float wj = expf(d.alpha * score_row(d, q, b, j) + mv - m) * inv_l;
        rv += wj * prow[j];
    }
    rv = block_reduce(rv, R_SUM, scratch);
    if (threadIdx.x == 0) R[ri] = rv;
    // Pass 2: dQ, weights recomputed per chunk.
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};   // k = threadIdx.x + 256*u, K <= 1024
    for (size_t j0 = 0; j0 < d.N; j0 += kChunk)
    {
        const size_t jn = (d.N - j0 < kChunk) ? d.N - j0 : kChunk;
        __syncthreads();
        for (size_t jj = threadIdx.x; jj < jn; jj += kThreads)
        {
            const size_t j = j0 + jj;
            const float mv = mask_at(d, i, j);
            w[jj] = mv == kNegInf ? 0.0f : expf(d.alpha * score_row(d, q, b, j) + mv - m) * inv_l;
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < 4; ++u)
        {
            const size_t k = threadIdx.x + kThreads * u;
            if (k >= d.K) break;
            float a = acc[u];
            for (size_t jj = 0; jj < jn; ++jj)
            {
                const size_t j = j0 + jj;
                a += w[jj] * (prow[j] - rv) * b_at(d, b, k, j);
            }
            acc[u] = a;
        }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
    {
        const size_t k = threadIdx.x + kThreads * u;
        if (k < d.K) dQ[(b * d.K + k) * d.M + i] = d.alpha * acc[u];
    }
}

// ── batched_matmul_softmax_backward_kv: one workgroup per (b, j) ──────────
//   dK[k][j] = alpha * sum_i W_ij (P_ij - R_i) A_b(i, k);  dV[k][j] = sum_i W_ij G[i][k]
__global__ __launch_bounds__(kThreads) void k_bmm_bwd_kv(Dims d, const float* P, const float* G, const float* R,
                                                         const float* row_max, const float* denom, float* dK,
                                                         float* dV, size_t D)
{
    extern __shared__ float kv[];   // K floats, then kChunk weights
    float* w = kv + d.K;
    const size_t b = blockIdx.y, j = blockIdx.x;
    for (size_t k = threadIdx.x; k < d.K; k += kThreads) kv[k] = b_at(d, b, k, j);
    float accK[4] = {0.0f, 0.0f, 0.0f, 0.0f}, accV[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (size_t i0 = 0; i0 < d.M; i0 += kChunk)
    {
        const size_t in = (d.M - i0 < kChunk) ? d.M - i0 : kChunk;
        __syncthreads();
        for (size_t ii = threadIdx.x; ii < in; ii += kThreads)
        {
            const size_t i = i0 + ii, ri = b * d.M + i;
            const float mv = mask_at(d, i, j);
            w[ii] = mv == kNegInf ? 0.0f : expf(d.alpha * score_col(d, kv, b, i) + mv - row_max[ri]) / denom[ri];
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < 4; ++u)
        {
            const size_t k = threadIdx.x + kThreads * u;
            if (k >= d.K) break;
            float ak = accK[u], av = accV[u];
            for (size_t ii = 0; ii < in; ++ii)
            {
                const size_t i = i0 + ii, ri = b * d.M + i;
                ak += w[ii] * (P[ri * d.N + j] - R[ri]) * a_at(d, b, i, k);
                av += w[ii] * G[ri * D + k];
            }
            accK[u] = ak;
            accV[u] = av;
        }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
    {
        const size_t k = threadIdx.x + kThreads * u;
        if (k < d.K)
        {
            dK[(b * d.K + k) * d.N + j] = d.alpha * accK[u];
            dV[(b * d.K + k) * d.N + j] = accV[u];
        }
    }
}

int check_dims(size_t batch, size_t M, size_t N, size_t K)
{
    if (batch > 65535 || M > 0x7fffffff || N > 0x7fffffff) return -1;
    if (K > 1024) return -3;   // this path keeps one operand vector per workgroup in registers / LDS
    return 0;
}

size_t lds_bytes(size_t K, bool chunk) { return (K + (chunk ? kChunk : 0)) * sizeof(float); }

} // namespace
} // namespace nnhip

using namespace nnhip;

extern "C" size_t nnhip_bmm_workspace_bytes(size_t batch, size_t M, size_t N, size_t K, size_t D)
{
    return attn_workspace_bytes(batch, M, N, K, D);
}

namespace
{
AttnArgs attn_args(const float* A, const float* B, const float* mask, size_t M, size_t N, size_t K, int tA, int tB,
                   float alpha)
{
    return AttnArgs{A, B, mask, static_cast<int>(M), static_cast<int>(N), static_cast<int>(K), tA, tB, alpha};
}
} // namespace

extern "C" int nnhip_bmm_reduce(const float* A, const float* B, const float* mask, float* out, size_t batch, size_t M,
                                size_t N, size_t K, int transA, int transB, unsigned op, float alpha, int reduce_cols,
                                void* workspace, void* stream)
{
    if (op > R_MIN) return -1;
    if (batch == 0 || (reduce_cols ? M : N) == 0) return 0;
    auto s = static_cast<hipStream_t>(stream);
    if (op == R_MAX && reduce_cols && workspace && attn_mfma_supported(batch, M, N, K))
        return attn_mfma_forward(attn_args(A, B, mask, M, N, K, transA, transB, alpha), batch, kFwdMax, nullptr,
                                 nullptr, nullptr, 0, out, workspace, s);
    if (int rc = check_dims(batch, M, N, K)) return rc;
    Dims d{A, B, mask, M, N, K, transA, transB, alpha};
    if (reduce_cols)
        hipLaunchKernelGGL(k_bmm_reduce_rows, dim3(static_cast<unsigned>(M), static_cast<unsigned>(batch)),
                           dim3(kThreads), lds_bytes(K, false), s, d, out, op);
    else
        hipLaunchKernelGGL(k_bmm_reduce_cols, dim3(static_cast<unsigned>(N), static_cast<unsigned>(batch)),
                           dim3(kThreads), lds_bytes(K, false), s, d, out, op);
    return launch_status();
}

extern "C" int nnhip_bmm_softmax_denom(const float* A, const float* B, const float* row_max, const float* mask,
                                       float* out, size_t batch, size_t M, size_t N, size_t K, int transA, int transB,
                                       float alpha, void* workspace, void* stream)
{
    if (batch == 0 || M == 0) return 0;
    auto s = static_cast<hipStream_t>(stream);
    if (workspace && attn_mfma_supported(batch, M, N, K))
        return attn_mfma_forward(attn_args(A, B, mask, M, N, K, transA, transB, alpha), batch, kFwdDenom, row_max,
                                 nullptr, nullptr, 0, out, workspace, s);
    if (int rc = check_dims(batch, M, N, K)) return rc;
    Dims d{A, B, mask, M, N, K, transA, transB, alpha};
    hipLaunchKernelGGL(k_bmm_denom, dim3(static_cast<unsigned>(M), static_cast<unsigned>(batch)), dim3(kThreads),
                       lds_bytes(K, false), s, d, row_max, out);
    return launch_status();
}

extern "C" int nnhip_bmm_softmax_apply(const float* A, const float* B, const float* V, const float* row_max,
                                       const float* denom, const float* mask, float* out, size_t batch, size_t M,
                                       size_t N, size_t K, size_t D, int transA, int transB, float alpha,
                                       void* workspace, void* stream)
{
    if (batch == 0 || M == 0 || D == 0) return 0;
    auto s = static_cast<hipStream_t>(stream);
    if (D <= 128 && workspace && attn_mfma_supported(batch, M, N, K))
        return attn_mfma_forward(attn_args(A, B, mask, M, N, K, transA, transB, alpha), batch, kFwdApply, row_max,
                                 denom, V, D, out, workspace, s);
    if (int rc = check_dims(batch, M, N, K)) return rc;
    if (D > 1024) return -3;
    Dims d{A, B, mask, M, N, K, transA, transB, alpha};
    hipLaunchKernelGGL(k_bmm_apply, dim3(static_cast<unsigned>(M), static_cast<unsigned>(batch)), dim3(kThreads),
                       lds_bytes(K, true), s, d, V, row_max, denom, out, D);
    return launch_status();
}

extern "C" int nnhip_bmm_softmax_backward_q(const float* A, const float* B, const float* P, const float* row_max,
                                            const float* denom, const float* mask, float* dQ, float* R, size_t batch,
                                            size_t M, size_t N, size_t K, int transA, int transB, float alpha,
                                            void* workspace, void* stream)
{
    if (batch == 0 || M == 0) return 0;
    auto s = static_cast<hipStream_t>(stream);
    if (workspace && attn_mfma_supported(batch, M, N, K))
        return attn_mfma_backward(attn_args(A, B, mask, M, N, K, transA, transB, alpha), batch, false, P, nullptr, 0,
                                  nullptr, row_max, denom, dQ, R, workspace, s);
    if (int rc = check_dims(batch, M, N, K)) return rc;
    Dims d{A, B, mask, M, N, K, transA, transB, alpha};
    hipLaunchKernelGGL(k_bmm_bwd_q, dim3(static_cast<unsigned>(M), static_cast<unsigned>(batch)), dim3(kThreads),
                       lds_bytes(K, true), s, d, P, row_max, denom, dQ, R);
    return launch_status();
}

extern "C" int nnhip_bmm_softmax_backward_kv(const float* A, const float* B, const float* P, const float* G,
                                             const float* R, const float* row_max, const float* denom,
                                             const float* mask, float* dK, float* dV, size_t batch, size_t M, size_t N,
                                             size_t K, size_t D, int transA, int transB, float alpha, void* workspace,
                                             void* stream)
{
    if (D < K) return -2;
    if (batch == 0 || N == 0) return 0;
    auto s = static_cast<hipStream_t>(stream);
    if (workspace && attn_mfma_supported(batch, M, N, K))
        return attn_mfma_backward(attn_args(A, B, mask, M, N, K, transA, transB, alpha), batch, true, P, G, D, R,
                                  row_max, denom, dK, dV, workspace, s);
    if (int rc = check_dims(batch, M, N, K)) return rc;
    Dims d{A, B, mask, M, N, K, transA, transB, alpha};
    hipLaunchKernelGGL(k_bmm_bwd_kv, dim3(static_cast<unsigned>(N), static_cast<unsigned>(batch)), dim3(kThreads),
                       lds_bytes(K, true), s, d, P, G, R, row_max, denom, dK, dV, D);
    return launch_status();
}
