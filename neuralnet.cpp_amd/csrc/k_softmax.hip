// k_softmax.hip — column softmax statistics, fused sparse cross-entropy and
// the fused row softmax (forward / backward) of the Softmax layer.
//
// Column kernels (ComputeEngine::col_softmax_denom / col_softmax_sparse_forward,
// cpu_engine.hpp:922-1006): logits are (C, N), one column per token. Lanes own
// columns, so every row is read as a coalesced 256-byte segment per wave.
// The row range is split into chunks that each produce a running
// (max, sum of exp) pair per column; the chunk pairs are merged in chunk
// order, then a second streaming pass writes the dense gradient
//   grad[r][i] = inv * exp(L[r][i] - max_i) / denom_i  - [r == label_i] * inv
// and loss_vec[i] = L[label_i][i] - max_i - log(denom_i), zeros for columns that
// are masked (mask < 0.5) or carry a label >= vocab_size.
//
// Row softmax (Softmax::forward/backward, compute_layer.hpp:832-862, which
// reach the engine as eval_expr programs): one workgroup per row keeps the
// row in registers: one read, one write.
#include "common.hpp"
#include "nnhip_kernels.h"

namespace nnhip
{
namespace
{

constexpr unsigned kThreads = 256;
constexpr unsigned kCols = 64;              // columns per workgroup (one per lane)
constexpr unsigned kWaves = kThreads / 64;  // row interleave inside a workgroup

struct ColPlan
{
    size_t col_blocks, chunks, rows_per_chunk;
};
ColPlan col_plan(size_t C, size_t N)
{
    ColPlan p;
    p.col_blocks = (N + kCols - 1) / kCols;
    size_t chunks = 2048 / (p.col_blocks ? p.col_blocks : 1);
    const size_t max_chunks = (C + 63) / 64;   // at least 64 rows per chunk
    if (chunks > max_chunks) chunks = max_chunks;
    if (chunks < 1) chunks = 1;
    p.rows_per_chunk = (C + chunks - 1) / chunks;
    if (p.rows_per_chunk == 0) p.rows_per_chunk = 1;
    p.chunks = (C + p.rows_per_chunk - 1) / p.rows_per_chunk;
    if (p.chunks < 1) p.chunks = 1;
    return p;
}

// Online merge of (m, s) pairs: s is the sum of exp(x - m).
__device__ __forceinline__ void merge(float& m, float& s, float m2, float s2)
{
    if (m2 > m)
    {
        s = s * expf(m - m2) + s2;
        m = m2;
    }
    else if (m2 > -__builtin_huge_valf())
    {
        s = s + s2 * expf(m2 - m);
    }
}

// Partial statistics over one row chunk. With col_max given, only the sum of
// exp(x - col_max) is accumulated (col_softmax_denom); otherwise the running
// (max, sum) pair (sparse cross-entropy).
template <bool GIVEN_MAX>
__global__ __launch_bounds__(kThreads) void k_col_stats(const float* L, const float* col_max, float* part_m,
                                                        float* part_s, size_t C, size_t N, size_t rows_per_chunk)
{
    __shared__ float sm[kWaves][kCols], ss[kWaves][kCols];
    const unsigned lane = threadIdx.x % 64, wave = threadIdx.x / 64;
    const size_t c = static_cast<size_t>(blockIdx.x) * kCols + lane;
    const size_t r0 = static_cast<size_t>(blockIdx.y) * rows_per_chunk;
    size_t r1 = r0 + rows_per_chunk;
    if (r1 > C) r1 = C;
    float m = -__builtin_huge_valf(), s = 0.0f;
    if (c < N)
    {
        if constexpr (GIVEN_MAX)
        {
            const float mx = col_max[c];
            for (size_t r = r0 + wave; r < r1; r += kWaves) s += expf(L[r * N + c] - mx);
        }
        else
        {
            for (size_t r = r0 + wave; r < r1; r += kWaves)
            {
                const float x = L[r * N + c];
                if (x > m)
                {
                    s = s * expf(m - x) + 1.0f;
                    m = x;
                }
                else
                {
                    s += expf(x - m);
                }
            }
        }
    }
    sm[wave][lane] = m;
    ss[wave][lane] = s;
    __syncthreads();
    if (wave == 0 && c < N)
    {
        for (unsigned w = 1; w < kWaves; ++w)
        {
            if constexpr (GIVEN_MAX) s += ss[w][lane];
            else merge(m, s, sm[w][lane], ss[w][lane]);
        }
        part_s[static_cast<size_t>(blockIdx.y) * N + c] = s;
        if (!GIVEN_MAX) part_m[static_cast<size_t>(blockIdx.y) * N + c] = m;
    }
}

__global__ __launch_bounds__(kThreads) void k_col_denom_combine(const float* part_s, float* out, size_t chunks,
                                                                size_t N)
{
    const size_t c = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (c >= N) return;
    float s = part_s[c];
    for (size_t k = 1; k < chunks; ++k) s += part_s[k * N + c];
    out[c] = s;
}

__device__ __forceinline__ size_t label_of(float f)
{
    // (lbl_f >= 0) ? size_t(lbl_f) : 0, as cpu_engine.hpp:979-981
    if (f >= 0.0f) return f < 1.8446744e19f ? static_cast<size_t>(f) : ~size_t{0};
    return 0;
}

// Merge chunk statistics; emit per-column max, denominator, validity and loss.
__global__ __launch_bounds__(kThreads) void k_ce_combine(const float* L, const float* labels, const float* mask,
                                                         const float* part_m, const float* part_s, float* col_m,
                                                         float* col_s, float* loss_vec, size_t chunks, size_t C,
                                                         size_t N, size_t vocab)
{
    const size_t c = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (c >= N) return;
    const size_t lbl = label_of(labels[c]);
    const bool valid = (!mask || mask[c] >= 0.5f) && lbl < vocab;
    float m = part_m[c], s = part_s[c];
    for (size_t k = 1; k < chunks; ++k) merge(m, s, part_m[k * N + c], part_s[k * N + c]);
    col_m[c] = m;
    col_s[c] = valid ? s : 0.0f;   // 0 marks an invalid column for the gradient pass
    loss_vec[c] = valid ? L[lbl * N + c] - m - logf(s) : 0.0f;
}

__global__ __launch_bounds__(kThreads) void k_ce_grad(const float* L, const float* labels, const float* col_m,
                                                      const float* col_s, float* grad, size_t C, size_t N,
                                                      float inv)
{
    const size_t total = C * N;
    const size_t stride = static_cast<size_t>(gridDim.x) * kThreads;
    for (size_t e = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x; e < total; e += stride)
    {
        const size_t r = e / N, c = e % N;
        const float s = col_s[c];
        float g = 0.0f;
        if (s != 0.0f)
        {
            g = inv * expf(L[e] - col_m[c]) / s;
            if (label_of(labels[c]) == r) g -= inv;
        }
        grad[e] = g;
    }
}

// ── row softmax ─────────────────────────────────────────────────────────────
constexpr unsigned kRowPer = 16;   // values per lane kept in registers: rows up to 4096 wide

__device__ float block_max(float v, float* scratch)
{
    v = wave_max(v);
    const unsigned lane = threadIdx.x % 64, wave = threadIdx.x / 64;
    __syncthreads();
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    float t = scratch[0];
    for (unsigned w = 1; w < kWaves; ++w) t = fmax_std(t, scratch[w]);
    return t;
}
__device__ float block_sum(float v, float* scratch)
{
    v = wave_sum(v);
    const unsigned lane = threadIdx.x % 64, wave = threadIdx.x / 64;
    __syncthreads();
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    float t = scratch[0];
    for (unsigned w = 1; w < kWaves; ++w) t += scratch[w];
    return t;
}

// out = exp(x - max) / sum(exp(x - max)); max starts at lowest().
__global__ __launch_bounds__(kThreads) void k_row_softmax_reg(const float* X, float* out, size_t cols)
{
    __shared__ float scratch[kWaves];
    const float* x = X + static_cast<size_t>(blockIdx.x) * cols;
    float* o = out + static_cast<size_t>(blockIdx.x) * cols;
    float v[kRowPer];
    float m = kLowest;
#pragma unroll
    for (unsigned u = 0; u < kRowPer; ++u)
    {
        const size_t c = threadIdx.x + u * kThreads;
        v[u] = c < cols ? x[c] : 0.0f;
        if (c < cols) m = fmax_std(m, v[u]);
    }
    m = block_max(m, scratch);
    float s = 0.0f;
#pragma unroll
    for (unsigned u = 0; u < kRowPer; ++u)
    {
        const size_t c = threadIdx.x + u * kThreads;
        v[u] = expf(v[u] - m);
        if (c < cols) s += v[u];
    }
    s = block_sum(s, scratch);
#pragma unroll
    for (unsigned u = 0; u < kRowPer; ++u)
    {
        const size_t c = threadIdx.x + u * kThreads;
        if (c < cols) o[c] = v[u] / s;
    }
}

__global__ __launch_bounds__(kThreads) void k_row_softmax_stream(const float* X, float* out, size_t cols)
{
    __shared__ float scratch[kWaves];
    const float* x = X + static_cast<size_t>(blockIdx.x) * cols;
    float* o = out + static_cast<size_t>(blockIdx.x) * cols;
    float m = kLowest;
    for (size_t c = threadIdx.x; c < cols; c += kThreads) m = fmax_std(m, x[c]);
    m = block_max(m, scratch);
    float s = 0.0f;
    for (size_t c = threadIdx.x; c < cols; c += kThreads) s += expf(x[c] - m);
    s = block_sum(s, scratch);
    for (size_t c = threadIdx.x; c < cols; c += kThreads) o[c] = expf(x[c] - m) / s;
}

// dx = y * (g - sum(y * g))
__global__ __launch_bounds__(kThreads) void k_row_softmax_bwd_reg(const float* Y, const float* G, float* out,
                                                                  size_t cols)
{
    __shared__ float scratch[kWaves];
    const size_t base = static_cast<size_t>(blockIdx.x) * cols;
    float y[kRowPer], g[kRowPer];
    float d = 0.0f;
#pragma unroll
    for (unsigned u = 0; u < kRowPer; ++u)
    {
        const size_t c = threadIdx.x + u * kThreads;
        y[u] = c < cols ? Y[base + c] : 0.0f;
        g[u] = c < cols ? G[base + c] : 0.0f;
        d += y[u] * g[u];
    }
    d = block_sum(d, scratch);
#pragma unroll
    for (unsigned u = 0; u < kRowPer; ++u)
    {
        const size_t c = threadIdx.x + u * kThreads;
        if (c < cols) out[base + c] = y[u] * (g[u] - d);
    }
}

__global__ __launch_bounds__(kThreads) void k_row_softmax_bwd_stream(const float* Y, const float* G, float* out,
                                                                     size_t cols)
{
    __shared__ float scratch[kWaves];
    const size_t base = static_cast<size_t>(blockIdx.x) * cols;
    float d = 0.0f;
    for (size_t c = threadIdx.x; c < cols; c += kThreads) d += Y[base + c] * G[base + c];
    d = block_sum(d, scratch);
    for (size_t c = threadIdx.x; c < cols; c += kThreads) out[base + c] = Y[base + c] * (G[base + c] - d);
}

} // namespace
} // namespace nnhip

using namespace nnhip;

extern "C" size_t nnhip_col_softmax_workspace_bytes(size_t C, size_t N)
{
    const ColPlan p = col_plan(C, N);
    return (2 * p.chunks + 2) * N * sizeof(float);
}

extern "C" int nnhip_col_softmax_denom(const float* logits, const float* col_max, float* out, size_t C, size_t N,
                                       void* workspace, void* stream)
{
    if (N == 0) return 0;
    if (C == 0) return nnhip_fill(out, N, 0.0f, stream);
    auto s = static_cast<hipStream_t>(stream);
    const ColPlan p = col_plan(C, N);
    float* ps = static_cast<float*>(workspace);
    hipLaunchKernelGGL(k_col_stats<true>, dim3(static_cast<unsigned>(p.col_blocks), static_cast<unsigned>(p.chunks)),
                       dim3(kThreads), 0, s, logits, col_max, nullptr, ps, C, N, p.rows_per_chunk);
    hipLaunchKernelGGL(k_col_denom_combine, dim3(grid_for(N, kThreads, 1u << 30)), dim3(kThreads), 0, s, ps, out,
                       p.chunks, N);
    return launch_status();
}

extern "C" int nnhip_col_softmax_sparse_forward(const float* logits, const float* labels, const float* mask,
                                                float* grad, float* loss_vec, size_t C, size_t N, size_t vocab_size,
                                                float inv_num_valid, void* workspace, void* stream)
{
    if (vocab_size > (size_t{1} << 24) || vocab_size > C) return -2;
    if (N == 0) return 0;
    auto s = static_cast<hipStream_t>(stream);
    if (C == 0) return nnhip_fill(loss_vec, N, 0.0f, stream);
    const ColPlan p = col_plan(C, N);
    float* pm = static_cast<float*>(workspace);
    float* ps = pm + p.chunks * N;
    float* cm = ps + p.chunks * N;
    float* cs = cm + N;
    hipLaunchKernelGGL(k_col_stats<false>, dim3(static_cast<unsigned>(p.col_blocks), static_cast<unsigned>(p.chunks)),
                       dim3(kThreads), 0, s, logits, nullptr, pm, ps, C, N, p.rows_per_chunk);
    hipLaunchKernelGGL(k_ce_combine, dim3(grid_for(N, kThreads, 1u << 30)), dim3(kThreads), 0, s, logits, labels, mask,
                       pm, ps, cm, cs, loss_vec, p.chunks, C, N, vocab_size);
    hipLaunchKernelGGL(k_ce_grad, dim3(grid_for(C * N, kThreads, 256 * 64)), dim3(kThreads), 0, s, logits, labels, cm,
                       cs, grad, C, N, inv_num_valid);
    return launch_status();
}

extern "C" int nnhip_row_softmax(const float* X, float* out, size_t rows, size_t cols, void* stream)
{
    if (rows == 0 || cols == 0) return 0;
    if (rows > 0x7fffffff) return -1;
    auto s = static_cast<hipStream_t>(stream);
    if (cols <= kRowPer * kThreads)
        hipLaunchKernelGGL(k_row_softmax_reg, dim3(static_cast<unsigned>(rows)), dim3(kThreads), 0, s, X, out, cols);
    else
        hipLaunchKernelGGL(k_row_softmax_stream, dim3(static_cast<unsigned>(rows)), dim3(kThreads), 0, s, X, out, cols);
    return launch_status();
}

extern "C" int nnhip_row_softmax_backward(const float* Y, const float* G, float* out, size_t rows, size_t cols,
                                          void* stream)
{
    if (rows == 0 || cols == 0) return 0;
    if (rows > 0x7fffffff) return -1;
    auto s = static_cast<hipStream_t>(stream);
    if (cols <= kRowPer * kThreads)
        hipLaunchKernelGGL(k_row_softmax_bwd_reg, dim3(static_cast<unsigned>(rows)), dim3(kThreads), 0, s, Y, G, out,
                           cols);
    else
        hipLaunchKernelGGL(k_row_softmax_bwd_stream, dim3(static_cast<unsigned>(rows)), dim3(kThreads), 0, s, Y, G, out,
                           cols);
    return launch_status();
}
