// k_reduce.hip — row and column reductions (sum / max).
//
// Semantics: ComputeEngine::row_reduce_* / col_reduce_* (cpu_engine.hpp:1050-1086);
// max starts from lowest(), sum from 0. Row reductions put one thread, one
// wave or one workgroup on a row depending on its length; column
// reductions stream rows coalesced across lanes (one lane per column) over
// row chunks, then combine the chunk partials in chunk order, so results
// are deterministic run to run.
#include "common.hpp"
#include "nnhip_kernels.h"

namespace nnhip
{
namespace
{

constexpr unsigned kThreads = 256;

__device__ __forceinline__ float combine(unsigned mode, float a, float b) { return mode ? fmax_std(a, b) : a + b; }

// The row kernels write out[r] = result, or with `add` out[r] = out[r] + sum
// (add_inplace of the sums, rounded as that separate call rounds).
__device__ __forceinline__ void put(float* out, size_t r, float v, bool add) { out[r] = add ? out[r] + v : v; }

// cols <= 32: one thread per row, serial along the row.
__global__ __launch_bounds__(kThreads) void k_row_thread(const float* A, float* out, size_t rows, size_t cols,
                                                         unsigned mode, bool add)
{
    const size_t r = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (r >= rows) return;
    float acc = mode ? kLowest : 0.0f;
    for (size_t c = 0; c < cols; ++c) acc = combine(mode, acc, A[r * cols + c]);
    put(out, r, acc, add);
}

// cols <= 4096: one wave per row (4 rows per workgroup).
__global__ __launch_bounds__(kThreads) void k_row_wave(const float* A, float* out, size_t rows, size_t cols,
                                                       unsigned mode, bool add)
{
    const size_t r = static_cast<size_t>(blockIdx.x) * 4 + threadIdx.x / 64;
    if (r >= rows) return;
    const unsigned lane = threadIdx.x % 64;
    float acc = mode ? kLowest : 0.0f;
    const float* row = A + r * cols;
    for (size_t c = lane; c < cols; c += 64) acc = combine(mode, acc, row[c]);
    acc = mode ? wave_max(acc) : wave_sum(acc);
    if (lane == 0) put(out, r, acc, add);
}

// long rows: one workgroup per row.
__global__ __launch_bounds__(kThreads) void k_row_block(const float* A, float* out, size_t rows, size_t cols,
                                                        unsigned mode, bool add)
{
    __shared__ float part[kThreads / 64];
    const size_t r = blockIdx.x;
    const float* row = A + r * cols;
    float acc = mode ? kLowest : 0.0f;
    if ((cols % 4) == 0 && (reinterpret_cast<uintptr_t>(row) & 15u) == 0)
    {
        // Eight float4 loads in flight per thread (a 8192-wide row is one
        // batch), then added in column order.
        const float4* r4 = reinterpret_cast<const float4*>(row);
        const size_t n4 = cols / 4;
        constexpr unsigned kBatch = 8;
        size_t c = threadIdx.x;
        for (; c + (kBatch - 1) * kThreads < n4; c += kBatch * kThreads)
        {
            float4 v[kBatch];
#pragma unroll
            for (unsigned k = 0; k < kBatch; ++k) v[k] = r4[c + k * kThreads];
#pragma unroll
            for (unsigned k = 0; k < kBatch; ++k)
            {
                acc = combine(mode, acc, v[k].x);
                acc = combine(mode, acc, v[k].y);
                acc = combine(mode, acc, v[k].z);
                acc = combine(mode, acc, v[k].w);
            }
        }
        for (; c < n4; c += kThreads)
        {
            const float4 v = r4[c];
            acc = combine(mode, acc, v.x);
            acc = combine(mode, acc, v.y);
            acc = combine(mode, acc, v.z);
            acc = combine(mode, acc, v.w);
        }
    }
    else
    {
        for (size_t c = threadIdx.x; c < cols; c += kThreads) acc = combine(mode, acc, row[c]);
    }
    acc = mode ? wave_max(acc) : wave_sum(acc);
    if (threadIdx.x % 64 == 0) part[threadIdx.x / 64] = acc;
    __syncthreads();
    if (threadIdx.x == 0)
    {
        float t = part[0];
        for (unsigned w = 1; w < kThreads / 64; ++w) t = combine(mode, t, part[w]);
        put(out, r, t, add);
    }
}

struct ColPlan
{
    size_t col_blocks, chunks, rows_per_chunk;
};
ColPlan col_plan(size_t rows, size_t cols)
{
    ColPlan p;
    p.col_blocks = (cols + kThreads - 1) / kThreads;
    size_t chunks = 2048 / (p.col_blocks ? p.col_blocks : 1);
    const size_t max_chunks = (rows + 15) / 16;   // at least 16 rows per chunk
    if (chunks > max_chunks) chunks = max_chunks;
    if (chunks < 1) chunks = 1;
    p.rows_per_chunk = (rows + chunks - 1) / chunks;
    p.chunks = p.rows_per_chunk ? (rows + p.rows_per_chunk - 1) / p.rows_per_chunk : 1;
    if (p.chunks < 1) p.chunks = 1;
    return p;
}

__global__ __launch_bounds__(kThreads) void k_col_partial(const float* A, float* part, size_t rows, size_t cols,
                                                          size_t rows_per_chunk, unsigned mode)
{
    const size_t c = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (c >= cols) return;
    const size_t r0 = static_cast<size_t>(blockIdx.y) * rows_per_chunk;
    size_t r1 = r0 + rows_per_chunk;
    if (r1 > rows) r1 = rows;
    float acc = mode ? kLowest : 0.0f;
    for (size_t r = r0; r < r1; ++r) acc = combine(mode, acc, A[r * cols + c]);
    part[static_cast<size_t>(blockIdx.y) * cols + c] = acc;
}

__global__ __launch_bounds__(kThreads) void k_col_combine(const float* part, float* out, size_t chunks, size_t cols,
                                                          unsigned mode)
{
    const size_t c = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (c >= cols) return;
    float acc = part[c];
    for (size_t k = 1; k < chunks; ++k) acc = combine(mode, acc, part[k * cols + c]);
    out[c] = acc;
}

} // namespace
} // namespace nnhip

using namespace nnhip;

namespace
{
int reduce_row(const float* A, float* out, size_t rows, size_t cols, unsigned mode, bool add, void* stream)
{
    if (mode > 1) return -1;
    if (rows == 0) return 0;
    auto s = static_cast<hipStream_t>(stream);
    if (cols <= 32)
        hipLaunchKernelGGL(k_row_thread, dim3(grid_for(rows, kThreads, 1u << 30)), dim3(kThreads), 0, s, A, out, rows,
                           cols, mode, add);
    else if (cols <= 4096)
        hipLaunchKernelGGL(k_row_wave, dim3(grid_for(rows, 4, 1u << 30)), dim3(kThreads), 0, s, A, out, rows, cols,
                           mode, add);
    else
        hipLaunchKernelGGL(k_row_block, dim3(static_cast<unsigned>(rows)), dim3(kThreads), 0, s, A, out, rows, cols,
                           mode, add);
    return launch_status();
}
} // namespace

extern "C" int nnhip_reduce_row(const float* A, float* out, size_t rows, size_t cols, unsigned mode, void* stream)
{
    return reduce_row(A, out, rows, cols, mode, false, stream);
}

extern "C" int nnhip_reduce_row_sum_add(const float* A, float* out, size_t rows, size_t cols, void* stream)
{
    return reduce_row(A, out, rows, cols, 0u, true, stream);
}

extern "C" size_t nnhip_reduce_col_workspace_bytes(size_t rows, size_t cols)
{
    const ColPlan p = col_plan(rows, cols);
    return p.chunks * cols * sizeof(float);
}

extern "C" int nnhip_reduce_col(const float* A, float* out, size_t rows, size_t cols, unsigned mode, void* workspace,
                                void* stream)
{
    if (mode > 1) return -1;
    if (cols == 0) return 0;
    auto s = static_cast<hipStream_t>(stream);
    if (rows == 0) return nnhip_fill(out, cols, mode ? kLowest : 0.0f, stream);
    const ColPlan p = col_plan(rows, cols);
    float* part = static_cast<float*>(workspace);
    hipLaunchKernelGGL(k_col_partial, dim3(static_cast<unsigned>(p.col_blocks), static_cast<unsigned>(p.chunks)),
                       dim3(kThreads), 0, s, A, part, rows, cols, p.rows_per_chunk, mode);
    hipLaunchKernelGGL(k_col_combine, dim3(static_cast<unsigned>(p.col_blocks)), dim3(kThreads), 0, s, part, out,
                       p.chunks, cols, mode);
    return launch_status();
}
