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

// Merge chunk statistics (one chunk per 256-row block of the logits or of a
// product's statistics); emit per-column max, denominator, validity and loss.
// A workgroup owns 64 columns, its 16 waves merge a sixteenth of the chunks
// each (loads first, then in chunk order), then wave 0 merges the 16 results
// in wave order.
constexpr unsigned kWideWaves = 16, kWideBatch = 8;
__global__ __launch_bounds__(64 * kWideWaves) void k_ce_combine_wide(const float* L, const float* labels,
                                                                     const float* mask, const float* part_m,
                                                                     const float* part_s, float* col_m, float* col_s,
                                                                     float* loss_vec, size_t chunks, size_t C,
                                                                     size_t N, size_t vocab)
{
    __shared__ float sm[kWideWaves][64], ss[kWideWaves][64];
    const unsigned lane = threadIdx.x % 64, wave = threadIdx.x / 64;
    const size_t c = static_cast<size_t>(blockIdx.x) * 64 + lane;
    const size_t per = (chunks + kWideWaves - 1) / kWideWaves, k0 = wave * per,
                 k1 = k0 + per < chunks ? k0 + per : chunks;
    float m = -__builtin_huge_valf(), s = 0.0f;
    if (c < N)
    {
        size_t k = k0;
        for (; k + kWideBatch <= k1; k += kWideBatch)
        {
            float pm[kWideBatch], ps[kWideBatch];
#pragma unroll
            for (unsigned j = 0; j < kWideBatch; ++j)
            {
                pm[j] = part_m[(k + j) * N + c];
                ps[j] = part_s[(k + j) * N + c];
            }
#pragma unroll
            for (unsigned j = 0; j < kWideBatch; ++j) merge(m, s, pm[j], ps[j]);
        }
        for (; k < k1; ++k) merge(m, s, part_m[k * N + c], part_s[k * N + c]);
    }
    sm[wave][lane] = m;
    ss[wave][lane] = s;
    __syncthreads();
    if (wave != 0 || c >= N) return;
    for (unsigned w = 1; w < kWideWaves; ++w) merge(m, s, sm[w][lane], ss[w][lane]);
    const size_t lbl = label_of(labels[c]);
    const bool valid = (!mask || mask[c] >= 0.5f) && lbl < vocab;
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

// ── float4 column kernels (N % 4 == 0, 16-byte aligned rows) ───────────────
// A lane owns 4 consecutive columns, so a wave reads 1 KB of one row per load;
// the 4 waves of a workgroup interleave rows. Per-column state stays in
// registers for the whole row chunk.
constexpr unsigned kGroupRows = 4;    // rows folded into the running (max, sum) at once

__device__ __forceinline__ float& at(float4& v, int e) { return reinterpret_cast<float*>(&v)[e]; }
__device__ __forceinline__ float at(const float4& v, int e) { return reinterpret_cast<const float*>(&v)[e]; }

template <bool GIVEN_MAX>
__global__ __launch_bounds__(kThreads) void k_col_stats4(const float* L, const float* col_max, float* part_m,
                                                         float* part_s, size_t C, size_t N, size_t rows_per_chunk)
{
    __shared__ float4 sm[kWaves][64], ss[kWaves][64];
    const unsigned lane = threadIdx.x % 64, wave = threadIdx.x / 64;
    const size_t N4 = N / 4, c4 = static_cast<size_t>(blockIdx.x) * 64 + lane;
    const size_t r0 = static_cast<size_t>(blockIdx.y) * rows_per_chunk;
    const size_t r1 = r0 + rows_per_chunk < C ? r0 + rows_per_chunk : C;
    const float4* L4 = reinterpret_cast<const float4*>(L);
    constexpr float kNinf = -__builtin_huge_valf();
    float4 m = make_float4(kNinf, kNinf, kNinf, kNinf), sum = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (c4 < N4)
    {
        if constexpr (GIVEN_MAX)
        {
            const float4 mx = reinterpret_cast<const float4*>(col_max)[c4];
            for (size_t r = r0 + wave; r < r1; r += kWaves)
            {
                const float4 x = L4[r * N4 + c4];
#pragma unroll
                for (int e = 0; e < 4; ++e) at(sum, e) += expf(at(x, e) - at(mx, e));
            }
        }
        else
        {
            // kGroupRows rows at a time: one rescale per group instead of a branch per element.
            for (size_t r = r0 + wave; r < r1; r += kWaves * kGroupRows)
            {
                float4 x[kGroupRows];
#pragma unroll
                for (unsigned k = 0; k < kGroupRows; ++k)
                {
                    const size_t rr = r + k * kWaves;
                    x[k] = rr < r1 ? L4[rr * N4 + c4] : make_float4(kNinf, kNinf, kNinf, kNinf);
                }
#pragma unroll
                for (int e = 0; e < 4; ++e)
                {
                    float gm = at(x[0], e);
#pragma unroll
                    for (unsigned k = 1; k < kGroupRows; ++k) gm = fmaxf(gm, at(x[k], e));
                    if (gm > at(m, e))
                    {
                        at(sum, e) *= expf(at(m, e) - gm);
                        at(m, e) = gm;
                    }
                    if (at(m, e) > kNinf)
                    {
#pragma unroll
                        for (unsigned k = 0; k < kGroupRows; ++k) at(sum, e) += expf(at(x[k], e) - at(m, e));
                    }
                }
            }
        }
    }
    sm[wave][lane] = m;
    ss[wave][lane] = sum;
    __syncthreads();
    if (wave == 0 && c4 < N4)
    {
        for (unsigned w = 1; w < kWaves; ++w)
        {
#pragma unroll
            for (int e = 0; e < 4; ++e)
            {
                if constexpr (GIVEN_MAX) at(sum, e) += at(ss[w][lane], e);
                else merge(at(m, e), at(sum, e), at(sm[w][lane], e), at(ss[w][lane], e));
            }
        }
        reinterpret_cast<float4*>(part_s + static_cast<size_t>(blockIdx.y) * N)[c4] = sum;
        if (!GIVEN_MAX) reinterpret_cast<float4*>(part_m + static_cast<size_t>(blockIdx.y) * N)[c4] = m;
    }
}

// Dense gradient of the sparse cross-entropy, a (rows_per_block x 256)-column
// strip per workgroup: per-column max, scale and label held in registers.
__global__ __launch_bounds__(kThreads) void k_ce_grad4(const float* L, const float* labels, const float* col_m,
                                                       const float* col_s, float* grad, size_t C, size_t N,
                                                       float inv, size_t rows_per_block)
{
    const unsigned lane = threadIdx.x % 64, wave = threadIdx.x / 64;
    const size_t N4 = N / 4, c4 = static_cast<size_t>(blockIdx.x) * 64 + lane;
    if (c4 >= N4) return;
    const size_t r0 = static_cast<size_t>(blockIdx.y) * rows_per_block;
    const size_t r1 = r0 + rows_per_block < C ? r0 + rows_per_block : C;
    const float4 m = reinterpret_cast<const float4*>(col_m)[c4], sv = reinterpret_cast<const float4*>(col_s)[c4];
    const float4 lb = reinterpret_cast<const float4*>(labels)[c4];
    float4 f;
    size_t lbl[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
    {
        // s == 0 marks an invalid column (masked or label out of range): all-zero gradient.
        at(f, e) = at(sv, e) != 0.0f ? inv / at(sv, e) : 0.0f;
        lbl[e] = at(sv, e) != 0.0f ? label_of(at(lb, e)) : ~size_t{0};
    }
    // The logits are read once and the gradient written once (each 4 bytes x C x N, far more than the
    // caches hold): non-temporal accesses.
    typedef float f4 __attribute__((ext_vector_type(4)));
    const f4* __restrict__ L4 = reinterpret_cast<const f4*>(L);
    f4* __restrict__ G4 = reinterpret_cast<f4*>(grad);
    auto one = [&](const f4& x, size_t r) {
        f4 gv;
#pragma unroll
        for (int e = 0; e < 4; ++e)
        {
            float gg = at(f, e) * __expf(x[e] - at(m, e));
            if (lbl[e] == r) gg -= inv;
            gv[e] = gg;
        }
        __builtin_nontemporal_store(gv, G4 + r * N4 + c4);
    };
    constexpr unsigned kBatch = 4;   // rows whose loads are in flight together
    size_t r = r0 + wave;
    for (; r + (kBatch - 1) * kWaves < r1; r += kBatch * kWaves)
    {
        f4 x[kBatch];
#pragma unroll
        for (unsigned k = 0; k < kBatch; ++k) x[k] = __builtin_nontemporal_load(L4 + (r + k * kWaves) * N4 + c4);
#pragma unroll
        for (unsigned k = 0; k < kBatch; ++k) one(x[k], r + k * kWaves);
    }
    for (; r < r1; r += kWaves) one(__builtin_nontemporal_load(L4 + r * N4 + c4), r);
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
        v[u] = x[c < cols ? c : cols - 1];
    }
#pragma unroll
    for (unsigned u = 0; u < kRowPer; ++u)
        if (threadIdx.x + u * kThreads < cols) m = fmax_std(m, v[u]);
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

// One wave per row for rows of cols % 4 == 0 (16-byte aligned), cols <= 256 * NV:
// the row sits in registers as NV float4 per lane, max and sum are wave
// reductions, 4 rows per workgroup, no barriers.
template <int NV>
__global__ __launch_bounds__(kThreads) void k_row_softmax_wave(const float* X, float* out, size_t rows, size_t cols)
{
    const size_t row = static_cast<size_t>(blockIdx.x) * kWaves + threadIdx.x / 64;
    if (row >= rows) return;
    const unsigned lane = threadIdx.x % 64;
    const size_t nq = cols / 4;
    const float4* x = reinterpret_cast<const float4*>(X + row * cols);
    float4* o = reinterpret_cast<float4*>(out + row * cols);
    float4 v[NV];
    float m = kLowest;
    // Unconditional loads (index clamped into the row) so that all NV are in flight at once.
#pragma unroll
    for (int u = 0; u < NV; ++u)
    {
        const size_t q = lane + 64 * u;
        v[u] = x[q < nq ? q : nq - 1];
    }
#pragma unroll
    for (int u = 0; u < NV; ++u)
        if (lane + 64 * u < nq) m = fmax_std(fmax_std(fmax_std(fmax_std(m, v[u].x), v[u].y), v[u].z), v[u].w);
    m = wave_max(m);
    float sum = 0.0f;
#pragma unroll
    for (int u = 0; u < NV; ++u)
    {
        const size_t q = lane + 64 * u;
        if (q < nq)
        {
            v[u].x = expf(v[u].x - m);
            v[u].y = expf(v[u].y - m);
            v[u].z = expf(v[u].z - m);
            v[u].w = expf(v[u].w - m);
            sum += (v[u].x + v[u].y) + (v[u].z + v[u].w);
        }
    }
    sum = wave_sum(sum);
#pragma unroll
    for (int u = 0; u < NV; ++u)
    {
        const size_t q = lane + 64 * u;
        if (q < nq) o[q] = make_float4(v[u].x / sum, v[u].y / sum, v[u].z / sum, v[u].w / sum);
    }
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

namespace
{
// Column plan of the float4 kernels: 256 columns per workgroup.
ColPlan col_plan4(size_t C, size_t N)
{
    ColPlan p;
    p.col_blocks = (N / 4 + 63) / 64;
    size_t chunks = 2048 / (p.col_blocks ? p.col_blocks : 1);
    const size_t max_chunks = (C + 63) / 64;   // at least 64 rows per chunk
    if (chunks > max_chunks) chunks = max_chunks;
    if (chunks < 1) chunks = 1;
    p.rows_per_chunk = (C + chunks - 1) / chunks;
    if (p.rows_per_chunk == 0) p.rows_per_chunk = 1;
    p.chunks = (C + p.rows_per_chunk - 1) / p.rows_per_chunk;
    return p;
}
bool cols4_ok(const float* L, size_t N) { return N % 4 == 0 && aligned16(L); }
} // namespace

extern "C" size_t nnhip_col_softmax_workspace_bytes(size_t C, size_t N)
{
    const ColPlan p = col_plan(C, N), p4 = col_plan4(C, N);
    const size_t chunks = p.chunks > p4.chunks ? p.chunks : p4.chunks;
    return (2 * chunks + 2) * N * sizeof(float) + 256;
}

extern "C" int nnhip_col_softmax_denom(const float* logits, const float* col_max, float* out, size_t C, size_t N,
                                       void* workspace, void* stream)
{
    if (N == 0) return 0;
    if (C == 0) return nnhip_fill(out, N, 0.0f, stream);
    auto s = static_cast<hipStream_t>(stream);
    const bool v4 = cols4_ok(logits, N) && aligned16(col_max) && aligned16(workspace) && aligned16(out);
    const ColPlan p = v4 ? col_plan4(C, N) : col_plan(C, N);
    float* ps = static_cast<float*>(workspace);
    if (v4)
        hipLaunchKernelGGL(k_col_stats4<true>, dim3(static_cast<unsigned>(p.col_blocks), static_cast<unsigned>(p.chunks)),
                           dim3(kThreads), 0, s, logits, col_max, nullptr, ps, C, N, p.rows_per_chunk);
    else
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
    const bool v4 = cols4_ok(logits, N) && aligned16(labels) && aligned16(workspace) && aligned16(grad);
    const ColPlan p = v4 ? col_plan4(C, N) : col_plan(C, N);
    float* pm = static_cast<float*>(workspace);
    float* ps = pm + p.chunks * N;
    float* cm = ps + p.chunks * N;
    float* cs = cm + N;
    if (v4)
        hipLaunchKernelGGL(k_col_stats4<false>, dim3(static_cast<unsigned>(p.col_blocks), static_cast<unsigned>(p.chunks)),
                           dim3(kThreads), 0, s, logits, nullptr, pm, ps, C, N, p.rows_per_chunk);
    else
        hipLaunchKernelGGL(k_col_stats<false>, dim3(static_cast<unsigned>(p.col_blocks), static_cast<unsigned>(p.chunks)),
                           dim3(kThreads), 0, s, logits, nullptr, pm, ps, C, N, p.rows_per_chunk);
    hipLaunchKernelGGL(k_ce_combine_wide, dim3(static_cast<unsigned>((N + 63) / 64)), dim3(64 * kWideWaves), 0, s, logits,
                       labels, mask, pm, ps, cm, cs, loss_vec, p.chunks, C, N, vocab_size);
    if (v4)
    {
        const size_t rows_per_block = 64, col_blocks = (N / 4 + 63) / 64;
        const size_t row_blocks = (C + rows_per_block - 1) / rows_per_block;
        if (row_blocks > 65535) return -3;
        hipLaunchKernelGGL(k_ce_grad4, dim3(static_cast<unsigned>(col_blocks), static_cast<unsigned>(row_blocks)),
                           dim3(kThreads), 0, s, logits, labels, cm, cs, grad, C, N, inv_num_valid, rows_per_block);
    }
    else
        hipLaunchKernelGGL(k_ce_grad, dim3(grid_for(C * N, kThreads, 256 * 64)), dim3(kThreads), 0, s, logits, labels,
                           cm, cs, grad, C, N, inv_num_valid);
    return launch_status();
}

extern "C" int nnhip_col_softmax_sparse_from_stats(const float* logits, const float* labels, const float* mask,
                                                   const float* stats, size_t tiles, float* grad, float* loss_vec,
                                                   size_t C, size_t N, size_t vocab_size, float inv_num_valid,
                                                   void* workspace, void* stream)
{
    if (vocab_size > (size_t{1} << 24) || vocab_size > C) return -2;
    if (N == 0) return 0;
    if (C == 0 || tiles == 0 || !stats || !workspace) return -1;
    auto s = static_cast<hipStream_t>(stream);
    float* cm = static_cast<float*>(workspace);
    float* cs = cm + N;
    hipLaunchKernelGGL(k_ce_combine_wide, dim3(static_cast<unsigned>((N + 63) / 64)), dim3(64 * kWideWaves), 0, s, logits,
                       labels, mask, stats, stats + tiles * N, cm, cs, loss_vec, tiles, C, N, vocab_size);
    const bool v4 = cols4_ok(logits, N) && aligned16(labels) && aligned16(workspace) && aligned16(grad);
    if (v4)
    {
        const size_t rows_per_block = 64, col_blocks = (N / 4 + 63) / 64;
        const size_t row_blocks = (C + rows_per_block - 1) / rows_per_block;
        if (row_blocks > 65535) return -3;
        hipLaunchKernelGGL(k_ce_grad4, dim3(static_cast<unsigned>(col_blocks), static_cast<unsigned>(row_blocks)),
                           dim3(kThreads), 0, s, logits, labels, cm, cs, grad, C, N, inv_num_valid, rows_per_block);
    }
    else
        hipLaunchKernelGGL(k_ce_grad, dim3(grid_for(C * N, kThreads, 256 * 64)), dim3(kThreads), 0, s, logits, labels,
                           cm, cs, grad, C, N, inv_num_valid);
    return launch_status();
}

extern "C" int nnhip_row_softmax(const float* X, float* out, size_t rows, size_t cols, void* stream)
{
    if (rows == 0 || cols == 0) return 0;
    if (rows > 0x7fffffff) return -1;
    auto s = static_cast<hipStream_t>(stream);
    if (cols % 4 == 0 && cols <= 4096 && aligned16(X) && aligned16(out))
    {
        const unsigned grid = static_cast<unsigned>((rows + kWaves - 1) / kWaves);
        if (cols <= 256) hipLaunchKernelGGL(k_row_softmax_wave<1>, dim3(grid), dim3(kThreads), 0, s, X, out, rows, cols);
        else if (cols <= 512) hipLaunchKernelGGL(k_row_softmax_wave<2>, dim3(grid), dim3(kThreads), 0, s, X, out, rows, cols);
        else if (cols <= 1024) hipLaunchKernelGGL(k_row_softmax_wave<4>, dim3(grid), dim3(kThreads), 0, s, X, out, rows, cols);
        else if (cols <= 2048) hipLaunchKernelGGL(k_row_softmax_wave<8>, dim3(grid), dim3(kThreads), 0, s, X, out, rows, cols);
        else hipLaunchKernelGGL(k_row_softmax_wave<16>, dim3(grid), dim3(kThreads), 0, s, X, out, rows, cols);
    }
    else if (cols <= kRowPer * kThreads)
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
