// k_layout.hip — transpose, rearrange_3d, gather and ordered scatter-add.
//
// Semantics: cpu_engine.hpp:125-179 (gather_rows), :184-216 (scatter_add_rows),
// :226-279 (rearrange_3d), :282-287 (transpose). All index work is exact.
//
// scatter_add reproduces the CPU engine's serial loop bit for bit: each
// destination row receives its gradient rows in increasing i order starting
// from its current value. Valid (row, i) pairs are packed into 64-bit keys
// (row << 32 | i), sorted (bitonic; keys are unique, so the sort is in effect
// stable), and one workgroup per run of equal rows accumulates the run
// sequentially per column. No float atomics are involved.
#include "common.hpp"
#include "nnhip_kernels.h"

namespace nnhip
{
namespace
{

constexpr unsigned kThreads = 256;

// ── transpose: 64x64 tiles through LDS (+1 column of padding) ──────────────
// blockIdx.z picks one of a batch of (R, C) matrices stored back to back.
__global__ __launch_bounds__(256) void k_transpose(const float* A, float* out, size_t R, size_t C)
{
    __shared__ float tile[64][65];
    A += static_cast<size_t>(blockIdx.z) * R * C;
    out += static_cast<size_t>(blockIdx.z) * R * C;
    const size_t r0 = static_cast<size_t>(blockIdx.y) * 64, c0 = static_cast<size_t>(blockIdx.x) * 64;
    const unsigned tx = threadIdx.x % 64, ty = threadIdx.x / 64;   // 64 x 4
    for (unsigned k = ty; k < 64; k += 4)
    {
        const size_t r = r0 + k, c = c0 + tx;
        if (r < R && c < C) tile[k][tx] = A[r * C + c];
    }
    __syncthreads();
    for (unsigned k = ty; k < 64; k += 4)
    {
        const size_t c = c0 + k, r = r0 + tx;   // out (C, R): row c, column r
        if (c < C && r < R) out[c * R + r] = tile[tx][k];
    }
}

// 64x64 tile per workgroup with 16-byte accesses on both sides (R, C multiples
// of 4, 16-byte aligned): 16 threads cover a 256-byte row segment of A on the
// way in and of out on the way out; the padded LDS tile turns the tile.
__global__ __launch_bounds__(256) void k_transpose4(const float* A, float* out, size_t R, size_t C)
{
    __shared__ float tile[64][65];
    A += static_cast<size_t>(blockIdx.z) * R * C;
    out += static_cast<size_t>(blockIdx.z) * R * C;
    const size_t r0 = static_cast<size_t>(blockIdx.y) * 64, c0 = static_cast<size_t>(blockIdx.x) * 64;
    const unsigned tx = threadIdx.x % 16, ty = threadIdx.x / 16;   // 16 x 16
#pragma unroll
    for (unsigned k = 0; k < 4; ++k)
    {
        const unsigned rr = ty + 16 * k;
        const size_t r = r0 + rr, c = c0 + 4 * tx;
        if (r < R && c < C)
        {
            const float4 v = *reinterpret_cast<const float4*>(A + r * C + c);
            tile[rr][4 * tx + 0] = v.x;
            tile[rr][4 * tx + 1] = v.y;
            tile[rr][4 * tx + 2] = v.z;
            tile[rr][4 * tx + 3] = v.w;
        }
    }
    __syncthreads();
#pragma unroll
    for (unsigned k = 0; k < 4; ++k)
    {
        const unsigned cc = ty + 16 * k;
        const size_t c = c0 + cc, r = r0 + 4 * tx;   // out (C, R): row c, columns r .. r+3
        if (c < C && r < R)
            *reinterpret_cast<float4*>(out + c * R + r) =
                make_float4(tile[4 * tx + 0][cc], tile[4 * tx + 1][cc], tile[4 * tx + 2][cc], tile[4 * tx + 3][cc]);
    }
}

// ── rearrange_3d: (M, B*N) <-> (B*M, N), contiguous runs of N ─────────────
// IT: index type, 32-bit when every index fits (integer division by a
// runtime divisor costs several times more in 64 bits).
template <bool VEC, class IT>
__global__ __launch_bounds__(kThreads) void k_rearrange(const float* in, float* out, IT M, IT B, IT N,
                                                        unsigned inverse)
{
    const IT W = VEC ? 4 : 1;
    const IT total = M * B * N / W;
    const IT Nw = N / W;
    const IT stride = static_cast<IT>(gridDim.x) * kThreads;
    for (IT o = static_cast<IT>(blockIdx.x) * kThreads + threadIdx.x; o < total; o += stride)
    {
        IT src;
        if (!inverse)
        {
            // out[(b*M+m), n] = in[m, b*N+n]
            const IT row = o / Nw, n = o - row * Nw, b = row / M, m = row - b * M;
            src = (m * B + b) * Nw + n;
        }
        else
        {
            // out[m, b*N+n] = in[(b*M+m), n]
            const IT m = o / (B * Nw), rem = o - m * (B * Nw), b = rem / Nw, n = rem - b * Nw;
            src = (b * M + m) * Nw + n;
        }
        if constexpr (VEC)
            reinterpret_cast<float4*>(out)[o] = reinterpret_cast<const float4*>(in)[src];
        else
            out[o] = in[src];
    }
}

// ── gather: out[i, :] = table[idx[i], :] or zeros ─────────────────────────
template <bool VEC, class IT>
__global__ __launch_bounds__(kThreads) void k_gather(const float* table, const float* idx, float* out, size_t vocab,
                                                     IT D, IT num)
{
    const IT W = VEC ? 4 : 1, Dw = D / W, total = num * Dw;
    const IT stride = static_cast<IT>(gridDim.x) * kThreads;
    for (IT o = static_cast<IT>(blockIdx.x) * kThreads + threadIdx.x; o < total; o += stride)
    {
        const IT i = o / Dw, d = o - i * Dw;
        size_t r;
        const bool ok = row_index(idx[i], vocab, r);
        if constexpr (VEC)
            reinterpret_cast<float4*>(out)[o] =
                ok ? reinterpret_cast<const float4*>(table)[r * size_t(Dw) + d] : make_float4(0, 0, 0, 0);
        else
            out[o] = ok ? table[r * size_t(D) + d] : 0.0f;
    }
}

// ── ordered scatter-add ────────────────────────────────────────────────────
constexpr unsigned long long kSentinel = ~0ull;
constexpr unsigned kSortChunk = 2048;   // elements sorted per workgroup in LDS
constexpr unsigned kSortThreads = 1024;

size_t pow2_at_least(size_t n)
{
    size_t p = 1;
    while (p < n) p <<= 1;
    return p;
}

__global__ __launch_bounds__(kThreads) void k_scatter_keys(const float* idx, unsigned long long* keys, size_t num,
                                                           size_t npow2, size_t vocab)
{
    const size_t i = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= npow2) return;
    unsigned long long k = kSentinel;
    size_t r;
    if (i < num && row_index(idx[i], vocab, r)) k = (static_cast<unsigned long long>(r) << 32) | i;
    keys[i] = k;
}

__device__ __forceinline__ void bitonic_cmp(unsigned long long& a, unsigned long long& b, bool asc)
{
    if ((a > b) == asc)
    {
        const unsigned long long t = a;
        a = b;
        b = t;
    }
}

// Full sort of each 2048-key chunk (merge_k == 0), or the j < 2048 steps of
// stage merge_k. Direction uses the global index, as the global passes do.
__global__ __launch_bounds__(kSortThreads) void k_bitonic_local(unsigned long long* keys, unsigned merge_k_log2)
{
    __shared__ unsigned long long s[kSortChunk];
    const size_t base = static_cast<size_t>(blockIdx.x) * kSortChunk;
    const unsigned t = threadIdx.x;
    s[t] = keys[base + t];
    s[t + kSortThreads] = keys[base + t + kSortThreads];
    __syncthreads();
    auto step = [&](size_t k, unsigned j) {
        const unsigned i = 2 * j * (t / j) + (t % j);
        const bool asc = ((base + i) & k) == 0;
        bitonic_cmp(s[i], s[i + j], asc);
        __syncthreads();
    };
    if (merge_k_log2 == 0)
    {
        for (size_t k = 2; k <= kSortChunk; k <<= 1)
            for (unsigned j = static_cast<unsigned>(k / 2); j > 0; j >>= 1) step(k, j);
    }
    else
    {
        const size_t k = size_t{1} << merge_k_log2;
        for (unsigned j = kSortChunk / 2; j > 0; j >>= 1) step(k, j);
    }
    keys[base + t] = s[t];
    keys[base + t + kSortThreads] = s[t + kSortThreads];
}

__global__ __launch_bounds__(kThreads) void k_bitonic_global(unsigned long long* keys, size_t n, size_t k, size_t j)
{
    const size_t p = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (p >= n / 2) return;
    const size_t i = 2 * j * (p / j) + (p % j);
    unsigned long long a = keys[i], b = keys[i + j];
    const bool asc = (i & k) == 0;
    if ((a > b) == asc)
    {
        keys[i] = b;
        keys[i + j] = a;
    }
}

// Small arrays (npow2 < 2048): one workgroup sorts everything.
__global__ __launch_bounds__(kSortThreads) void k_bitonic_small(unsigned long long* keys, unsigned n)
{
    __shared__ unsigned long long s[kSortChunk];
    const unsigned t = threadIdx.x;
    for (unsigned i = t; i < n; i += kSortThreads) s[i] = keys[i];
    __syncthreads();
    for (unsigned k = 2; k <= n; k <<= 1)
        for (unsigned j = k / 2; j > 0; j >>= 1)
        {
            for (unsigned p = t; p < n / 2; p += kSortThreads)
            {
                const unsigned i = 2 * j * (p / j) + (p % j);
                bitonic_cmp(s[i], s[i + j], (i & k) == 0);
            }
            __syncthreads();
        }
    for (unsigned i = t; i < n; i += kSortThreads) keys[i] = s[i];
}

// One workgroup per sorted position; the first position of each run of equal
// destination rows adds the run's gradient rows in order.
__global__ __launch_bounds__(kThreads) void k_scatter_runs(float* dst, const float* grad,
                                                           const unsigned long long* keys, size_t num, size_t D)
{
    const size_t p = blockIdx.x;
    const unsigned long long k = keys[p];
    if (k == kSentinel) return;
    const unsigned long long row = k >> 32;
    if (p > 0 && (keys[p - 1] >> 32) == row) return;
    size_t end = p + 1;
    while (end < num && keys[end] != kSentinel && (keys[end] >> 32) == row) ++end;
    for (size_t c = threadIdx.x; c < D; c += kThreads)
    {
        float acc = dst[row * D + c];
        for (size_t q = p; q < end; ++q) acc += grad[(keys[q] & 0xffffffffull) * D + c];
        dst[row * D + c] = acc;
    }
}

} // namespace
} // namespace nnhip

using namespace nnhip;

extern "C" int nnhip_transpose(const float* A, float* out, size_t R, size_t C, void* stream)
{
    return nnhip_transpose_batched(A, out, 1, R, C, stream);
}

extern "C" int nnhip_transpose_batched(const float* A, float* out, size_t batch, size_t R, size_t C, void* stream)
{
    if (batch == 0 || R == 0 || C == 0) return 0;
    // A row or column vector's transpose holds the same floats in the same order.
    if (R == 1 || C == 1) return nnhip_copy(A, out, batch * R * C, stream);
    if ((C + 63) / 64 > 0x7fffffff || (R + 63) / 64 > 65535 || batch > 65535) return -1;
    const dim3 grid(static_cast<unsigned>((C + 63) / 64), static_cast<unsigned>((R + 63) / 64),
                    static_cast<unsigned>(batch));
    if (R % 4 == 0 && C % 4 == 0 && aligned16(A) && aligned16(out))
        hipLaunchKernelGGL(k_transpose4, grid, dim3(256), 0, static_cast<hipStream_t>(stream), A, out, R, C);
    else
        hipLaunchKernelGGL(k_transpose, grid, dim3(256), 0, static_cast<hipStream_t>(stream), A, out, R, C);
    return launch_status();
}

extern "C" int nnhip_rearrange_3d(const float* A, float* out, size_t M, size_t B, size_t N, unsigned inverse,
                                  void* stream)
{
    const size_t total = M * B * N;
    if (total == 0) return 0;
    auto s = static_cast<hipStream_t>(stream);
    const bool vec = N % 4 == 0 && aligned16(A) && aligned16(out);
    const unsigned grid = grid_for(vec ? total / 4 : total, kThreads, 256 * 32);
    // 32-bit indices when o + stride cannot wrap
    const bool i32 = total + static_cast<size_t>(grid) * kThreads < (size_t{1} << 32);
    if (vec && i32)
        hipLaunchKernelGGL((k_rearrange<true, unsigned>), dim3(grid), dim3(kThreads), 0, s, A, out, unsigned(M),
                           unsigned(B), unsigned(N), inverse);
    else if (vec)
        hipLaunchKernelGGL((k_rearrange<true, size_t>), dim3(grid), dim3(kThreads), 0, s, A, out, M, B, N, inverse);
    else if (i32)
        hipLaunchKernelGGL((k_rearrange<false, unsigned>), dim3(grid), dim3(kThreads), 0, s, A, out, unsigned(M),
                           unsigned(B), unsigned(N), inverse);
    else
        hipLaunchKernelGGL((k_rearrange<false, size_t>), dim3(grid), dim3(kThreads), 0, s, A, out, M, B, N, inverse);
    return launch_status();
}

extern "C" int nnhip_gather(const float* table, const float* indices, float* out, size_t vocab, size_t D, size_t num,
                            void* stream)
{
    const size_t total = num * D;
    if (total == 0) return 0;
    auto s = static_cast<hipStream_t>(stream);
    const bool vec = D % 4 == 0 && aligned16(table) && aligned16(out);
    const unsigned grid = grid_for(vec ? total / 4 : total, kThreads, 256 * 32);
    const bool i32 = total + static_cast<size_t>(grid) * kThreads < (size_t{1} << 32);
    if (vec && i32)
        hipLaunchKernelGGL((k_gather<true, unsigned>), dim3(grid), dim3(kThreads), 0, s, table, indices, out, vocab,
                           unsigned(D), unsigned(num));
    else if (vec)
        hipLaunchKernelGGL((k_gather<true, size_t>), dim3(grid), dim3(kThreads), 0, s, table, indices, out, vocab, D,
                           num);
    else if (i32)
        hipLaunchKernelGGL((k_gather<false, unsigned>), dim3(grid), dim3(kThreads), 0, s, table, indices, out, vocab,
                           unsigned(D), unsigned(num));
    else
        hipLaunchKernelGGL((k_gather<false, size_t>), dim3(grid), dim3(kThreads), 0, s, table, indices, out, vocab, D,
                           num);
    return launch_status();
}

extern "C" size_t nnhip_scatter_add_workspace_bytes(size_t num)
{
    size_t n = pow2_at_least(num < 2 ? 2 : num);
    return n * sizeof(unsigned long long);
}

extern "C" int nnhip_scatter_add(float* dst, const float* indices, const float* grad, size_t vocab, size_t D,
                                 size_t num, void* workspace, void* stream)
{
    if (num == 0 || D == 0) return 0;
    if (num > 0xffffffffull || vocab > 0xffffffffull) return -1;   // keys pack row and i in 32 bits each
    auto s = static_cast<hipStream_t>(stream);
    auto* keys = static_cast<unsigned long long*>(workspace);
    const size_t n = pow2_at_least(num < 2 ? 2 : num);
    hipLaunchKernelGGL(k_scatter_keys, dim3(grid_for(n, kThreads, 1u << 30)), dim3(kThreads), 0, s, indices, keys, num,
                       n, vocab);
    if (n <= kSortChunk)
    {
        hipLaunchKernelGGL(k_bitonic_small, dim3(1), dim3(kSortThreads), 0, s, keys, static_cast<unsigned>(n));
    }
    else
    {
        const unsigned chunks = static_cast<unsigned>(n / kSortChunk);
        hipLaunchKernelGGL(k_bitonic_local, dim3(chunks), dim3(kSortThreads), 0, s, keys, 0u);
        unsigned klog = 12;   // first stage beyond the chunk: k = 4096
        for (size_t k = 2 * kSortChunk; k <= n; k <<= 1, ++klog)
        {
            for (size_t j = k / 2; j >= kSortChunk; j >>= 1)
                hipLaunchKernelGGL(k_bitonic_global, dim3(grid_for(n / 2, kThreads, 1u << 30)), dim3(kThreads), 0, s,
                                   keys, n, k, j);
            hipLaunchKernelGGL(k_bitonic_local, dim3(chunks), dim3(kSortThreads), 0, s, keys, klog);
        }
    }
    if (num > 0x7fffffffull) return -1;
    hipLaunchKernelGGL(k_scatter_runs, dim3(static_cast<unsigned>(num)), dim3(kThreads), 0, s, dst, grad, keys, num, D);
    return launch_status();
}
