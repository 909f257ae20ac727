// k_elementwise.hip — HBM-streaming elementwise, broadcast and fill kernels.
//
// Semantics: cpu_engine.hpp:1008-1044 (in-place ops), :1092-1125 (broadcast),
// :1131-1266 (unary / binary / scalar / select). One grid-stride kernel
// template moves float4 per lane when every pointer is 16-byte aligned (the
// engine's allocations always are) and falls back to scalar lanes otherwise.
// Output may alias an input (in-place ops): no __restrict__.
#include "common.hpp"
#include "nnhip_kernels.h"

namespace nnhip
{
namespace
{

struct UnaryF
{
    unsigned op;
    __device__ float operator()(float a, float) const { return unary_op(op, a); }
};
struct BinaryF
{
    unsigned op;
    __device__ float operator()(float a, float b) const { return binary_op(op, a, b); }
};
struct ScalarF
{
    unsigned op;
    float s;
    int first;
    __device__ float operator()(float a, float) const { return first ? binary_op(op, s, a) : binary_op(op, a, s); }
};
struct AxpyF
{
    float s;
    __device__ float operator()(float a, float b) const { return a + s * b; }
};
struct SelectF
{
    unsigned cmp;
    float sb, se;
    __device__ float operator()(float a, float t) const { return compare_op(cmp, a, sb) ? t : se; }
};
struct FillF
{
    float v;
    __device__ float operator()(float, float) const { return v; }
};

constexpr unsigned kThreads = 256;

template <bool VEC, bool HAS_A, bool HAS_B, class F>
__global__ __launch_bounds__(kThreads) void k_map(const float* a, const float* b, float* out, size_t n, F f)
{
    const size_t tid = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x;
    const size_t stride = static_cast<size_t>(gridDim.x) * kThreads;
    if constexpr (VEC)
    {
        const size_t n4 = n / 4;
        const float4* a4 = reinterpret_cast<const float4*>(a);
        const float4* b4 = reinterpret_cast<const float4*>(b);
        float4* o4 = reinterpret_cast<float4*>(out);
        for (size_t i = tid; i < n4; i += stride)
        {
            float4 va = HAS_A ? a4[i] : make_float4(0, 0, 0, 0);
            float4 vb = HAS_B ? b4[i] : make_float4(0, 0, 0, 0);
            float4 r;
            r.x = f(va.x, vb.x);
            r.y = f(va.y, vb.y);
            r.z = f(va.z, vb.z);
            r.w = f(va.w, vb.w);
            o4[i] = r;
        }
        const size_t t = n4 * 4 + tid;
        if (t < n) out[t] = f(HAS_A ? a[t] : 0.0f, HAS_B ? b[t] : 0.0f);
    }
    else
    {
        for (size_t i = tid; i < n; i += stride) out[i] = f(HAS_A ? a[i] : 0.0f, HAS_B ? b[i] : 0.0f);
    }
}

template <bool HAS_A, bool HAS_B, class F>
int launch_map(const float* a, const float* b, float* out, size_t n, F f, void* stream)
{
    if (n == 0) return 0;
    const bool vec = aligned16(out) && (!HAS_A || aligned16(a)) && (!HAS_B || aligned16(b));
    const size_t work = vec ? (n + 3) / 4 : n;
    // Enough blocks to fill 256 CUs several times over; grid-stride beyond that.
    const unsigned grid = grid_for(work, kThreads, 256 * 32);
    auto s = static_cast<hipStream_t>(stream);
    if (vec)
        hipLaunchKernelGGL((k_map<true, HAS_A, HAS_B, F>), dim3(grid), dim3(kThreads), 0, s, a, b, out, n, f);
    else
        hipLaunchKernelGGL((k_map<false, HAS_A, HAS_B, F>), dim3(grid), dim3(kThreads), 0, s, a, b, out, n, f);
    return launch_status();
}

// A (rows, cols) op= vec: vec indexed by row (ROW) or by column.
template <bool ROW>
__global__ __launch_bounds__(kThreads) void k_broadcast(const float* A, const float* v, float* out, size_t rows,
                                                        size_t cols, unsigned op)
{
    const size_t n = rows * cols;
    const size_t stride = static_cast<size_t>(gridDim.x) * kThreads;
    for (size_t i = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x; i < n; i += stride)
        out[i] = binary_op(op, A[i], ROW ? v[i / cols] : v[i % cols]);
}

// Vector form when cols % 4 == 0: one float4 per lane, never straddling rows.
template <bool ROW>
__global__ __launch_bounds__(kThreads) void k_broadcast4(const float* A, const float* v, float* out, size_t rows,
                                                         size_t cols, unsigned op)
{
    const size_t c4 = cols / 4, n4 = rows * c4;
    const size_t stride = static_cast<size_t>(gridDim.x) * kThreads;
    const float4* a4 = reinterpret_cast<const float4*>(A);
    float4* o4 = reinterpret_cast<float4*>(out);
    for (size_t i = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x; i < n4; i += stride)
    {
        const float4 a = a4[i];
        float4 r;
        if constexpr (ROW)
        {
            const float s = v[i / c4];
            r = make_float4(binary_op(op, a.x, s), binary_op(op, a.y, s), binary_op(op, a.z, s),
                            binary_op(op, a.w, s));
        }
        else
        {
            const size_t c = (i % c4) * 4;
            r = make_float4(binary_op(op, a.x, v[c]), binary_op(op, a.y, v[c + 1]), binary_op(op, a.z, v[c + 2]),
                            binary_op(op, a.w, v[c + 3]));
        }
        o4[i] = r;
    }
}

template <bool ROW>
int launch_broadcast(const float* A, const float* v, float* out, size_t rows, size_t cols, unsigned op,
                     void* stream)
{
    const size_t n = rows * cols;
    if (n == 0) return 0;
    auto s = static_cast<hipStream_t>(stream);
    if (cols % 4 == 0 && aligned16(A) && aligned16(out))
        hipLaunchKernelGGL(k_broadcast4<ROW>, dim3(grid_for(n / 4, kThreads, 256 * 32)), dim3(kThreads), 0, s, A, v,
                           out, rows, cols, op);
    else
        hipLaunchKernelGGL(k_broadcast<ROW>, dim3(grid_for(n, kThreads, 256 * 32)), dim3(kThreads), 0, s, A, v,
                           out, rows, cols, op);
    return launch_status();
}

} // namespace
} // namespace nnhip

using namespace nnhip;

extern "C" int nnhip_elementwise_unary(const float* A, float* out, size_t count, unsigned op, void* stream)
{
    if (op > U_TANH) return -1;
    return launch_map<true, false>(A, nullptr, out, count, UnaryF{op}, stream);
}

extern "C" int nnhip_elementwise_binary(const float* A, const float* B, float* out, size_t count, unsigned op,
                                        void* stream)
{
    if (op > B_MIN) return -1;
    return launch_map<true, true>(A, B, out, count, BinaryF{op}, stream);
}

extern "C" int nnhip_elementwise_binary_scalar(const float* A, float* out, size_t count, unsigned op, float scalar,
                                               int scalar_first, void* stream)
{
    if (op > B_MIN) return -1;
    return launch_map<true, false>(A, nullptr, out, count, ScalarF{op, scalar, scalar_first}, stream);
}

extern "C" int nnhip_axpy(const float* A, const float* B, float* out, size_t count, float scalar, void* stream)
{
    return launch_map<true, true>(A, B, out, count, AxpyF{scalar}, stream);
}

extern "C" int nnhip_elementwise_select_scalar_cond(const float* A, const float* then_v, float* out, size_t count,
                                                    unsigned cmp, float scalar_b, float scalar_else, void* stream)
{
    if (cmp > C_NE) return -1;
    return launch_map<true, true>(A, then_v, out, count, SelectF{cmp, scalar_b, scalar_else}, stream);
}

extern "C" int nnhip_fill(float* out, size_t count, float value, void* stream)
{
    return launch_map<false, false>(nullptr, nullptr, out, count, FillF{value}, stream);
}

extern "C" int nnhip_broadcast_row(const float* A, const float* vec, float* out, size_t rows, size_t cols,
                                   unsigned op, void* stream)
{
    if (op > B_MIN) return -1;
    return launch_broadcast<true>(A, vec, out, rows, cols, op, stream);
}

extern "C" int nnhip_broadcast_col(const float* A, const float* vec, float* out, size_t rows, size_t cols,
                                   unsigned op, void* stream)
{
    if (op > B_MIN) return -1;
    return launch_broadcast<false>(A, vec, out, rows, cols, op, stream);
}
