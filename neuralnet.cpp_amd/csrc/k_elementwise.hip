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
// One rounding (fused multiply-add), spelled out so that k_adam's axpy step
// rounds identically.
struct AxpyF
{
    float s;
    __device__ float operator()(float a, float b) const { return __builtin_fmaf(s, b, a); }
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

// The Adam(W) per-tensor chain of engine primitives (reference
// compute_optimizer.hpp:252-304, AdamW decay :388-412) in one pass: p, m, v
// read and written once, g read once, 28 bytes per element. Every step is
// rounded exactly as its separate primitive kernel rounds it (k_map with
// ScalarF / AxpyF / BinaryF / UnaryF), in the same order, so the fused and
// unfused chains agree bit for bit; contraction into FMAs is switched off for
// that reason.
struct AdamArgs
{
    float decay, b1, c1, b2, c2, ib1, ib2, eps, neg_lr;
    int has_decay;
};

__device__ __forceinline__ void adam_elem(float& p, float& m, float& v, float g, const AdamArgs& a)
{
#pragma clang fp contract(off)
    float pp = a.has_decay ? p * a.decay : p;   // scale_inplace(p, 1 - lr*wd)
    float mm = m * a.b1;                        // scale_inplace(m, b1)
    mm = __builtin_fmaf(a.c1, g, mm);           // axpy_inplace(m, 1 - b1, g)
    float vv = v * a.b2;                        // scale_inplace(v, b2)
    float g2 = g * g;                           // g2 = g * g
    g2 = g2 * a.c2;                             // scale_inplace(g2, 1 - b2)
    vv = vv + g2;                               // add_inplace(v, g2)
    const float mh = mm * a.ib1;                // m_hat = clone(m) * inv_bc1
    const float vh = vv * a.ib2;                // v_hat = clone(v) * inv_bc2
    const float den = sqrtf(vh) + a.eps;        // sqrt(v_hat) + eps
    float r = mh / den;                         // m_hat / den
    r = r * a.neg_lr;                           // scale_inplace(ratio, -lr)
    p = pp + r;                                 // add_inplace(p, ratio)
    m = mm;
    v = vv;
}

template <bool VEC>
__global__ __launch_bounds__(kThreads) void k_adam(float* p, float* m, float* v, const float* g, size_t n, AdamArgs a)
{
    const size_t tid = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x;
    const size_t stride = static_cast<size_t>(gridDim.x) * kThreads;
    size_t done = 0;
    if constexpr (VEC)
    {
        const size_t n4 = n / 4;
        float4* p4 = reinterpret_cast<float4*>(p);
        float4* m4 = reinterpret_cast<float4*>(m);
        float4* v4 = reinterpret_cast<float4*>(v);
        const float4* g4 = reinterpret_cast<const float4*>(g);
        for (size_t i = tid; i < n4; i += stride)
        {
            float4 pp = p4[i], mm = m4[i], vv = v4[i];
            const float4 gg = g4[i];
            adam_elem(pp.x, mm.x, vv.x, gg.x, a);
            adam_elem(pp.y, mm.y, vv.y, gg.y, a);
            adam_elem(pp.z, mm.z, vv.z, gg.z, a);
            adam_elem(pp.w, mm.w, vv.w, gg.w, a);
            p4[i] = pp;
            m4[i] = mm;
            v4[i] = vv;
        }
        done = n4 * 4;
    }
    for (size_t i = done + tid; i < n; i += stride)
    {
        float pp = p[i], mm = m[i], vv = v[i];
        adam_elem(pp, mm, vv, g[i], a);
        p[i] = pp;
        m[i] = mm;
        v[i] = vv;
    }
}

// The SwiGLU forward chain of engine primitives (reference compute_layer.hpp,
// SwiGLU::forward: t = -gate, t = exp(t), t = t + c_add, s = c_div / t,
// sw = gate * s, out = sw * up) in one pass with the same roundings: gate and
// up read once, s (kept by the layer) and out written once.
template <bool VEC>
__global__ __launch_bounds__(kThreads) void k_swiglu_fwd(const float* gate, const float* up, float* s_out,
                                                         float* out, size_t n, float c_add, float c_div)
{
    const size_t tid = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x;
    const size_t stride = static_cast<size_t>(gridDim.x) * kThreads;
    auto one = [&](float g, float u, float& sv, float& o) {
        sv = c_div / (expf(-g) + c_add);
        o = (g * sv) * u;
    };
    size_t done = 0;
    if constexpr (VEC)
    {
        const size_t n4 = n / 4;
        for (size_t i = tid; i < n4; i += stride)
        {
            const float4 g = reinterpret_cast<const float4*>(gate)[i], u = reinterpret_cast<const float4*>(up)[i];
            float4 sv, o;
            one(g.x, u.x, sv.x, o.x);
            one(g.y, u.y, sv.y, o.y);
            one(g.z, u.z, sv.z, o.z);
            one(g.w, u.w, sv.w, o.w);
            if (s_out) reinterpret_cast<float4*>(s_out)[i] = sv;
            reinterpret_cast<float4*>(out)[i] = o;
        }
        done = n4 * 4;
    }
    for (size_t i = done + tid; i < n; i += stride)
    {
        float sv, o;
        one(gate[i], up[i], sv, o);
        if (s_out) s_out[i] = sv;
        out[i] = o;
    }
}

// Plain copy, float4 per lane and two in flight (slices, row inserts, clones).
__global__ __launch_bounds__(kThreads) void k_copy4(const float4* __restrict__ src, float4* __restrict__ dst, size_t n4)
{
    const size_t stride = static_cast<size_t>(gridDim.x) * kThreads;
    size_t i = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x;
    for (; i + stride < n4; i += 2 * stride)
    {
        const float4 a = src[i], b = src[i + stride];
        dst[i] = a;
        dst[i + stride] = b;
    }
    if (i < n4) dst[i] = src[i];
}
__global__ __launch_bounds__(kThreads) void k_copy1(const float* __restrict__ src, float* __restrict__ dst, size_t n)
{
    const size_t stride = static_cast<size_t>(gridDim.x) * kThreads;
    for (size_t i = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x; i < n; i += stride) dst[i] = src[i];
}

// Adam / AdamW over up to kAdamMax tensors in one launch (the optimizer's
// per-parameter chains with one set of scalars: Optimizer::step issues them
// back to back). Blocks of 256 threads x 4 float4 per tensor, block ranges
// from the prefix sums in `first`; the same per-element steps as k_adam.
constexpr int kAdamMax = 48;
constexpr unsigned kAdamBlockFloats = kThreads * 16;
struct AdamList
{
    float* p[kAdamMax];
    float* m[kAdamMax];
    float* v[kAdamMax];
    const float* g[kAdamMax];
    unsigned long long n[kAdamMax];
    unsigned first[kAdamMax + 1];
    int count;
    AdamArgs a;
};
__global__ __launch_bounds__(kThreads) void k_adam_list(AdamList L)
{
    const unsigned b = blockIdx.x;
    int lo = 0, hi = L.count - 1;   // last tensor whose first block is <= b
    while (lo < hi)
    {
        const int mid = (lo + hi + 1) / 2;
        if (L.first[mid] <= b) lo = mid;
        else hi = mid - 1;
    }
    const int t = lo;
    const size_t base = static_cast<size_t>(b - L.first[t]) * kAdamBlockFloats, n = L.n[t];
    float* __restrict__ p = L.p[t];
    float* __restrict__ m = L.m[t];
    float* __restrict__ v = L.v[t];
    const float* __restrict__ g = L.g[t];
    const bool vec = ((reinterpret_cast<uintptr_t>(p) | reinterpret_cast<uintptr_t>(m) |
                       reinterpret_cast<uintptr_t>(v) | reinterpret_cast<uintptr_t>(g)) & 15u) == 0;
    if (vec && base + kAdamBlockFloats <= n)
    {
        // A whole block of float4s: every load issued before any update. Each
        // value is read and written once per step, so the accesses are
        // non-temporal (streamed past the caches).
        typedef float f4 __attribute__((ext_vector_type(4)));
        f4 pp[4], mm[4], vv[4], gg[4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
        {
            const size_t i = base + (static_cast<size_t>(k) * kThreads + threadIdx.x) * 4;
            pp[k] = __builtin_nontemporal_load(reinterpret_cast<const f4*>(p + i));
            mm[k] = __builtin_nontemporal_load(reinterpret_cast<const f4*>(m + i));
            vv[k] = __builtin_nontemporal_load(reinterpret_cast<const f4*>(v + i));
            gg[k] = __builtin_nontemporal_load(reinterpret_cast<const f4*>(g + i));
        }
#pragma unroll
        for (int k = 0; k < 4; ++k)
        {
            const size_t i = base + (static_cast<size_t>(k) * kThreads + threadIdx.x) * 4;
#pragma unroll
            for (int e = 0; e < 4; ++e)
            {
                float pe = pp[k][e], me = mm[k][e], ve = vv[k][e];
                adam_elem(pe, me, ve, gg[k][e], L.a);
                pp[k][e] = pe;
                mm[k][e] = me;
                vv[k][e] = ve;
            }
            __builtin_nontemporal_store(pp[k], reinterpret_cast<f4*>(p + i));
            __builtin_nontemporal_store(mm[k], reinterpret_cast<f4*>(m + i));
            __builtin_nontemporal_store(vv[k], reinterpret_cast<f4*>(v + i));
        }
        return;
    }
#pragma unroll
    for (int k = 0; k < 4; ++k)
    {
        const size_t i = base + (static_cast<size_t>(k) * kThreads + threadIdx.x) * 4;
        if (vec && i + 4 <= n)
        {
            float4 pp = *reinterpret_cast<float4*>(p + i), mm = *reinterpret_cast<float4*>(m + i),
                   vv = *reinterpret_cast<float4*>(v + i);
            const float4 gg = *reinterpret_cast<const float4*>(g + i);
            adam_elem(pp.x, mm.x, vv.x, gg.x, L.a);
            adam_elem(pp.y, mm.y, vv.y, gg.y, L.a);
            adam_elem(pp.z, mm.z, vv.z, gg.z, L.a);
            adam_elem(pp.w, mm.w, vv.w, gg.w, L.a);
            *reinterpret_cast<float4*>(p + i) = pp;
            *reinterpret_cast<float4*>(m + i) = mm;
            *reinterpret_cast<float4*>(v + i) = vv;
        }
        else
            for (size_t e = i; e < i + 4 && e < n; ++e)
            {
                float pp = p[e], mm = m[e], vv = v[e];
                adam_elem(pp, mm, vv, g[e], L.a);
                p[e] = pp;
                m[e] = mm;
                v[e] = vv;
            }
    }
}

// Zero fill of up to kFillMax tensors in one launch: block ranges per tensor
// from the prefix sums in `first` (blocks of 256 threads x 4 floats x 4).
constexpr int kFillMax = 96;
struct FillList
{
    float* p[kFillMax];
    unsigned long long n[kFillMax];
    unsigned first[kFillMax + 1];
    int count;
};
__global__ __launch_bounds__(kThreads) void k_fill_list(FillList f)
{
    // The block's tensor: the last t with first[t] <= b (binary search over the
    // strictly increasing prefix sums; a scan of up to 96 kernel-argument
    // loads per 16 KB block cost more than the block's stores).
    const unsigned b = blockIdx.x;
    int t = 0, hi = f.count - 1;
    while (t < hi)
    {
        const int mid = (t + hi + 1) >> 1;
        if (f.first[mid] <= b)
            t = mid;
        else
            hi = mid - 1;
    }
    const size_t base = static_cast<size_t>(b - f.first[t]) * kThreads * 16, n = f.n[t];
    float* p = f.p[t];
    const bool vec = (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
#pragma unroll
    for (int k = 0; k < 4; ++k)
    {
        const size_t i = base + (static_cast<size_t>(k) * kThreads + threadIdx.x) * 4;
        if (vec && i + 4 <= n)
            *reinterpret_cast<float4*>(p + i) = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        else
            for (size_t e = i; e < i + 4 && e < n; ++e) p[e] = 0.0f;
    }
}

} // namespace
} // namespace nnhip

using namespace nnhip;

extern "C" int nnhip_swiglu_forward(const float* gate, const float* up, float* s_out, float* out, size_t count,
                                    float c_add, float c_div, void* stream)
{
    if (count == 0) return 0;
    if (!gate || !up || !out) return -1;
    const bool vec = aligned16(gate) && aligned16(up) && aligned16(out) && (!s_out || aligned16(s_out));
    const unsigned grid = grid_for(vec ? (count + 3) / 4 : count, kThreads, 256 * 32);
    auto s = static_cast<hipStream_t>(stream);
    if (vec)
        hipLaunchKernelGGL(k_swiglu_fwd<true>, dim3(grid), dim3(kThreads), 0, s, gate, up, s_out, out, count, c_add,
                           c_div);
    else
        hipLaunchKernelGGL(k_swiglu_fwd<false>, dim3(grid), dim3(kThreads), 0, s, gate, up, s_out, out, count,
                           c_add, c_div);
    return launch_status();
}

extern "C" int nnhip_copy(const float* src, float* dst, size_t count, void* stream)
{
    if (count == 0) return 0;
    if (!src || !dst) return -1;
    auto s = static_cast<hipStream_t>(stream);
    if (aligned16(src) && aligned16(dst) && count % 4 == 0)
        hipLaunchKernelGGL(k_copy4, dim3(grid_for(count / 8 + 1, kThreads, 256 * 16)), dim3(kThreads), 0, s,
                           reinterpret_cast<const float4*>(src), reinterpret_cast<float4*>(dst), count / 4);
    else
        hipLaunchKernelGGL(k_copy1, dim3(grid_for(count, kThreads, 256 * 16)), dim3(kThreads), 0, s, src, dst, count);
    return launch_status();
}

extern "C" int nnhip_zero_list(float* const* ptrs, const size_t* counts, size_t n, void* stream)
{
    auto s = static_cast<hipStream_t>(stream);
    for (size_t i0 = 0; i0 < n; i0 += kFillMax)
    {
        FillList f{};
        unsigned blocks = 0;
        f.count = 0;
        for (size_t i = i0; i < n && i < i0 + kFillMax; ++i)
        {
            if (counts[i] == 0) continue;
            if (!ptrs[i]) return -1;
            const size_t nb = (counts[i] + kThreads * 16 - 1) / (kThreads * 16);
            if (blocks + nb > 0x7fffffffu) return -3;
            f.p[f.count] = ptrs[i];
            f.n[f.count] = counts[i];
            f.first[f.count] = blocks;
            blocks += static_cast<unsigned>(nb);
            ++f.count;
        }
        if (f.count == 0) continue;
        f.first[f.count] = blocks;
        hipLaunchKernelGGL(k_fill_list, dim3(blocks), dim3(kThreads), 0, s, f);
        if (int rc = launch_status()) return rc;
    }
    return 0;
}

extern "C" int nnhip_adam_update(float* p, float* m, float* v, const float* g, size_t count, int has_decay,
                                 float decay, float beta1, float one_minus_beta1, float beta2, float one_minus_beta2,
                                 float inv_bc1, float inv_bc2, float eps, float neg_lr, void* stream)
{
    if (count == 0) return 0;
    if (!p || !m || !v || !g) return -1;
    const AdamArgs a{decay, beta1, one_minus_beta1, beta2, one_minus_beta2, inv_bc1, inv_bc2, eps, neg_lr,
                     has_decay ? 1 : 0};
    const bool vec = aligned16(p) && aligned16(m) && aligned16(v) && aligned16(g);
    const size_t work = vec ? (count + 3) / 4 : count;
    const unsigned grid = grid_for(work, kThreads, 256 * 32);
    auto s = static_cast<hipStream_t>(stream);
    if (vec)
        hipLaunchKernelGGL(k_adam<true>, dim3(grid), dim3(kThreads), 0, s, p, m, v, g, count, a);
    else
        hipLaunchKernelGGL(k_adam<false>, dim3(grid), dim3(kThreads), 0, s, p, m, v, g, count, a);
    return launch_status();
}

extern "C" int nnhip_adam_update_list(float* const* p, float* const* m, float* const* v, const float* const* g,
                                      const size_t* counts, size_t n, int has_decay, float decay, float beta1,
                                      float one_minus_beta1, float beta2, float one_minus_beta2, float inv_bc1,
                                      float inv_bc2, float eps, float neg_lr, void* stream)
{
    if (n && (!p || !m || !v || !g || !counts)) return -1;
    const AdamArgs a{decay, beta1, one_minus_beta1, beta2, one_minus_beta2, inv_bc1, inv_bc2, eps, neg_lr,
                     has_decay ? 1 : 0};
    auto s = static_cast<hipStream_t>(stream);
    for (size_t i0 = 0; i0 < n; i0 += kAdamMax)
    {
        AdamList L{};
        L.a = a;
        unsigned blocks = 0;
        for (size_t i = i0; i < n && i < i0 + kAdamMax; ++i)
        {
            if (counts[i] == 0) continue;
            if (!p[i] || !m[i] || !v[i] || !g[i]) return -1;
            const size_t nb = (counts[i] + kAdamBlockFloats - 1) / kAdamBlockFloats;
            if (blocks + nb > 0x7fffffffu) return -3;
            L.p[L.count] = p[i];
            L.m[L.count] = m[i];
            L.v[L.count] = v[i];
            L.g[L.count] = g[i];
            L.n[L.count] = counts[i];
            L.first[L.count] = blocks;
            blocks += static_cast<unsigned>(nb);
            ++L.count;
        }
        if (L.count == 0) continue;
        L.first[L.count] = blocks;
        hipLaunchKernelGGL(k_adam_list, dim3(blocks), dim3(kThreads), 0, s, L);
        if (int rc = launch_status()) return rc;
    }
    return 0;
}

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
