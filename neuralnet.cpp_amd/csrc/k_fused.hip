// k_fused.hip — one kernel per ExprSpec program of the GPT layers.
//
// The HIP engine recognises the RMSNorm and SwiGLU programs structurally
// (include/nn/layer_exprs.hpp) and runs them here instead of in the generic
// interpreter, which is what the reference's ahead-of-time fused shaders do
// for their GPU engine (tools/scan_exprs.cpp, tools/gen_fused.cpp). Each
// kernel evaluates its program with the same operation order as the program
// (left operand before right); reductions sum in a fixed order.
//
// All tensors are row-major (F, N) fp32 with N % 4 == 0 and 16-byte aligned
// base pointers (the entry points reject anything else with -5), so every
// thread moves float4s. The kernels are HBM-bound: per element they read
// each (F, N) input once and write each output once.
#include "common.hpp"
#include "nnhip_kernels.h"

namespace nnhip
{
namespace
{

constexpr unsigned kT = 256;

__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ __forceinline__ void st4(float* p, float4 v) { *reinterpret_cast<float4*>(p) = v; }

// ── elementwise over (rows, cols): one float4 of one row per thread ──────────
template <class Op>
__global__ __launch_bounds__(kT) void k_fused_ew(Op op, unsigned rows, unsigned cols4)
{
    const unsigned q = blockIdx.x * kT + threadIdx.x;
    if (q >= cols4) return;
    for (unsigned r = blockIdx.y; r < rows; r += gridDim.y) op(r, q);
}

// normed = x * colbcast(v)
struct ColBcastMul
{
    const float* x;
    const float* v;
    float* o;
    size_t cols;
    __device__ void operator()(unsigned r, unsigned q) const
    {
        const size_t i = size_t(r) * cols + 4u * q;
        const float4 a = ld4(x + i), b = ld4(v + 4u * q);
        st4(o + i, make_float4(a.x * b.x, a.y * b.y, a.z * b.z, a.w * b.w));
    }
};

// out = x * rowbcast(v)
struct RowBcastMul
{
    const float* x;
    const float* v;
    float* o;
    size_t cols;
    __device__ void operator()(unsigned r, unsigned q) const
    {
        const size_t i = size_t(r) * cols + 4u * q;
        const float4 a = ld4(x + i);
        const float s = v[r];
        st4(o + i, make_float4(a.x * s, a.y * s, a.z * s, a.w * s));
    }
};

// dx = (g * gamma[r] - m[c] * normed) * rinv[c]
struct RmsDx
{
    const float* g;
    const float* gamma;
    const float* m;
    const float* n;
    const float* rinv;
    float* o;
    size_t cols;
    __device__ static float one(float g, float gr, float m, float n, float ri) { return (g * gr - m * n) * ri; }
    __device__ void operator()(unsigned r, unsigned q) const
    {
        const size_t i = size_t(r) * cols + 4u * q;
        const float4 a = ld4(g + i), b = ld4(m + 4u * q), c = ld4(n + i), d = ld4(rinv + 4u * q);
        const float gr = gamma[r];
        st4(o + i, make_float4(one(a.x, gr, b.x, c.x, d.x), one(a.y, gr, b.y, c.y, d.y), one(a.z, gr, b.z, c.z, d.z),
                               one(a.w, gr, b.w, c.w, d.w)));
    }
};

// ── flat elementwise (SwiGLU backward) ───────────────────────────────────────
template <class Op>
__global__ __launch_bounds__(kT) void k_fused_flat(Op op, size_t n4)
{
    for (size_t q = size_t(blockIdx.x) * kT + threadIdx.x; q < n4; q += size_t(gridDim.x) * kT) op(4 * q);
}

// grad_gate = g * up * (s * (1 + gate * (1 - s)))
struct SwigluGradGate
{
    const float* g;
    const float* up;
    const float* s;
    const float* gate;
    float* o;
    __device__ static float one(float g, float u, float s, float t) { return (g * u) * (s * (1.0f + t * (1.0f - s))); }
    __device__ void operator()(size_t i) const
    {
        const float4 a = ld4(g + i), b = ld4(up + i), c = ld4(s + i), d = ld4(gate + i);
        st4(o + i, make_float4(one(a.x, b.x, c.x, d.x), one(a.y, b.y, c.y, d.y), one(a.z, b.z, c.z, d.z),
                               one(a.w, b.w, c.w, d.w)));
    }
};

// grad_up = g * gate * s
struct SwigluGradUp
{
    const float* g;
    const float* gate;
    const float* s;
    float* o;
    __device__ void operator()(size_t i) const
    {
        const float4 a = ld4(g + i), b = ld4(gate + i), c = ld4(s + i);
        st4(o + i, make_float4((a.x * b.x) * c.x, (a.y * b.y) * c.y, (a.z * b.z) * c.z, (a.w * b.w) * c.w));
    }
};

// Both SwiGLU gradients in one pass (G, up, s, gate read once), each rounded as
// its own program rounds it.
struct SwigluGradBoth
{
    const float* g;
    const float* up;
    const float* s;
    const float* gate;
    float* og;
    float* ou;
    __device__ void operator()(size_t i) const
    {
        const float4 a = ld4(g + i), b = ld4(up + i), c = ld4(s + i), d = ld4(gate + i);
        st4(og + i, make_float4(SwigluGradGate::one(a.x, b.x, c.x, d.x), SwigluGradGate::one(a.y, b.y, c.y, d.y),
                                SwigluGradGate::one(a.z, b.z, c.z, d.z), SwigluGradGate::one(a.w, b.w, c.w, d.w)));
        st4(ou + i, make_float4((a.x * d.x) * c.x, (a.y * d.y) * c.y, (a.z * d.z) * c.z, (a.w * d.w) * c.w));
    }
};

// ── column sums: out[c] = sum_r f(r, c) ──────────────────────────────────────
// A workgroup of 16 waves owns 32 columns (8 float4s: one 128-byte line per
// row) and splits the rows over 128 row groups (8 per wave); each thread
// issues the loads of up to 8 of its rows before adding them. The partial
// sums are combined in a fixed order (inside each wave, then over waves), so
// the result does not depend on scheduling. At the GPT shapes (768 x 8192)
// this puts 4 waves on every SIMD with 6 loads each in flight, where the
// first version (4 waves per workgroup) had one wave per SIMD.
constexpr unsigned kColT = 1024, kColQuads = 8, kRowGroups = kColT / kColQuads, kColWaves = kColT / 64;

struct SumSq
{
    const float* x;
    size_t cols;
    __device__ float4 operator()(unsigned r, unsigned q) const
    {
        const float4 a = ld4(x + size_t(r) * cols + 4u * q);
        return make_float4(a.x * a.x, a.y * a.y, a.z * a.z, a.w * a.w);
    }
};

// g * gamma[r] * normed
struct GGammaN
{
    const float* g;
    const float* gamma;
    const float* n;
    size_t cols;
    __device__ float4 operator()(unsigned r, unsigned q) const
    {
        const size_t i = size_t(r) * cols + 4u * q;
        const float4 a = ld4(g + i), c = ld4(n + i);
        const float gr = gamma[r];
        return make_float4((a.x * gr) * c.x, (a.y * gr) * c.y, (a.z * gr) * c.z, (a.w * gr) * c.w);
    }
};

template <class F>
__global__ __launch_bounds__(kColT) void k_fused_colsum(F f, float* out, unsigned rows, unsigned cols4)
{
    __shared__ float4 part[kColWaves][kColQuads];
    const unsigned lane = threadIdx.x % 64, wave = threadIdx.x / 64;
    const unsigned qi = lane % kColQuads, rg = threadIdx.x / kColQuads;
    const unsigned q = blockIdx.x * kColQuads + qi;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    auto add = [&](const float4& v) {
        acc.x += v.x;
        acc.y += v.y;
        acc.z += v.z;
        acc.w += v.w;
    };
    if (q < cols4)
    {
        constexpr unsigned kBatch = 8;   // rows whose loads are in flight together
        unsigned r = rg;
        for (; r + (kBatch - 1) * kRowGroups < rows; r += kBatch * kRowGroups)
        {
            float4 v[kBatch];
#pragma unroll
            for (unsigned k = 0; k < kBatch; ++k) v[k] = f(r + k * kRowGroups, q);
#pragma unroll
            for (unsigned k = 0; k < kBatch; ++k) add(v[k]);
        }
        for (; r < rows; r += kRowGroups) add(f(r, q));
    }
    // The wave's 8 row groups of one column quad sit 8 lanes apart: add them
    // pairwise (lane bits 3, 4, 5), every lane ending with the same sums.
#pragma unroll
    for (int o = 8; o < 64; o <<= 1)
    {
        acc.x += __shfl_xor(acc.x, o, 64);
        acc.y += __shfl_xor(acc.y, o, 64);
        acc.z += __shfl_xor(acc.z, o, 64);
        acc.w += __shfl_xor(acc.w, o, 64);
    }
    if (lane < kColQuads) part[wave][lane] = acc;
    __syncthreads();
    if (threadIdx.x < kColQuads)
    {
        const unsigned qo = blockIdx.x * kColQuads + threadIdx.x;
        float4 s = part[0][threadIdx.x];
        for (unsigned k = 1; k < kColWaves; ++k)
        {
            const float4 v = part[k][threadIdx.x];
            s.x += v.x;
            s.y += v.y;
            s.z += v.z;
            s.w += v.w;
        }
        if (qo < cols4) st4(out + 4u * qo, s);
    }
}

// ── RMSNorm forward in one pass (compute_layer.hpp RMSNorm::forward) ──────────
// The layer's six calls over x (F, N): s = column sums of x^2 (the SumSq
// program), scaled = s * inv_f, var_eps = scaled + eps, rinv = 1 / sqrt(var_eps),
// normed = x * rinv (per column), out = normed * gamma (per row). The sums take
// k_fused_colsum's geometry and order (thread rows rg, rg + 128, ... added in
// turn, the same lane and wave merges; x^2 + acc as one fma, as the compiler
// contracts it there) and every other value the same expression as its
// separate kernel, so the results equal the six calls' bit for bit. A thread
// keeps its KM rows of x in registers between the sums and the products:
// x is read once. s, scaled and var_eps are written when their pointer is set.
// SUM: x is formed as x + xb while it is read (the block's residual add that
// precedes the layer, GPTBlock::forward, rounded as that add) and written to xs.
template <unsigned KM, bool SUM = false>
__global__ __launch_bounds__(kColT) void k_rms_fwd(const float* __restrict__ x, const float* __restrict__ gamma,
                                                   float inv_f, float eps, float* s_raw, float* scaled,
                                                   float* var_eps, float* __restrict__ rinv,
                                                   float* __restrict__ normed, float* __restrict__ out,
                                                   unsigned rows, unsigned cols4, size_t cols,
                                                   const float* __restrict__ xb, float* __restrict__ xs)
{
    __shared__ float4 part[kColWaves][kColQuads];
    __shared__ float4 rq[kColQuads];
    const unsigned lane = threadIdx.x % 64, wave = threadIdx.x / 64;
    const unsigned qi = lane % kColQuads, rg = threadIdx.x / kColQuads;
    const unsigned q = blockIdx.x * kColQuads + qi;
    float4 xv[KM];
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    if (q < cols4)
    {
#pragma unroll
        for (unsigned k = 0; k < KM; ++k)
        {
            const unsigned r = rg + k * kRowGroups;
            if (r < rows) xv[k] = ld4(x + size_t(r) * cols + 4u * q);
        }
        if constexpr (SUM)
        {
            float4 yv[KM];
#pragma unroll
            for (unsigned k = 0; k < KM; ++k)
                if (rg + k * kRowGroups < rows) yv[k] = ld4(xb + size_t(rg + k * kRowGroups) * cols + 4u * q);
#pragma unroll
            for (unsigned k = 0; k < KM; ++k)
                if (rg + k * kRowGroups < rows)
                {
#pragma clang fp contract(off)
                    xv[k] = make_float4(xv[k].x + yv[k].x, xv[k].y + yv[k].y, xv[k].z + yv[k].z, xv[k].w + yv[k].w);
                    st4(xs + size_t(rg + k * kRowGroups) * cols + 4u * q, xv[k]);
                }
        }
#pragma unroll
        for (unsigned k = 0; k < KM; ++k)
            if (rg + k * kRowGroups < rows)
            {
                acc.x = __builtin_fmaf(xv[k].x, xv[k].x, acc.x);
                acc.y = __builtin_fmaf(xv[k].y, xv[k].y, acc.y);
                acc.z = __builtin_fmaf(xv[k].z, xv[k].z, acc.z);
                acc.w = __builtin_fmaf(xv[k].w, xv[k].w, acc.w);
            }
    }
#pragma unroll
    for (int o = 8; o < 64; o <<= 1)
    {
        acc.x += __shfl_xor(acc.x, o, 64);
        acc.y += __shfl_xor(acc.y, o, 64);
        acc.z += __shfl_xor(acc.z, o, 64);
        acc.w += __shfl_xor(acc.w, o, 64);
    }
    if (lane < kColQuads) part[wave][lane] = acc;
    __syncthreads();
    if (threadIdx.x < kColQuads)
    {
        const unsigned qo = blockIdx.x * kColQuads + threadIdx.x;
        float4 s = part[0][threadIdx.x];
        for (unsigned k = 1; k < kColWaves; ++k)
        {
            const float4 v = part[k][threadIdx.x];
            s.x += v.x;
            s.y += v.y;
            s.z += v.z;
            s.w += v.w;
        }
        {
#pragma clang fp contract(off)
            const float4 sc = make_float4(s.x * inv_f, s.y * inv_f, s.z * inv_f, s.w * inv_f);
            const float4 ve = make_float4(sc.x + eps, sc.y + eps, sc.z + eps, sc.w + eps);
            const float4 ri =
                make_float4(1.0f / sqrtf(ve.x), 1.0f / sqrtf(ve.y), 1.0f / sqrtf(ve.z), 1.0f / sqrtf(ve.w));
            if (qo < cols4)
            {
                if (s_raw) st4(s_raw + 4u * qo, s);
                if (scaled) st4(scaled + 4u * qo, sc);
                if (var_eps) st4(var_eps + 4u * qo, ve);
                st4(rinv + 4u * qo, ri);
            }
            rq[threadIdx.x] = ri;
        }
    }
    __syncthreads();
    if (q < cols4)
    {
        const float4 ri = rq[qi];
#pragma unroll
        for (unsigned k = 0; k < KM; ++k)
        {
            const unsigned r = rg + k * kRowGroups;
            if (r < rows)
            {
#pragma clang fp contract(off)
                const size_t i = size_t(r) * cols + 4u * q;
                const float4 n = make_float4(xv[k].x * ri.x, xv[k].y * ri.y, xv[k].z * ri.z, xv[k].w * ri.w);
                st4(normed + i, n);
                const float g = gamma[r];
                st4(out + i, make_float4(n.x * g, n.y * g, n.z * g, n.w * g));
            }
        }
    }
}

// ── RMSNorm backward's column sum, scale and dx in one pass ───────────────────
// The layer's calls (compute_layer.hpp RMSNorm::backward): m_raw = column sums
// of g * gamma[r] * normed (the GGammaN program), m = m_raw * inv_f, dx =
// (g * gamma[r] - m * normed) * rinv, each with its separate kernel's
// expression and k_fused_colsum's summation order, so equal bit for bit; g and
// normed are read once.
// ADD: also out2 = addend + dx (the block's residual add of the gradient that
// follows the layer, GPTBlock::backward, rounded as that add).
template <unsigned KM, bool ADD = false>
__global__ __launch_bounds__(kColT) void k_rms_bwd(const float* __restrict__ g, const float* __restrict__ gamma,
                                                   const float* __restrict__ nrm, const float* __restrict__ rinv,
                                                   float inv_f, float* m_raw, float* __restrict__ m,
                                                   float* __restrict__ dx, unsigned rows, unsigned cols4, size_t cols,
                                                   const float* __restrict__ addend, float* __restrict__ out2)
{
    __shared__ float4 part[kColWaves][kColQuads];
    __shared__ float4 mq[kColQuads];
    const unsigned lane = threadIdx.x % 64, wave = threadIdx.x / 64;
    const unsigned qi = lane % kColQuads, rg = threadIdx.x / kColQuads;
    const unsigned q = blockIdx.x * kColQuads + qi;
    float4 gv[KM], nv[KM], av[ADD ? KM : 1];
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    if (q < cols4)
    {
#pragma unroll
        for (unsigned k = 0; k < KM; ++k)
        {
            const unsigned r = rg + k * kRowGroups;
            if (r < rows)
            {
                const size_t i = size_t(r) * cols + 4u * q;
                gv[k] = ld4(g + i);
                nv[k] = ld4(nrm + i);
                if constexpr (ADD) av[k] = ld4(addend + i);
            }
        }
#pragma unroll
        for (unsigned k = 0; k < KM; ++k)
        {
            const unsigned r = rg + k * kRowGroups;
            if (r < rows)
            {
                const float gr = gamma[r];
                const float4 a = gv[k], c = nv[k];
                const float4 v = make_float4((a.x * gr) * c.x, (a.y * gr) * c.y, (a.z * gr) * c.z, (a.w * gr) * c.w);
                acc.x += v.x;
                acc.y += v.y;
                acc.z += v.z;
                acc.w += v.w;
            }
        }
    }
#pragma unroll
    for (int o = 8; o < 64; o <<= 1)
    {
        acc.x += __shfl_xor(acc.x, o, 64);
        acc.y += __shfl_xor(acc.y, o, 64);
        acc.z += __shfl_xor(acc.z, o, 64);
        acc.w += __shfl_xor(acc.w, o, 64);
    }
    if (lane < kColQuads) part[wave][lane] = acc;
    __syncthreads();
    if (threadIdx.x < kColQuads)
    {
        const unsigned qo = blockIdx.x * kColQuads + threadIdx.x;
        float4 s = part[0][threadIdx.x];
        for (unsigned k = 1; k < kColWaves; ++k)
        {
            const float4 v = part[k][threadIdx.x];
            s.x += v.x;
            s.y += v.y;
            s.z += v.z;
            s.w += v.w;
        }
        const float4 mm = make_float4(s.x * inv_f, s.y * inv_f, s.z * inv_f, s.w * inv_f);
        if (qo < cols4)
        {
            if (m_raw) st4(m_raw + 4u * qo, s);
            st4(m + 4u * qo, mm);
        }
        mq[threadIdx.x] = mm;
    }
    __syncthreads();
    if (q < cols4)
    {
        const float4 b = mq[qi], d = ld4(rinv + 4u * q);
#pragma unroll
        for (unsigned k = 0; k < KM; ++k)
        {
            const unsigned r = rg + k * kRowGroups;
            if (r < rows)
            {
                const float gr = gamma[r];
                const float4 a = gv[k], c = nv[k];
                const size_t i = size_t(r) * cols + 4u * q;
                const float4 v = make_float4(RmsDx::one(a.x, gr, b.x, c.x, d.x), RmsDx::one(a.y, gr, b.y, c.y, d.y),
                                             RmsDx::one(a.z, gr, b.z, c.z, d.z), RmsDx::one(a.w, gr, b.w, c.w, d.w));
                st4(dx + i, v);
                if constexpr (ADD)
                {
#pragma clang fp contract(off)   // dx rounded first, as the separate add reads it
                    const float4 e = av[k];
                    st4(out2 + i, make_float4(e.x + v.x, e.y + v.y, e.z + v.z, e.w + v.w));
                }
            }
        }
    }
}

// ── narrow matrices (N % 4 != 0: one token's (F, 1) activations in incremental inference) ──
// One workgroup of 256 threads per column. Thread t holds rows t, t + 256, ...
// of the column (x^2 + acc as one fma, in row order); lane 0 of each wave
// takes the wave's butterfly sum and the four waves are added in order. The
// sum of squares and the one-pass forward share this order, so the forward
// equals the separate calls bit for bit, as the float4 kernels do.
constexpr unsigned kNarrowT = 256, kNarrowKM = 4;   // F <= 1024
__device__ __forceinline__ float narrow_sumsq(const float* __restrict__ x, size_t N, unsigned F, unsigned c,
                                              float (&xv)[kNarrowKM])
{
    __shared__ float part[kNarrowT / 64];
#pragma unroll
    for (unsigned k = 0; k < kNarrowKM; ++k)
    {
        const unsigned r = threadIdx.x + k * kNarrowT;
        xv[k] = r < F ? x[size_t(r) * N + c] : 0.0f;
    }
    float acc = 0.0f;
#pragma unroll
    for (unsigned k = 0; k < kNarrowKM; ++k)
        if (threadIdx.x + k * kNarrowT < F) acc = __builtin_fmaf(xv[k], xv[k], acc);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) acc += __shfl_xor(acc, o, 64);
    if (threadIdx.x % 64 == 0) part[threadIdx.x / 64] = acc;
    __syncthreads();
    float s = part[0];
#pragma unroll
    for (unsigned w = 1; w < kNarrowT / 64; ++w) s += part[w];
    return s;
}

__global__ __launch_bounds__(kNarrowT) void k_sumsq_narrow(const float* __restrict__ x, float* __restrict__ out,
                                                           unsigned F, size_t N)
{
    float xv[kNarrowKM];
    const float s = narrow_sumsq(x, N, F, blockIdx.x, xv);
    if (threadIdx.x == 0) out[blockIdx.x] = s;
}

// RMSNorm::forward's six calls on a narrow x, as k_rms_fwd.
__global__ __launch_bounds__(kNarrowT) void k_rms_fwd_narrow(const float* __restrict__ x,
                                                             const float* __restrict__ gamma, float inv_f, float eps,
                                                             float* s_raw, float* scaled, float* var_eps,
                                                             float* __restrict__ rinv, float* __restrict__ normed,
                                                             float* __restrict__ out, unsigned F, size_t N)
{
    const unsigned c = blockIdx.x;
    float xv[kNarrowKM];
    const float s = narrow_sumsq(x, N, F, c, xv);
    float ri;
    {
#pragma clang fp contract(off)
        const float sc = s * inv_f, ve = sc + eps;
        ri = 1.0f / sqrtf(ve);
        if (threadIdx.x == 0)
        {
            if (s_raw) s_raw[c] = s;
            if (scaled) scaled[c] = sc;
            if (var_eps) var_eps[c] = ve;
            rinv[c] = ri;
        }
    }
#pragma unroll
    for (unsigned k = 0; k < kNarrowKM; ++k)
    {
        const unsigned r = threadIdx.x + k * kNarrowT;
        if (r < F)
        {
#pragma clang fp contract(off)
            const float n = xv[k] * ri;
            normed[size_t(r) * N + c] = n;
            out[size_t(r) * N + c] = n * gamma[r];
        }
    }
}

// out = x * colbcast(v) on a narrow x.
__global__ __launch_bounds__(kNarrowT) void k_colbcast_mul_narrow(const float* __restrict__ x,
                                                                  const float* __restrict__ v, float* __restrict__ o,
                                                                  size_t total, size_t N)
{
    const size_t i = size_t(blockIdx.x) * kNarrowT + threadIdx.x;
    if (i < total) o[i] = x[i] * v[i % N];
}

// ── row sums: out[r] = sum_c g[r,c] * gamma[r] * normed[r,c], one workgroup per row ──
__global__ __launch_bounds__(kT) void k_fused_rowsum_ggn(const float* g, const float* gamma, const float* n,
                                                         float* out, unsigned cols4, size_t cols, bool add)
{
    __shared__ float wsum[kT / 64];
    const unsigned r = blockIdx.x;
    const float gr = gamma[r];
    const float* gp = g + size_t(r) * cols;
    const float* np = n + size_t(r) * cols;
    float acc = 0.f;
    for (unsigned q = threadIdx.x; q < cols4; q += kT)
    {
        const float4 a = ld4(gp + 4u * q), c = ld4(np + 4u * q);
        acc += (a.x * gr) * c.x;
        acc += (a.y * gr) * c.y;
        acc += (a.z * gr) * c.z;
        acc += (a.w * gr) * c.w;
    }
    acc = wave_sum(acc);
    if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0)
    {
        float s = wsum[0];
        for (unsigned w = 1; w < kT / 64; ++w) s += wsum[w];
        out[r] = add ? out[r] + s : s;   // add: add_inplace of the sums, rounded as that call rounds
    }
}

constexpr int kBadShape = -5;

bool shape_ok(size_t rows, size_t cols, std::initializer_list<const void*> ptrs)
{
    if (cols % 4 != 0 || cols / 4 > 0xffffffffu || rows > 0xffffffffu) return false;
    for (const void* p : ptrs)
        if (!aligned16(p)) return false;
    return true;
}

template <class Op>
int launch_ew(Op op, size_t rows, size_t cols, hipStream_t s)
{
    if (rows == 0 || cols == 0) return 0;
    const unsigned cols4 = unsigned(cols / 4);
    const dim3 grid((cols4 + kT - 1) / kT, unsigned(rows < 65535 ? rows : 65535));
    hipLaunchKernelGGL(k_fused_ew<Op>, grid, dim3(kT), 0, s, op, unsigned(rows), cols4);
    return launch_status();
}

template <class F>
int launch_colsum(F f, float* out, size_t rows, size_t cols, hipStream_t s)
{
    if (cols == 0) return 0;
    const unsigned cols4 = unsigned(cols / 4);
    hipLaunchKernelGGL(k_fused_colsum<F>, dim3((cols4 + kColQuads - 1) / kColQuads), dim3(kColT), 0, s, f, out,
                       unsigned(rows), cols4);
    return launch_status();
}

template <class Op>
int launch_flat(Op op, size_t count, hipStream_t s)
{
    if (count == 0) return 0;
    const size_t n4 = count / 4;
    hipLaunchKernelGGL(k_fused_flat<Op>, dim3(grid_for(n4, kT, 1u << 16)), dim3(kT), 0, s, op, n4);
    return launch_status();
}

} // namespace
} // namespace nnhip

using namespace nnhip;

namespace
{
// Narrow shapes (N % 4 != 0) the narrow kernels take.
bool narrow_ok(size_t F, size_t N) { return N % 4 != 0 && F >= 1 && F <= kNarrowT * kNarrowKM && N <= 65535; }
} // namespace

extern "C" int nnhip_rmsnorm_sumsq(const float* X, float* out, size_t F, size_t N, void* stream)
{
    if (X && out && narrow_ok(F, N))
    {
        hipLaunchKernelGGL(k_sumsq_narrow, dim3(unsigned(N)), dim3(kNarrowT), 0, static_cast<hipStream_t>(stream), X,
                           out, unsigned(F), N);
        return launch_status();
    }
    if (!shape_ok(F, N, {X, out})) return kBadShape;
    return launch_colsum(SumSq{X, N}, out, F, N, static_cast<hipStream_t>(stream));
}

namespace
{
template <bool SUM>
int rms_forward_wide(const float* X, const float* Xb, float* Xs, const float* gamma, float inv_f, float eps,
                     float* s_raw, float* scaled, float* var_eps, float* rinv, float* normed, float* out, size_t F,
                     size_t N, hipStream_t s)
{
    if (!shape_ok(F, N, {X, rinv, normed, out, s_raw, scaled, var_eps})) return kBadShape;
    if (N == 0) return 0;
    const unsigned cols4 = unsigned(N / 4);
    const dim3 grid((cols4 + kColQuads - 1) / kColQuads), block(kColT);
    if (F <= 2 * kRowGroups)
        hipLaunchKernelGGL((k_rms_fwd<2, SUM>), grid, block, 0, s, X, gamma, inv_f, eps, s_raw, scaled, var_eps, rinv,
                           normed, out, unsigned(F), cols4, N, Xb, Xs);
    else if (F <= 6 * kRowGroups)
        hipLaunchKernelGGL((k_rms_fwd<6, SUM>), grid, block, 0, s, X, gamma, inv_f, eps, s_raw, scaled, var_eps, rinv,
                           normed, out, unsigned(F), cols4, N, Xb, Xs);
    else
        hipLaunchKernelGGL((k_rms_fwd<8, SUM>), grid, block, 0, s, X, gamma, inv_f, eps, s_raw, scaled, var_eps, rinv,
                           normed, out, unsigned(F), cols4, N, Xb, Xs);
    return launch_status();
}

template <bool ADD>
int rms_backward_wide(const float* G, const float* gamma, const float* Nrm, const float* rinv, float inv_f,
                      float* m_raw, float* m, float* dx, const float* addend, float* out2, size_t F, size_t N,
                      hipStream_t s)
{
    if (!shape_ok(F, N, {G, Nrm, rinv, m, dx, m_raw})) return kBadShape;
    if (N == 0) return 0;
    const unsigned cols4 = unsigned(N / 4);
    const dim3 grid((cols4 + kColQuads - 1) / kColQuads), block(kColT);
    if (F <= 2 * kRowGroups)
        hipLaunchKernelGGL((k_rms_bwd<2, ADD>), grid, block, 0, s, G, gamma, Nrm, rinv, inv_f, m_raw, m, dx,
                           unsigned(F), cols4, N, addend, out2);
    else if (F <= 6 * kRowGroups)
        hipLaunchKernelGGL((k_rms_bwd<6, ADD>), grid, block, 0, s, G, gamma, Nrm, rinv, inv_f, m_raw, m, dx,
                           unsigned(F), cols4, N, addend, out2);
    else
        hipLaunchKernelGGL((k_rms_bwd<8, ADD>), grid, block, 0, s, G, gamma, Nrm, rinv, inv_f, m_raw, m, dx,
                           unsigned(F), cols4, N, addend, out2);
    return launch_status();
}
} // namespace

extern "C" int nnhip_rmsnorm_forward(const float* X, const float* gamma, float inv_f, float eps, float* s_raw,
                                     float* scaled, float* var_eps, float* rinv, float* normed, float* out, size_t F,
                                     size_t N, void* stream)
{
    if (!X || !gamma || !rinv || !normed || !out || F == 0 || F > 8 * kRowGroups) return kBadShape;
    const auto s = static_cast<hipStream_t>(stream);
    if (narrow_ok(F, N))
    {
        hipLaunchKernelGGL(k_rms_fwd_narrow, dim3(unsigned(N)), dim3(kNarrowT), 0, s, X, gamma, inv_f, eps, s_raw,
                           scaled, var_eps, rinv, normed, out, unsigned(F), N);
        return launch_status();
    }
    return rms_forward_wide<false>(X, nullptr, nullptr, gamma, inv_f, eps, s_raw, scaled, var_eps, rinv, normed, out,
                                   F, N, s);
}

extern "C" int nnhip_rmsnorm_forward_sum(const float* A, const float* B, float* X, const float* gamma, float inv_f,
                                         float eps, float* s_raw, float* scaled, float* var_eps, float* rinv,
                                         float* normed, float* out, size_t F, size_t N, void* stream)
{
    if (!A || !B || !X || !gamma || !rinv || !normed || !out || F == 0 || F > 8 * kRowGroups) return kBadShape;
    if (!shape_ok(F, N, {A, B, X})) return kBadShape;
    return rms_forward_wide<true>(A, B, X, gamma, inv_f, eps, s_raw, scaled, var_eps, rinv, normed, out, F, N,
                                  static_cast<hipStream_t>(stream));
}

extern "C" int nnhip_rmsnorm_backward(const float* G, const float* gamma, const float* Nrm, const float* rinv,
                                      float inv_f, float* m_raw, float* m, float* dx, size_t F, size_t N,
                                      void* stream)
{
    if (!G || !gamma || !Nrm || !rinv || !m || !dx || F == 0 || F > 8 * kRowGroups) return kBadShape;
    return rms_backward_wide<false>(G, gamma, Nrm, rinv, inv_f, m_raw, m, dx, nullptr, nullptr, F, N,
                                    static_cast<hipStream_t>(stream));
}

extern "C" int nnhip_rmsnorm_backward_add(const float* G, const float* gamma, const float* Nrm, const float* rinv,
                                          float inv_f, float* m_raw, float* m, float* dx, const float* addend,
                                          float* out2, size_t F, size_t N, void* stream)
{
    if (!G || !gamma || !Nrm || !rinv || !m || !dx || !addend || !out2 || F == 0 || F > 8 * kRowGroups)
        return kBadShape;
    if (!shape_ok(F, N, {addend, out2})) return kBadShape;
    return rms_backward_wide<true>(G, gamma, Nrm, rinv, inv_f, m_raw, m, dx, addend, out2, F, N,
                                   static_cast<hipStream_t>(stream));
}

extern "C" int nnhip_colbcast_mul(const float* X, const float* v, float* out, size_t F, size_t N, void* stream)
{
    if (X && v && out && N % 4 != 0)
    {
        const size_t total = F * N;
        if (total == 0) return 0;
        hipLaunchKernelGGL(k_colbcast_mul_narrow, dim3(unsigned((total + kNarrowT - 1) / kNarrowT)), dim3(kNarrowT), 0,
                           static_cast<hipStream_t>(stream), X, v, out, total, N);
        return launch_status();
    }
    if (!shape_ok(F, N, {X, v, out})) return kBadShape;
    return launch_ew(ColBcastMul{X, v, out, N}, F, N, static_cast<hipStream_t>(stream));
}

extern "C" int nnhip_rowbcast_mul(const float* X, const float* v, float* out, size_t F, size_t N, void* stream)
{
    if (!shape_ok(F, N, {X, out})) return kBadShape;
    return launch_ew(RowBcastMul{X, v, out, N}, F, N, static_cast<hipStream_t>(stream));
}

extern "C" int nnhip_rmsnorm_bwd_colsum(const float* G, const float* gamma, const float* normed, float* out, size_t F,
                                        size_t N, void* stream)
{
    if (!shape_ok(F, N, {G, normed, out})) return kBadShape;
    return launch_colsum(GGammaN{G, gamma, normed, N}, out, F, N, static_cast<hipStream_t>(stream));
}

extern "C" int nnhip_rmsnorm_bwd_dx(const float* G, const float* gamma, const float* m, const float* normed,
                                    const float* rinv, float* out, size_t F, size_t N, void* stream)
{
    if (!shape_ok(F, N, {G, m, normed, rinv, out})) return kBadShape;
    return launch_ew(RmsDx{G, gamma, m, normed, rinv, out, N}, F, N, static_cast<hipStream_t>(stream));
}

namespace
{
int rowsum_ggn(const float* G, const float* gamma, const float* normed, float* out, size_t F, size_t N, bool add,
               void* stream)
{
    if (!shape_ok(F, N, {G, normed})) return kBadShape;
    if (F == 0) return 0;
    hipLaunchKernelGGL(k_fused_rowsum_ggn, dim3(unsigned(F)), dim3(kT), 0, static_cast<hipStream_t>(stream), G, gamma,
                       normed, out, unsigned(N / 4), N, add);
    return launch_status();
}
} // namespace

extern "C" int nnhip_rmsnorm_bwd_rowsum(const float* G, const float* gamma, const float* normed, float* out, size_t F,
                                        size_t N, void* stream)
{
    return rowsum_ggn(G, gamma, normed, out, F, N, false, stream);
}

extern "C" int nnhip_rmsnorm_bwd_rowsum_add(const float* G, const float* gamma, const float* normed, float* out,
                                            size_t F, size_t N, void* stream)
{
    return rowsum_ggn(G, gamma, normed, out, F, N, true, stream);
}

extern "C" int nnhip_swiglu_grad_gate(const float* G, const float* up, const float* s, const float* gate, float* out,
                                      size_t count, void* stream)
{
    if (!shape_ok(1, count, {G, up, s, gate, out})) return kBadShape;
    return launch_flat(SwigluGradGate{G, up, s, gate, out}, count, static_cast<hipStream_t>(stream));
}

extern "C" int nnhip_swiglu_grad_up(const float* G, const float* gate, const float* s, float* out, size_t count,
                                    void* stream)
{
    if (!shape_ok(1, count, {G, gate, s, out})) return kBadShape;
    return launch_flat(SwigluGradUp{G, gate, s, out}, count, static_cast<hipStream_t>(stream));
}

extern "C" int nnhip_swiglu_grad_both(const float* G, const float* up, const float* s, const float* gate,
                                      float* out_gate, float* out_up, size_t count, void* stream)
{
    if (!shape_ok(1, count, {G, up, s, gate, out_gate, out_up})) return kBadShape;
    return launch_flat(SwigluGradBoth{G, up, s, gate, out_gate, out_up}, count, static_cast<hipStream_t>(stream));
}
