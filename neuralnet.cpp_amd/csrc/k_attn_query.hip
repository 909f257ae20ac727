// k_attn_query.hip — attention of one query per batch entry (one head of one
// token in incremental inference, reference compute_layer.hpp:1426-1511):
//
//   s_j = alpha q . k_j + mask[j]   (j < N)
//   m = max_j s_j,  l = sum_j exp(s_j - m),  O = sum_j exp(s_j - m) v_j / l
//
// the same m / l / O as the one-pass forward (k_flash.hip) gives for M = 1:
// m is lowest() and l = 0, O = 0 when every key is masked (-inf).
//
// Keys and values are read where they lie, through strides: element k of key
// j of entry b at Kp[b kb + j kj + k kk] (values likewise with vb, vj, vd). A
// KV cache of (seq, heads * d) rows is read in place (kb = d, kj = heads * d,
// kk = 1), so the per-token transposes of the cache that the reference's
// formulation implies are not needed; the transposed per-head layout
// (kb = d N, kj = 1, kk = N) works too.
//
// One workgroup takes 256 keys of one entry: a thread per key forms the
// score, the workgroup's maximum and sum follow, and 16 groups of 16 threads
// (4 value dims each) accumulate p_j v_j over every 16th key. Entries with
// more keys use several workgroups, whose (m, l, O) partials a second kernel
// merges in key order.
#include "common.hpp"
#include "nnhip_kernels.h"

namespace nnhip
{
namespace
{

constexpr int kQChunk = 256;          // keys per workgroup
constexpr int kQMaxDim = 64;          // head and value dims
constexpr float kQLog2e = 1.4426950408889634f;

struct QueryArgs
{
    const float* Q;
    const float* Kp;
    const float* V;
    const float* mask;
    float* m;
    float* l;
    float* O;
    float* P;      // probabilities (batch, N), or nullptr
    float* part;   // chunks > 1: per (entry, chunk) m, l, then D unnormalised sums
    long kb, kj, kk, vb, vj, vd, mask_bs;
    int N, K, D, chunks;
    float alpha;
};

// VK: key dims contiguous and 16-byte aligned (float4 reads); VV: likewise for values.
// Every load a thread needs (its key, its mask entry, its value rows) is
// issued before the first wait, so the launch costs about one memory latency.
template <bool VK, bool VV>
__global__ __launch_bounds__(256) void k_attn_query(QueryArgs a)
{
    __shared__ float qs[kQMaxDim];
    __shared__ float ps[kQChunk];
    __shared__ float red[2][4];
    __shared__ float4 acc_s[16][kQMaxDim / 4];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int c = blockIdx.x;
    const long b = blockIdx.y;
    const int j = c * kQChunk + t;
    const bool key = j < a.N;
    const float* kr = a.Kp + b * a.kb + (long)j * a.kj;
    float4 kv[kQMaxDim / 4];
    if constexpr (VK)
    {
        const float4* k4 = reinterpret_cast<const float4*>(kr);
        const int K4 = a.K / 4;
#pragma unroll
        for (int i = 0; i < kQMaxDim / 4; ++i)
            if (key && i < K4) kv[i] = k4[i];
    }
    const float mval = key && a.mask ? a.mask[b * a.mask_bs + j] : 0.0f;
    // value rows of thread (g, dg): dims 4 dg .. 4 dg + 3 of keys g, g + 16, ... of the chunk
    const int dg = t & 15, g = t >> 4;
    const int D4 = (a.D + 3) / 4;
    const int nk = min(kQChunk, a.N - c * kQChunk);
    const float* vbase = a.V + b * a.vb + (long)c * kQChunk * a.vj;
    float4 vv[kQChunk / 16];
    if constexpr (VV)
    {
#pragma unroll
        for (int u = 0; u < kQChunk / 16; ++u)
            if (dg < D4 && g + 16 * u < nk) vv[u] = reinterpret_cast<const float4*>(vbase + (long)(g + 16 * u) * a.vj)[dg];
    }
    if (t < a.K) qs[t] = a.Q[b * a.K + t];
    __syncthreads();

    float s = -__builtin_inff();
    if (key)
    {
        float dot = 0.0f;
        if constexpr (VK)
        {
            const int K4 = a.K / 4;
#pragma unroll
            for (int i = 0; i < kQMaxDim / 4; ++i)
                if (i < K4)
                {
                    dot = __builtin_fmaf(qs[4 * i], kv[i].x, dot);
                    dot = __builtin_fmaf(qs[4 * i + 1], kv[i].y, dot);
                    dot = __builtin_fmaf(qs[4 * i + 2], kv[i].z, dot);
                    dot = __builtin_fmaf(qs[4 * i + 3], kv[i].w, dot);
                }
        }
        else
        {
            for (int k = 0; k < a.K; ++k) dot = __builtin_fmaf(qs[k], kr[(long)k * a.kk], dot);
        }
        {
#pragma clang fp contract(off)
            s = a.alpha * dot;
            if (a.mask) s = s + mval;
        }
    }
    // Maximum over the chunk (lowest() when every key is -inf, as the one-pass forward keeps it).
    float mx = fmax_std(kLowest, wave_max(s));
    if (lane == 0) red[0][wave] = mx;
    __syncthreads();
    mx = fmax_std(fmax_std(red[0][0], red[0][1]), fmax_std(red[0][2], red[0][3]));
    const float mb = mx == kLowest ? 0.0f : mx * kQLog2e;
    const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s, kQLog2e, -mb));   // 0 for -inf
    ps[t] = p;
    const float ws = wave_sum(p);
    if (lane == 0) red[1][wave] = ws;
    __syncthreads();
    const float lsum = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]);
    // The probabilities (a chunk's own, relative to its maximum, when the merge rescales them).
    if (a.P && key) a.P[b * a.N + j] = a.chunks == 1 ? p * (lsum > 0.0f ? 1.0f / lsum : 0.0f) : p;

    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (dg < D4)
    {
#pragma unroll
        for (int u = 0; u < kQChunk / 16; ++u)
        {
            const int jj = g + 16 * u;
            if (jj >= nk) continue;
            const float w = ps[jj];
            float4 v;
            if constexpr (VV)
                v = vv[u];
            else
            {
                const float* vr = vbase + (long)jj * a.vj;
                const int d0 = 4 * dg;
                v.x = vr[(long)d0 * a.vd];
                v.y = d0 + 1 < a.D ? vr[(long)(d0 + 1) * a.vd] : 0.0f;
                v.z = d0 + 2 < a.D ? vr[(long)(d0 + 2) * a.vd] : 0.0f;
                v.w = d0 + 3 < a.D ? vr[(long)(d0 + 3) * a.vd] : 0.0f;
            }
            acc.x = __builtin_fmaf(w, v.x, acc.x);
            acc.y = __builtin_fmaf(w, v.y, acc.y);
            acc.z = __builtin_fmaf(w, v.z, acc.z);
            acc.w = __builtin_fmaf(w, v.w, acc.w);
        }
        acc_s[g][dg] = acc;
    }
    __syncthreads();
    if (t >= a.D) return;
    float o = 0.0f;
    for (int gg = 0; gg < 16; ++gg)
    {
        const float4 v = acc_s[gg][t >> 2];
        const int r = t & 3;
        o += r == 0 ? v.x : r == 1 ? v.y : r == 2 ? v.z : v.w;
    }
    if (a.chunks == 1)
    {
        if (t == 0)
        {
            a.m[b] = mx;
            a.l[b] = lsum;
        }
        const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
        a.O[b * a.D + t] = o * inv;
        return;
    }
    float* pp = a.part + (b * a.chunks + c) * (2 + a.D);
    if (t == 0)
    {
        pp[0] = mx;
        pp[1] = lsum;
    }
    pp[2 + t] = o;
}

// Merges the chunks of an entry in key order: one workgroup of 64 threads per entry.
__global__ __launch_bounds__(64) void k_attn_query_merge(QueryArgs a)
{
    const int t = threadIdx.x;
    const long b = blockIdx.x;
    float m = kLowest, l = 0.0f, o = 0.0f;
    for (int c = 0; c < a.chunks; ++c)
    {
        const float* pp = a.part + (b * a.chunks + c) * (2 + a.D);
        const float mc = pp[0], lc = pp[1];
        const float mn = fmax_std(m, mc);
        const float sa = __builtin_amdgcn_exp2f((m - mn) * kQLog2e), sb = __builtin_amdgcn_exp2f((mc - mn) * kQLog2e);
        l = l * sa + lc * sb;
        if (t < a.D) o = o * sa + pp[2 + t] * sb;
        m = mn;
    }
    if (t == 0)
    {
        a.m[b] = m;
        a.l[b] = l;
    }
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    if (t < a.D) a.O[b * a.D + t] = o * inv;
    if (!a.P) return;
    for (int c = 0; c < a.chunks; ++c)
    {
        const float mc = a.part[(b * a.chunks + c) * (2 + a.D)];
        const float f = __builtin_amdgcn_exp2f((mc - m) * kQLog2e) * inv;
        const int j1 = min(a.N, (c + 1) * kQChunk);
        for (int j = c * kQChunk + t; j < j1; j += 64) a.P[b * a.N + j] *= f;
    }
}

size_t query_chunks(size_t N) { return (N + kQChunk - 1) / kQChunk; }

} // namespace
} // namespace nnhip

using namespace nnhip;

extern "C" size_t nnhip_attn_query_workspace_bytes(size_t batch, size_t N, size_t D)
{
    const size_t c = query_chunks(N);
    return c > 1 ? batch * c * (2 + D) * sizeof(float) : 0;
}

extern "C" int nnhip_attn_query(const float* Q, const float* Kp, long kb, long kj, long kk, const float* V, long vb,
                                long vj, long vd, const float* mask, long mask_bs, float* m, float* l, float* O,
                                float* P, size_t batch, size_t N, size_t K, size_t D, float alpha, void* workspace,
                                void* stream)
{
    if (batch == 0) return 0;
    if (!Q || !Kp || !V || !m || !l || !O || N == 0 || K == 0 || K > kQMaxDim || D == 0 || D > kQMaxDim ||
        batch > 65535 || N > 0x7fffffffu || kb < 0 || kj < 0 || kk < 0 || vb < 0 || vj < 0 || vd < 0 || mask_bs < 0)
        return -1;
    const size_t chunks = query_chunks(N);
    if (chunks > 65535 || (chunks > 1 && !workspace)) return -1;
    QueryArgs a{Q, Kp, V, mask, m, l, O, P, static_cast<float*>(workspace), kb, kj, kk, vb, vj, vd, mask_bs,
                static_cast<int>(N), static_cast<int>(K), static_cast<int>(D), static_cast<int>(chunks), alpha};
    const bool vk = kk == 1 && K % 4 == 0 && kb % 4 == 0 && kj % 4 == 0 && aligned16(Kp);
    const bool vv = vd == 1 && D % 4 == 0 && vb % 4 == 0 && vj % 4 == 0 && aligned16(V);
    auto s = static_cast<hipStream_t>(stream);
    const dim3 grid(static_cast<unsigned>(chunks), static_cast<unsigned>(batch));
    if (vk && vv)
        hipLaunchKernelGGL((k_attn_query<true, true>), grid, dim3(256), 0, s, a);
    else if (vk)
        hipLaunchKernelGGL((k_attn_query<true, false>), grid, dim3(256), 0, s, a);
    else if (vv)
        hipLaunchKernelGGL((k_attn_query<false, true>), grid, dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL((k_attn_query<false, false>), grid, dim3(256), 0, s, a);
    if (int rc = launch_status()) return rc;
    if (chunks > 1)
    {
        hipLaunchKernelGGL(k_attn_query_merge, dim3(static_cast<unsigned>(batch)), dim3(64), 0, s, a);
        return launch_status();
    }
    return 0;
}
