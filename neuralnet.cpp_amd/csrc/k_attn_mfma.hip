// k_attn_mfma.hip — the fused attention primitives on the fp32 matrix cores.
//
// Same semantics as the general path in k_attention.hip (CPU engine,
// cpu_engine.hpp:426-915), for head dims K <= 128 (and value width D <= 128):
//   s_ij = alpha * dot_k(Q(i,k), Kt(k,j)) + mask(i,j),  W_ij = exp(s_ij - m_i) / l_i  (0 where s_ij = -inf)
// with Q(i,k) = A_b(i,k) and Kt(k,j) = B_b(k,j) in the transpose conventions of
// ComputeEngine (compute_engine.hpp:217-276).
//
// Every score tile is one v_mfma_f32_32x32x2_f32 chain over k. The forward and
// backward_q kernels compute it transposed, S^T = Kt^T Q (rows = keys,
// columns = queries): each lane then owns one query (column l%32), so row
// statistics need no cross-lane work until the very end, and the score
// registers are already laid out as the B operand of the next MFMA
// (O^T = V^T W^T, dQ^T = Kt dS^T). backward_kv computes S = Q Kt (rows =
// queries) so that W and dS feed dK = Q^T dS and dV = G^T W the same way.
//
// MFMA 32x32x2 operand layout (lane l, h = l/32, c = l%32), step r of 2 k's:
//   A[row c][k h], B[k h][col c];  D register r <-> row drow(r,h), col c,
//   drow(r,h) = 8*(r/4) + 4*h + r%4.
// Feeding D registers as a B operand, step r consumes reduction indices
// drow(r,0) and drow(r,1): over r = 0..15 each of the 32 is used once, and the
// A operand is read with the same index map.
//
// Masks: a pre-pass classifies every 32x32 (query, key) cell of the shared
// (M,N) mask as all -inf (skipped), all zero (no mask read) or general, so a
// causal or document mask costs only the cells that hold allowed pairs.
#include "attn_mfma.hpp"
#include "common.hpp"

namespace nnhip
{
namespace
{

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr float kNegInf = -__builtin_huge_valf();
constexpr int JT = 64;   // keys per step (forward, backward_q)
constexpr int IT = 64;   // queries per step (backward_kv)
constexpr int LP = 1;    // LDS row padding: rows of 65 floats are bank-conflict free both ways

__device__ __forceinline__ f32x16 mfma(float a, float b, f32x16 c)
{
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 zero16()
{
    f32x16 z;
#pragma unroll
    for (int r = 0; r < 16; ++r) z[r] = 0.0f;
    return z;
}
__device__ __forceinline__ int drow(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }

__device__ __forceinline__ float q_at(const AttnArgs& d, const float* Ab, int i, int k)
{
    return d.tA ? Ab[(long)k * d.M + i] : Ab[(long)i * d.K + k];
}
__device__ __forceinline__ float kt_at(const AttnArgs& d, const float* Bb, int k, int j)
{
    return d.tB ? Bb[(long)j * d.K + k] : Bb[(long)k * d.N + j];
}
// Class of the 32x32 cell (query block ib, key block jb): 0 skip, 1 no mask add, 2 general.
__device__ __forceinline__ int cell(const AttnArgs& d, int ib, int jb)
{
    if (!d.mask) return 1;
    if (!d.cls) return 2;
    return d.cls[(long)ib * d.n_j32 + jb];
}

__global__ __launch_bounds__(256) void k_mask_classify(const float* __restrict__ mask, int M, int N, int n_j32,
                                                       unsigned char* __restrict__ cls)
{
    const int jb = blockIdx.x, ib = blockIdx.y;
    int finite = 0, nonzero = 0;
    for (int e = threadIdx.x; e < 1024; e += 256)
    {
        const int i = ib * 32 + e / 32, j = jb * 32 + e % 32;
        if (i < M && j < N)
        {
            const float v = mask[(long)i * N + j];
            finite |= (v != kNegInf);
            nonzero |= (v != 0.0f);
        }
    }
    finite = __syncthreads_or(finite);
    nonzero = __syncthreads_or(nonzero);
    if (threadIdx.x == 0) cls[(long)ib * n_j32 + jb] = !finite ? 0 : (nonzero ? 2 : 1);
}

// Stages Ks[k][jj] = Kt(k, j0 + jj) for k < KP, jj < JT (zero outside K x N).
template <int KP, int NT>
__device__ __forceinline__ void stage_keys(const AttnArgs& d, const float* Bb, int j0, float (*Ks)[JT + LP])
{
    for (int e = threadIdx.x; e < KP * JT; e += NT)
    {
        int k, jj;
        if (d.tB) { jj = e / KP; k = e % KP; }   // consecutive threads walk consecutive addresses
        else { k = e / JT; jj = e % JT; }
        const int j = j0 + jj;
        Ks[k][jj] = (k < d.K && j < d.N) ? kt_at(d, Bb, k, j) : 0.0f;
    }
}

// Does any wave of the block need key step [j0, j0+64) for query rows starting at qb0?
template <int WQ>
__device__ __forceinline__ bool block_needs_keys(const AttnArgs& d, int qb0, int j0)
{
    for (int w = 0; w < WQ; ++w)
        for (int t = 0; t < 2; ++t)
        {
            const int ib = qb0 / 32 + w, jb = j0 / 32 + t;
            if (ib * 32 < d.M && jb * 32 < d.N && cell(d, ib, jb) != 0) return true;
        }
    return false;
}

// Scores of one transposed 32x32 tile: sv[r] for key j0 + drow(r,h), query qi.
__device__ __forceinline__ void scores_t(const AttnArgs& d, const f32x16& s, int qi, int jbase, int h, int cl,
                                         float* sv)
{
#pragma unroll
    for (int r = 0; r < 16; ++r)
    {
        const int j = jbase + drow(r, h);
        float x = d.alpha * s[r];
        if (j >= d.N || qi >= d.M)
            x = kNegInf;
        else if (cl == 2)
            x += d.mask[(long)qi * d.N + j];
        sv[r] = x;
    }
}

// ── forward: row max (bmm_reduce Max, reduce_cols), denominators, apply ──────
template <int KP, int WQ, int MODE>
__global__ __launch_bounds__(64 * WQ) void k_attn_fwd(AttnArgs d, const float* __restrict__ row_max,
                                                      const float* __restrict__ denom, const float* __restrict__ V,
                                                      int D, float* __restrict__ out)
{
    constexpr int NT = 64 * WQ;
    constexpr bool APPLY = MODE == kFwdApply;
    __shared__ float Ks[KP][JT + LP];
    __shared__ float Vs[APPLY ? JT : 1][APPLY ? 128 + LP : 1];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, h = lane >> 5, c = lane & 31;
    const int qblk = gridDim.x - 1 - blockIdx.x;   // last query blocks carry the most causal work: start them first
    const int b = blockIdx.y;
    const int qb0 = qblk * 32 * WQ, i0 = qb0 + wave * 32, qi = i0 + c;
    const float* Ab = d.A + (long)b * d.M * d.K;
    const float* Bb = d.B + (long)b * d.K * d.N;

    float qf[KP / 2];   // B operand of S^T: Q(qi, 2kk + h)
#pragma unroll
    for (int kk = 0; kk < KP / 2; ++kk)
    {
        const int k = 2 * kk + h;
        qf[kk] = (qi < d.M && k < d.K) ? q_at(d, Ab, qi, k) : 0.0f;
    }
    float m_i = 0.0f, inv_l = 0.0f;
    if (MODE != kFwdMax && qi < d.M) m_i = row_max[(long)b * d.M + qi];
    if (APPLY && qi < d.M) inv_l = 1.0f / denom[(long)b * d.M + qi];
    float red = MODE == kFwdMax ? kLowest : 0.0f;
    const int DU = (D + 31) / 32;
    f32x16 acc_o[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) acc_o[u] = zero16();

    const int steps = (d.N + JT - 1) / JT;
    for (int st = 0; st < steps; ++st)
    {
        const int j0 = st * JT;
        if (!block_needs_keys<WQ>(d, qb0, j0)) continue;
        __syncthreads();
        stage_keys<KP, NT>(d, Bb, j0, Ks);
        if constexpr (APPLY)
        {
            const int dw = DU * 32;
            for (int e = threadIdx.x; e < JT * dw; e += NT)
            {
                const int jj = e / dw, k = e % dw, j = j0 + jj;
                Vs[jj][k] = (k < D && j < d.N) ? V[((long)b * d.N + j) * D + k] : 0.0f;
            }
        }
        __syncthreads();
        if (i0 >= d.M) continue;
#pragma unroll
        for (int t = 0; t < 2; ++t)
        {
            const int jbase = j0 + 32 * t;
            if (jbase >= d.N) continue;
            const int cl = cell(d, i0 / 32, jbase / 32);
            if (cl == 0) continue;
            f32x16 s = zero16();
#pragma unroll
            for (int kk = 0; kk < KP / 2; ++kk) s = mfma(Ks[2 * kk + h][32 * t + c], qf[kk], s);
            float sv[16];
            scores_t(d, s, qi, jbase, h, cl, sv);
            if constexpr (MODE == kFwdMax)
            {
#pragma unroll
                for (int r = 0; r < 16; ++r) red = fmax_std(red, sv[r]);
            }
            else if constexpr (MODE == kFwdDenom)
            {
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (sv[r] != kNegInf) red += expf(sv[r] - m_i);
            }
            else
            {
                float w[16];
#pragma unroll
                for (int r = 0; r < 16; ++r) w[r] = sv[r] == kNegInf ? 0.0f : expf(sv[r] - m_i) * inv_l;
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    if (u < DU)
                    {
#pragma unroll
                        for (int r = 0; r < 16; ++r)
                            acc_o[u] = mfma(Vs[32 * t + drow(r, h)][32 * u + c], w[r], acc_o[u]);
                    }
            }
        }
    }
    if constexpr (!APPLY)
    {
        const float o = __shfl_xor(red, 32, 64);
        red = MODE == kFwdMax ? fmax_std(red, o) : red + o;
        if (h == 0 && qi < d.M) out[(long)b * d.M + qi] = red;
    }
    else if (qi < d.M)
    {
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if (u < DU)
            {
#pragma unroll
                for (int r = 0; r < 16; ++r)
                {
                    const int k = 32 * u + drow(r, h);
                    if (k < D) out[((long)b * d.M + qi) * D + k] = acc_o[u][r];
                }
            }
    }
}

// ── backward_q: pass 0 R_i = sum_j W P; pass 1 dQ^T[k][i] = alpha sum_j Kt(k,j) W (P - R_i) ──
template <int KP, int WQ>
__global__ __launch_bounds__(64 * WQ) void k_attn_bwd_q(AttnArgs d, const float* __restrict__ P,
                                                        const float* __restrict__ row_max,
                                                        const float* __restrict__ denom, float* __restrict__ dQ,
                                                        float* __restrict__ R)
{
    constexpr int NT = 64 * WQ;
    __shared__ float Ks[KP][JT + LP];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, h = lane >> 5, c = lane & 31;
    const int qblk = gridDim.x - 1 - blockIdx.x;
    const int b = blockIdx.y;
    const int qb0 = qblk * 32 * WQ, i0 = qb0 + wave * 32, qi = i0 + c;
    const float* Ab = d.A + (long)b * d.M * d.K;
    const float* Bb = d.B + (long)b * d.K * d.N;
    const float* prow = P + ((long)b * d.M + (qi < d.M ? qi : 0)) * d.N;

    float qf[KP / 2];
#pragma unroll
    for (int kk = 0; kk < KP / 2; ++kk)
    {
        const int k = 2 * kk + h;
        qf[kk] = (qi < d.M && k < d.K) ? q_at(d, Ab, qi, k) : 0.0f;
    }
    const float m_i = qi < d.M ? row_max[(long)b * d.M + qi] : 0.0f;
    const float inv_l = qi < d.M ? 1.0f / denom[(long)b * d.M + qi] : 0.0f;
    float r_i = 0.0f, rsum = 0.0f;
    f32x16 acc[KP / 32];
#pragma unroll
    for (int u = 0; u < KP / 32; ++u) acc[u] = zero16();

    const int steps = (d.N + JT - 1) / JT;
    for (int pass = 0; pass < 2; ++pass)
    {
        for (int st = 0; st < steps; ++st)
        {
            const int j0 = st * JT;
            if (!block_needs_keys<WQ>(d, qb0, j0)) continue;
            __syncthreads();
            stage_keys<KP, NT>(d, Bb, j0, Ks);
            __syncthreads();
            if (i0 >= d.M) continue;
#pragma unroll
            for (int t = 0; t < 2; ++t)
            {
                const int jbase = j0 + 32 * t;
                if (jbase >= d.N) continue;
                const int cl = cell(d, i0 / 32, jbase / 32);
                if (cl == 0) continue;
                f32x16 s = zero16();
#pragma unroll
                for (int kk = 0; kk < KP / 2; ++kk) s = mfma(Ks[2 * kk + h][32 * t + c], qf[kk], s);
                float sv[16];
                scores_t(d, s, qi, jbase, h, cl, sv);
                float w[16], p[16];
#pragma unroll
                for (int r = 0; r < 16; ++r)
                {
                    const int j = jbase + drow(r, h);
                    w[r] = sv[r] == kNegInf ? 0.0f : expf(sv[r] - m_i) * inv_l;
                    p[r] = (qi < d.M && j < d.N) ? prow[j] : 0.0f;
                }
                if (pass == 0)
                {
#pragma unroll
                    for (int r = 0; r < 16; ++r) rsum += w[r] * p[r];
                }
                else
                {
#pragma unroll
                    for (int u = 0; u < KP / 32; ++u)
                    {
#pragma unroll
                        for (int r = 0; r < 16; ++r)
                            acc[u] = mfma(Ks[32 * u + c][32 * t + drow(r, h)], w[r] * (p[r] - r_i), acc[u]);
                    }
                }
            }
        }
        if (pass == 0)
        {
            r_i = rsum + __shfl_xor(rsum, 32, 64);
            if (h == 0 && qi < d.M) R[(long)b * d.M + qi] = r_i;
        }
    }
    if (qi < d.M)
    {
#pragma unroll
        for (int u = 0; u < KP / 32; ++u)
        {
#pragma unroll
            for (int r = 0; r < 16; ++r)
            {
                const int k = 32 * u + drow(r, h);
                if (k < d.K) dQ[((long)b * d.K + k) * d.M + qi] = d.alpha * acc[u][r];
            }
        }
    }
}

// ── backward_kv: dK[k][j] = alpha sum_i Q(i,k) W (P - R_i), dV[k][j] = sum_i G(i,k) W ──
template <int KP, int WQ>
__global__ __launch_bounds__(64 * WQ) void k_attn_bwd_kv(AttnArgs d, const float* __restrict__ P,
                                                         const float* __restrict__ G, int D,
                                                         const float* __restrict__ R,
                                                         const float* __restrict__ row_max,
                                                         const float* __restrict__ denom, float* __restrict__ dK,
                                                         float* __restrict__ dV)
{
    constexpr int NT = 64 * WQ;
    __shared__ float Qs[IT][KP + LP];
    __shared__ float Gs[IT][KP + LP];
    __shared__ float ms[IT], ls[IT], rs[IT];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, h = lane >> 5, c = lane & 31;
    const int b = blockIdx.y;
    const int kb0 = blockIdx.x * 32 * WQ, j0w = kb0 + wave * 32, kj = j0w + c;
    const float* Ab = d.A + (long)b * d.M * d.K;
    const float* Bb = d.B + (long)b * d.K * d.N;

    float kf[KP / 2];   // B operand of S = Q Kt: Kt(2kk + h, kj)
#pragma unroll
    for (int kk = 0; kk < KP / 2; ++kk)
    {
        const int k = 2 * kk + h;
        kf[kk] = (kj < d.N && k < d.K) ? kt_at(d, Bb, k, kj) : 0.0f;
    }
    f32x16 acck[KP / 32], accv[KP / 32];
#pragma unroll
    for (int u = 0; u < KP / 32; ++u)
    {
        acck[u] = zero16();
        accv[u] = zero16();
    }

    const int steps = (d.M + IT - 1) / IT;
    for (int st = 0; st < steps; ++st)
    {
        const int i0 = st * IT;
        bool need = false;
        for (int w = 0; w < WQ && !need; ++w)
            for (int t = 0; t < 2; ++t)
            {
                const int ib = i0 / 32 + t, jb = kb0 / 32 + w;
                if (ib * 32 < d.M && jb * 32 < d.N && cell(d, ib, jb) != 0) need = true;
            }
        if (!need) continue;
        __syncthreads();
        for (int e = threadIdx.x; e < IT * KP; e += NT)
        {
            int ii, k;
            if (d.tA) { k = e / IT; ii = e % IT; }
            else { ii = e / KP; k = e % KP; }
            const int i = i0 + ii;
            Qs[ii][k] = (i < d.M && k < d.K) ? q_at(d, Ab, i, k) : 0.0f;
        }
        for (int e = threadIdx.x; e < IT * KP; e += NT)
        {
            const int ii = e / KP, k = e % KP, i = i0 + ii;
            Gs[ii][k] = (i < d.M && k < d.K) ? G[((long)b * d.M + i) * D + k] : 0.0f;
        }
        for (int ii = threadIdx.x; ii < IT; ii += NT)
        {
            const int i = i0 + ii;
            const bool ok = i < d.M;
            ms[ii] = ok ? row_max[(long)b * d.M + i] : 0.0f;
            ls[ii] = ok ? denom[(long)b * d.M + i] : 1.0f;
            rs[ii] = ok ? R[(long)b * d.M + i] : 0.0f;
        }
        __syncthreads();
        if (j0w >= d.N) continue;
#pragma unroll
        for (int t = 0; t < 2; ++t)
        {
            const int ibase = i0 + 32 * t;
            if (ibase >= d.M) continue;
            const int cl = cell(d, ibase / 32, j0w / 32);
            if (cl == 0) continue;
            f32x16 s = zero16();
#pragma unroll
            for (int kk = 0; kk < KP / 2; ++kk) s = mfma(Qs[32 * t + c][2 * kk + h], kf[kk], s);
            float w[16], ds[16];
#pragma unroll
            for (int r = 0; r < 16; ++r)
            {
                const int ii = 32 * t + drow(r, h), i = i0 + ii;
                float x = d.alpha * s[r];
                float p = 0.0f;
                if (i >= d.M || kj >= d.N)
                    x = kNegInf;
                else
                {
                    if (cl == 2) x += d.mask[(long)i * d.N + kj];
                    p = P[((long)b * d.M + i) * d.N + kj];
                }
                w[r] = x == kNegInf ? 0.0f : expf(x - ms[ii]) / ls[ii];
                ds[r] = w[r] * (p - rs[ii]);
            }
#pragma unroll
            for (int u = 0; u < KP / 32; ++u)
            {
#pragma unroll
                for (int r = 0; r < 16; ++r)
                {
                    const int ii = 32 * t + drow(r, h);
                    acck[u] = mfma(Qs[ii][32 * u + c], ds[r], acck[u]);
                    accv[u] = mfma(Gs[ii][32 * u + c], w[r], accv[u]);
                }
            }
        }
    }
    if (kj < d.N)
    {
#pragma unroll
        for (int u = 0; u < KP / 32; ++u)
        {
#pragma unroll
            for (int r = 0; r < 16; ++r)
            {
                const int k = 32 * u + drow(r, h);
                if (k < d.K)
                {
                    dK[((long)b * d.K + k) * d.N + kj] = d.alpha * acck[u][r];
                    dV[((long)b * d.K + k) * d.N + kj] = accv[u][r];
                }
            }
        }
    }
}

// Queries (or keys) per workgroup: 4 waves when that still gives the GPU
// enough workgroups, else 2.
int waves_for(size_t rows, size_t batch)
{
    const size_t blocks4 = (rows + 127) / 128 * batch;
    return blocks4 >= 512 ? 4 : 2;
}

template <int KP, int WQ, int MODE>
int launch_fwd(const AttnArgs& d, size_t batch, const float* row_max, const float* denom, const float* V, int D,
               float* out, hipStream_t s)
{
    const unsigned gx = static_cast<unsigned>((d.M + 32 * WQ - 1) / (32 * WQ));
    hipLaunchKernelGGL((k_attn_fwd<KP, WQ, MODE>), dim3(gx, static_cast<unsigned>(batch)), dim3(64 * WQ), 0, s, d,
                       row_max, denom, V, D, out);
    return launch_status();
}

template <int KP, int WQ>
int launch_bwd(const AttnArgs& d, size_t batch, bool kv, const float* P, const float* G, int D, const float* R_in,
               const float* row_max, const float* denom, float* o1, float* o2, hipStream_t s)
{
    if (!kv)
    {
        const unsigned gx = static_cast<unsigned>((d.M + 32 * WQ - 1) / (32 * WQ));
        hipLaunchKernelGGL((k_attn_bwd_q<KP, WQ>), dim3(gx, static_cast<unsigned>(batch)), dim3(64 * WQ), 0, s, d,
                           P, row_max, denom, o1, o2);
    }
    else
    {
        const unsigned gx = static_cast<unsigned>((d.N + 32 * WQ - 1) / (32 * WQ));
        hipLaunchKernelGGL((k_attn_bwd_kv<KP, WQ>), dim3(gx, static_cast<unsigned>(batch)), dim3(64 * WQ), 0, s,
                           d, P, G, D, R_in, row_max, denom, o1, o2);
    }
    return launch_status();
}

} // namespace

size_t attn_workspace_bytes(size_t M, size_t N)
{
    const size_t cells = ((M + 31) / 32) * ((N + 31) / 32);
    return (cells + 255) / 256 * 256;
}

bool attn_mfma_supported(size_t batch, size_t M, size_t N, size_t K)
{
    return K >= 1 && K <= 128 && batch >= 1 && batch <= 65535 && M <= (1u << 30) && N <= (1u << 30);
}

int attn_prepare(AttnArgs& d, void* workspace, hipStream_t s)
{
    d.n_j32 = static_cast<int>((static_cast<size_t>(d.N) + 31) / 32);
    d.cls = nullptr;
    if (!d.mask || !workspace || d.M == 0 || d.N == 0 || (d.M + 31) / 32 > 65535) return 0;
    auto* cls = static_cast<unsigned char*>(workspace);
    hipLaunchKernelGGL(k_mask_classify, dim3(static_cast<unsigned>(d.n_j32), static_cast<unsigned>((d.M + 31) / 32)),
                       dim3(256), 0, s, d.mask, d.M, d.N, d.n_j32, cls);
    d.cls = cls;
    return launch_status();
}

int attn_mfma_forward(const AttnArgs& d, size_t batch, int mode, const float* row_max, const float* denom,
                      const float* V, size_t D, float* out, hipStream_t s)
{
    if (mode == kFwdApply && (D == 0 || D > 128)) return -3;
    const bool big = d.K > 64;
    const int wq = waves_for(static_cast<size_t>(d.M), batch);
    const int Di = static_cast<int>(D);
#define NNHIP_FWD(KP, WQ)                                                                                          \
    switch (mode)                                                                                                  \
    {                                                                                                              \
    case kFwdMax: return launch_fwd<KP, WQ, kFwdMax>(d, batch, row_max, denom, V, Di, out, s);                    \
    case kFwdDenom: return launch_fwd<KP, WQ, kFwdDenom>(d, batch, row_max, denom, V, Di, out, s);                \
    default: return launch_fwd<KP, WQ, kFwdApply>(d, batch, row_max, denom, V, Di, out, s);                       \
    }
    if (!big && wq == 4) { NNHIP_FWD(64, 4) }
    if (!big) { NNHIP_FWD(64, 2) }
    if (wq == 4) { NNHIP_FWD(128, 4) }
    NNHIP_FWD(128, 2)
#undef NNHIP_FWD
}

int attn_mfma_backward(const AttnArgs& d, size_t batch, bool kv, const float* P, const float* G, size_t D,
                       const float* R_in, const float* row_max, const float* denom, float* o1, float* o2,
                       hipStream_t s)
{
    const bool big = d.K > 64;
    const int wq = waves_for(static_cast<size_t>(kv ? d.N : d.M), batch);
    const int Di = static_cast<int>(D);
    if (!big && wq == 4) return launch_bwd<64, 4>(d, batch, kv, P, G, Di, R_in, row_max, denom, o1, o2, s);
    if (!big) return launch_bwd<64, 2>(d, batch, kv, P, G, Di, R_in, row_max, denom, o1, o2, s);
    if (wq == 4) return launch_bwd<128, 4>(d, batch, kv, P, G, Di, R_in, row_max, denom, o1, o2, s);
    return launch_bwd<128, 2>(d, batch, kv, P, G, Di, R_in, row_max, denom, o1, o2, s);
}

} // namespace nnhip
