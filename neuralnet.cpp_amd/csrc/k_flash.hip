// k_flash.hip — one-pass attention chains on the fp32 matrix cores.
//
// The reference's two-pass attention is a chain of engine primitives
// (compute_layer.hpp:1196-1221 forward, :1304-1327 backward):
//   m      = batched_matmul_reduce(Q, K, Max)              cpu_engine.hpp:426-532
//   l      = batched_matmul_softmax_denom(Q, K, m)         cpu_engine.hpp:535-604
//   O      = batched_matmul_softmax_apply(Q, K, V, m, l)   cpu_engine.hpp:607-699
//   P      = batched_matmul(dO, V', transA)                cpu_engine.hpp:335-419
//   dQ, R  = batched_matmul_softmax_backward_q(Q, K, P, m, l)         :702-801
//   dK, dV = batched_matmul_softmax_backward_kv(Q, K, P, G, R, m, l)  :804-915
// HipEngine defers each chain and runs it here, one pass per direction:
//   forward (query lines): online row max and sum (m, l) and the weighted value sum O;
//   backward, query lines: with P_ij = alpha2 dO_i . V'_j recomputed per cell,
//     R_i = sum_j W P,  X_i = sum_j W P k_j,  Y_i = sum_j W k_j,  dQ_i = alpha (X_i - R_i Y_i)
//     (= alpha sum_j W (P - R_i) k_j, the reference's dQ);
//   backward, key lines: dK_j = alpha sum_i W (P - R_i) q_i,  dV_j = sum_i W G_i.
// W_ij = exp(s_ij - m_i) / l_i with s_ij = alpha q_i . k_j + mask_ij; entries whose
// mask is -inf are excluded everywhere, as in the reference.
//
// Operand layouts (the ones the reference's attention layer passes):
//   Q  per batch (K, M)  [dim][query]   (the transA = 1 operand)
//   Kt per batch (K, N)  [dim][key]     (transB = 0)
//   V  per batch (N, D)  [key][dim]     (apply's value rows)
//   dO per batch (Kd, M) [dim][query],  V' per batch (Kd, N) [dim][key]   (P's operands)
//   G  per batch (M, ldg) [query][dim]  (backward_kv's value gradient rows, dims < K used)
// Outputs: m, l, R (batch*M); O (batch*M, D); dQ (batch*K, M); dK, dV (batch*K, N).
//
// Work decomposition. Scores are cut into 32x32 cells; a mask pre-pass marks
// each cell of the shared (M, N) mask as all -inf (skipped), all zero (mask not
// read) or general. A workgroup is 4 waves = 4 consecutive 32-wide lines
// (query tiles for the row kernels, key tiles for the column kernel) that walk
// a range of R cells along the line; the tiles of the other side are staged
// once per cell in LDS (double-buffered, one barrier per cell) and shared by
// the 4 waves. When lines are cut into several ranges, every (line, range)
// writes a partial result and a combine kernel merges them in range order, so
// results never depend on scheduling.
//
// MFMA v_mfma_f32_32x32x2_f32 layout (lane l, h = l/32, c = l%32): A[row c][k h],
// B[k h][col c]; D register r <-> row drow(r,h) = 8(r/4) + 4h + r%4, col c.
// Score chains put the line's tokens on the columns: each lane owns one token
// of the line, the 16 registers hold 16 tokens of the other side, and those
// registers are already the B operand of the value/gradient chains when step r
// contracts over tokens drow(r,0), drow(r,1). Contraction dims are permuted so
// LDS reads are vectors: score step kk reads dim kk + KP/2*h (4 steps per
// 16-byte read); output tile u row i holds dim DU*i + u (one 8-byte read feeds
// both tiles when DU = 2).
#include "flash.hpp"

#include <algorithm>

#include "common.hpp"
#include "nnhip_kernels.h"

namespace nnhip
{
namespace
{

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr float kNegInf = -__builtin_huge_valf();
constexpr float kLog2e = 1.44269504088896340736f;
constexpr int kWaves = 4;
constexpr int kMaxRange = 64;   // cells per range: one 64-bit ballot

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
// exp(x) for x <= 0 (or -inf -> 0) on the hardware exp2.
__device__ __forceinline__ float exp_neg(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }
__device__ __forceinline__ float fmax_f(float a, float b) { return a < b ? b : a; }

// Workgroups are dispatched round-robin over the 8 XCDs (one L2 each); this
// gives each XCD a contiguous run of work items, so the items of one batch
// entry, which re-read its tiles, share an L2.
__device__ __forceinline__ int xcd_item(int bid, int nb)
{
    const int x = bid % 8, k = bid / 8, q = nb / 8, r = nb % 8;
    return x * q + min(x, r) + k;
}

struct Item
{
    int b, grp, rg;
};
// Batch entry, line group (heaviest first: with causal masks later groups
// have more cells) and range of this workgroup.
__device__ __forceinline__ Item item_of(const FlashGeo& g)
{
    const int it = xcd_item(blockIdx.x, gridDim.x), per = g.G * g.NR;
    Item r;
    r.b = it / per;
    const int rem = it % per;
    r.grp = g.G - 1 - rem / g.NR;
    r.rg = rem % g.NR;
    return r;
}

struct Bits
{
    unsigned long long nz, gen;
};
// Non-empty / general cells of this wave's line within [cell0, cell0 + ncell).
// rows: the line is a query tile and cells run along keys; else a key tile, cells along queries.
__device__ __forceinline__ Bits line_bits(const FlashGeo& g, bool rows, int line, int cell0, int ncell)
{
    const int lane = threadIdx.x & 63;
    int cl = 0;
    if (line < (rows ? g.RT : g.CT) && lane < ncell)
    {
        const int x = cell0 + lane;
        cl = !g.cls ? 1 : (rows ? g.cls[(long)line * g.CT + x] : g.cls[(long)x * g.CT + line]);
    }
    return {__ballot(cl != 0), __ballot(cl == 2)};
}

// A 32-token x KP-dim tile of a (dims, T) [dim][token] array, staged
// transposed as [token][dim]. Thread t holds token t%32, dim quads t/32 + 8s.
template <int KP>
struct TTile
{
    static constexpr int NQ = KP / 32;
    float4 r[NQ];
    __device__ __forceinline__ void load(const float* base, int dims, int T, int t0)
    {
        const int tok = threadIdx.x & 31, q0 = threadIdx.x >> 5, t = t0 + tok;
#pragma unroll
        for (int s = 0; s < NQ; ++s)
        {
            const int d0 = 4 * (q0 + 8 * s);
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = (t < T && d0 + e < dims) ? base[(long)(d0 + e) * T + t] : 0.0f;
            r[s] = make_float4(v[0], v[1], v[2], v[3]);
        }
    }
    __device__ __forceinline__ void store(float (*lds)[KP + 4]) const
    {
        const int tok = threadIdx.x & 31, q0 = threadIdx.x >> 5;
#pragma unroll
        for (int s = 0; s < NQ; ++s) *reinterpret_cast<float4*>(&lds[tok][4 * (q0 + 8 * s)]) = r[s];
    }
};

// A 32-token x DP-dim tile of a (T, ld) [token][dim] array (dims < ncols,
// ncols and ld multiples of 4), staged as [token][dim].
template <int DP>
struct RTile
{
    static constexpr int QPR = DP / 4, NQ = DP / 32;
    float4 r[NQ];
    __device__ __forceinline__ void load(const float* base, int ld, int ncols, int T, int t0)
    {
#pragma unroll
        for (int s = 0; s < NQ; ++s)
        {
            const int idx = threadIdx.x + 256 * s, tok = idx / QPR, q = idx % QPR;
            r[s] = (t0 + tok < T && 4 * q < ncols)
                       ? *reinterpret_cast<const float4*>(base + (long)(t0 + tok) * ld + 4 * q)
                       : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    }
    __device__ __forceinline__ void store(float (*lds)[DP + 4]) const
    {
#pragma unroll
        for (int s = 0; s < NQ; ++s)
        {
            const int idx = threadIdx.x + 256 * s, tok = idx / QPR, q = idx % QPR;
            *reinterpret_cast<float4*>(&lds[tok][4 * q]) = r[s];
        }
    }
};

// mask(row, jbase + drow(r, h)) for r = 0..15 (zero past column N).
__device__ __forceinline__ void mask_row16(const float* mrow, int N, int jbase, int h, float* mv)
{
    if ((N & 3) == 0)
    {
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4)
        {
            const int j = jbase + 8 * g4 + 4 * h;
            const float4 v = j < N ? *reinterpret_cast<const float4*>(mrow + j) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            mv[4 * g4 + 0] = v.x;
            mv[4 * g4 + 1] = v.y;
            mv[4 * g4 + 2] = v.z;
            mv[4 * g4 + 3] = v.w;
        }
    }
    else
    {
#pragma unroll
        for (int r = 0; r < 16; ++r)
        {
            const int j = jbase + drow(r, h);
            mv[r] = j < N ? mrow[j] : 0.0f;
        }
    }
}

// Score chain: D[token drow(r,h)][line token c] = sum_k tile[c][k] * reg[k] over KP dims.
template <int KP>
__device__ __forceinline__ f32x16 score_chain(const float (*tile)[KP + 4], const float* reg, int h, int c)
{
    constexpr int KH = KP / 2;
    f32x16 s = zero16();
#pragma unroll
    for (int q4 = 0; q4 < KH / 4; ++q4)
    {
        const float4 a = *reinterpret_cast<const float4*>(&tile[c][KH * h + 4 * q4]);
        s = mfma(a.x, reg[4 * q4 + 0], s);
        s = mfma(a.y, reg[4 * q4 + 1], s);
        s = mfma(a.z, reg[4 * q4 + 2], s);
        s = mfma(a.w, reg[4 * q4 + 3], s);
    }
    return s;
}

// acc[u] += tile^T (dims DU*c + u, tokens drow(r,h)) x w (tokens drow(r,h), line token c).
template <int DP>
__device__ __forceinline__ void value_chain(const float (*tile)[DP + 4], const float* w, int h, int c, f32x16* acc)
{
    constexpr int DU = DP / 32;
#pragma unroll
    for (int r = 0; r < 16; ++r)
    {
        if constexpr (DU == 2)
        {
            const float2 a = *reinterpret_cast<const float2*>(&tile[drow(r, h)][2 * c]);
            acc[0] = mfma(a.x, w[r], acc[0]);
            acc[1] = mfma(a.y, w[r], acc[1]);
        }
        else
            acc[0] = mfma(tile[drow(r, h)][c], w[r], acc[0]);
    }
}

// Same A operand feeding two chains (dQ's X and Y; dK and dV use different tiles).
template <int DP>
__device__ __forceinline__ void value_chain2(const float (*tile)[DP + 4], const float* w1, const float* w2, int h,
                                             int c, f32x16* acc1, f32x16* acc2)
{
    constexpr int DU = DP / 32;
#pragma unroll
    for (int r = 0; r < 16; ++r)
    {
        if constexpr (DU == 2)
        {
            const float2 a = *reinterpret_cast<const float2*>(&tile[drow(r, h)][2 * c]);
            acc1[0] = mfma(a.x, w1[r], acc1[0]);
            acc1[1] = mfma(a.y, w1[r], acc1[1]);
            acc2[0] = mfma(a.x, w2[r], acc2[0]);
            acc2[1] = mfma(a.y, w2[r], acc2[1]);
        }
        else
        {
            const float a = tile[drow(r, h)][c];
            acc1[0] = mfma(a, w1[r], acc1[0]);
            acc2[0] = mfma(a, w2[r], acc2[0]);
        }
    }
}

// Per-lane B operand of a score chain: reg[kk] = X(dim kk + KP/2*h, token t) of a (dims, T) array.
template <int KP>
__device__ __forceinline__ void line_operand(const float* base, int dims, int T, int t, int h, float* reg)
{
    constexpr int KH = KP / 2;
    const int tc = min(t, T - 1);
#pragma unroll
    for (int kk = 0; kk < KH; ++kk)
    {
        const int d = kk + KH * h;
        reg[kk] = (t < T && d < dims) ? base[(long)d * T + tc] : 0.0f;
    }
}

// ── forward: m, l and (WITH_O) O over query lines ──────────────────────────
template <int KP, int DP, bool WITH_O>
__global__ __launch_bounds__(64 * kWaves) void k_flash_fwd(FlashFwdArgs a, FlashGeo g)
{
    constexpr int DU = DP / 32;
    __shared__ __align__(16) float Ks[2][32][KP + 4];
    __shared__ __align__(16) float Vs[WITH_O ? 2 : 1][WITH_O ? 32 : 1][DP + 4];
    __shared__ unsigned long long nz_s[kWaves];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, h = lane >> 5, c = lane & 31;
    const Item it = item_of(g);
    const int line = it.grp * kWaves + wave, qi = line * 32 + c;
    const int cell0 = it.rg * g.R, ncell = min(g.R, g.CT - cell0);
    const Bits bits = line_bits(g, true, line, cell0, ncell);
    if (lane == 0) nz_s[wave] = bits.nz;
    __syncthreads();
    const unsigned long long any = nz_s[0] | nz_s[1] | nz_s[2] | nz_s[3];

    float mrun = kLowest, lrun = 0.0f;
    f32x16 o[DU];
#pragma unroll
    for (int u = 0; u < DU; ++u) o[u] = zero16();

    if (any)
    {
        const float* Qb = a.Q + (long)it.b * a.K * g.M;
        const float* Kb = a.Kt + (long)it.b * a.K * g.N;
        const float* Vb = WITH_O ? a.V + (long)it.b * g.N * a.D : nullptr;
        TTile<KP> kt;
        RTile<DP> vt;
        int cur = __builtin_ctzll(any);
        unsigned long long rest = any & (any - 1);
        kt.load(Kb, a.K, g.N, 32 * (cell0 + cur));
        if constexpr (WITH_O) vt.load(Vb, a.D, a.D, g.N, 32 * (cell0 + cur));
        float qf[KP / 2];
        line_operand<KP>(Qb, a.K, g.M, qi, h, qf);
        const int qc = min(qi, g.M - 1);
        const float* mrow = a.mask ? a.mask + (long)qc * g.N : nullptr;
        kt.store(Ks[0]);
        if constexpr (WITH_O) vt.store(Vs[0]);
        __syncthreads();
        int buf = 0;
        while (true)
        {
            const int nxt = rest ? __builtin_ctzll(rest) : -1;
            if (nxt >= 0)
            {
                kt.load(Kb, a.K, g.N, 32 * (cell0 + nxt));
                if constexpr (WITH_O) vt.load(Vb, a.D, a.D, g.N, 32 * (cell0 + nxt));
            }
            if ((bits.nz >> cur) & 1ull)
            {
                const int jbase = 32 * (cell0 + cur);
                float mv[16];
                if ((bits.gen >> cur) & 1ull)
                    mask_row16(mrow, g.N, jbase, h, mv);
                else
                {
#pragma unroll
                    for (int r = 0; r < 16; ++r) mv[r] = 0.0f;
                }
                const f32x16 s = score_chain<KP>(Ks[buf], qf, h, c);
                float sv[16], cmax = kLowest;
#pragma unroll
                for (int r = 0; r < 16; ++r)
                {
                    sv[r] = jbase + drow(r, h) < g.N ? a.alpha * s[r] + mv[r] : kNegInf;
                    cmax = fmax_f(cmax, sv[r]);
                }
                cmax = fmax_f(cmax, __shfl_xor(cmax, 32));
                const float mnew = fmax_f(mrun, cmax);
                const float scale = exp_neg(mrun - mnew);
                lrun *= scale;
                mrun = mnew;
#pragma unroll
                for (int r = 0; r < 16; ++r)
                {
                    sv[r] = exp_neg(sv[r] - mnew);
                    lrun += sv[r];
                }
                if constexpr (WITH_O)
                {
#pragma unroll
                    for (int u = 0; u < DU; ++u) o[u] *= scale;
                    value_chain<DP>(Vs[buf], sv, h, c, o);
                }
            }
            if (nxt < 0) break;
            kt.store(Ks[buf ^ 1]);
            if constexpr (WITH_O) vt.store(Vs[buf ^ 1]);
            __syncthreads();
            buf ^= 1;
            cur = nxt;
            rest &= rest - 1;
        }
    }
    lrun += __shfl_xor(lrun, 32);
    if (line >= g.RT) return;
    if (g.NR == 1)
    {
        if (qi >= g.M) return;
        const long row = (long)it.b * g.M + qi;
        if (h == 0)
        {
            a.m[row] = mrun;
            a.l[row] = lrun;
        }
        if constexpr (WITH_O)
        {
            const float inv = lrun > 0.0f ? 1.0f / lrun : 0.0f;
            float* orow = a.O + row * a.D;
#pragma unroll
            for (int r = 0; r < 16; ++r)
            {
                const int d0 = DU * drow(r, h);
                if (d0 >= a.D) continue;
                if constexpr (DU == 2)
                    *reinterpret_cast<float2*>(orow + d0) = make_float2(o[0][r] * inv, o[1][r] * inv);
                else
                    orow[d0] = o[0][r] * inv;
            }
        }
        return;
    }
    const long pi = ((long)it.b * g.RT + line) * g.NR + it.rg;
    if (!bits.nz)
    {
        if (lane == 0) g.flag[pi] = 0;
        return;
    }
    float* pp = g.part + pi * g.pw;
    if (h == 0)
    {
        pp[c] = mrun;
        pp[32 + c] = lrun;
    }
    if constexpr (WITH_O)
    {
#pragma unroll
        for (int u = 0; u < DU; ++u)
#pragma unroll
            for (int r = 0; r < 16; ++r) pp[64 + (u * 16 + r) * 64 + lane] = o[u][r];
    }
    if (lane == 0) g.flag[pi] = 1;
}

// Merges a query line's range partials in range order (online max / rescaled sums).
template <int DP, bool WITH_O>
__global__ __launch_bounds__(64) void k_flash_fwd_combine(FlashFwdArgs a, FlashGeo g)
{
    constexpr int DU = DP / 32;
    const int lane = threadIdx.x, h = lane >> 5, c = lane & 31;
    const long lidx = blockIdx.x;
    const int b = static_cast<int>(lidx / g.RT), line = static_cast<int>(lidx % g.RT), qi = line * 32 + c;
    float m = kLowest, l = 0.0f;
    f32x16 o[DU];
#pragma unroll
    for (int u = 0; u < DU; ++u) o[u] = zero16();
    for (int rg = 0; rg < g.NR; ++rg)
    {
        const long pi = lidx * g.NR + rg;
        if (!g.flag[pi]) continue;
        const float* pp = g.part + pi * g.pw;
        const float mr = pp[c], lr = pp[32 + c];
        const float mn = fmax_f(m, mr);
        const float sa = exp_neg(m - mn), sb = exp_neg(mr - mn);
        l = l * sa + lr * sb;
        m = mn;
        if constexpr (WITH_O)
        {
#pragma unroll
            for (int u = 0; u < DU; ++u)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[u][r] = o[u][r] * sa + pp[64 + (u * 16 + r) * 64 + lane] * sb;
        }
    }
    if (qi >= g.M) return;
    const long row = (long)b * g.M + qi;
    if (h == 0)
    {
        a.m[row] = m;
        a.l[row] = l;
    }
    if constexpr (WITH_O)
    {
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        float* orow = a.O + row * a.D;
#pragma unroll
        for (int r = 0; r < 16; ++r)
        {
            const int d0 = DU * drow(r, h);
            if (d0 >= a.D) continue;
            if constexpr (DU == 2)
                *reinterpret_cast<float2*>(orow + d0) = make_float2(o[0][r] * inv, o[1][r] * inv);
            else
                orow[d0] = o[0][r] * inv;
        }
    }
}

// ── backward over query lines: R and dQ ────────────────────────────────────
template <int KP>
__global__ __launch_bounds__(64 * kWaves, 2) void k_flash_bwd_rows(FlashBwdArgs a, FlashGeo g)
{
    constexpr int DU = KP / 32;
    __shared__ __align__(16) float Ks[2][32][KP + 4];   // key tile [key][dim]
    __shared__ __align__(16) float Vs[2][32][KP + 4];   // V' tile [key][dim]
    __shared__ unsigned long long nz_s[kWaves];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, h = lane >> 5, c = lane & 31;
    const Item it = item_of(g);
    const int line = it.grp * kWaves + wave, qi = line * 32 + c;
    const int cell0 = it.rg * g.R, ncell = min(g.R, g.CT - cell0);
    const Bits bits = line_bits(g, true, line, cell0, ncell);
    if (lane == 0) nz_s[wave] = bits.nz;
    __syncthreads();
    const unsigned long long any = nz_s[0] | nz_s[1] | nz_s[2] | nz_s[3];

    float racc = 0.0f;
    f32x16 x[DU], y[DU];
#pragma unroll
    for (int u = 0; u < DU; ++u)
    {
        x[u] = zero16();
        y[u] = zero16();
    }
    if (any)
    {
        const float* Qb = a.Q + (long)it.b * a.K * g.M;
        const float* Kb = a.Kt + (long)it.b * a.K * g.N;
        const float* Ob = a.dO + (long)it.b * a.Kd * g.M;
        const float* Vb = a.Vp + (long)it.b * a.Kd * g.N;
        TTile<KP> kt, vt;
        int cur = __builtin_ctzll(any);
        unsigned long long rest = any & (any - 1);
        kt.load(Kb, a.K, g.N, 32 * (cell0 + cur));
        vt.load(Vb, a.Kd, g.N, 32 * (cell0 + cur));
        float qf[KP / 2], of[KP / 2];
        line_operand<KP>(Qb, a.K, g.M, qi, h, qf);
        line_operand<KP>(Ob, a.Kd, g.M, qi, h, of);
        const int qc = min(qi, g.M - 1);
        const long srow = (long)it.b * g.M + qc;
        const float mi = a.m[srow], li = a.l[srow];
        const float linv = li != 0.0f ? 1.0f / li : 0.0f;
        const float* mrow = a.mask ? a.mask + (long)qc * g.N : nullptr;
        kt.store(Ks[0]);
        vt.store(Vs[0]);
        __syncthreads();
        int buf = 0;
        while (true)
        {
            const int nxt = rest ? __builtin_ctzll(rest) : -1;
            if (nxt >= 0)
            {
                kt.load(Kb, a.K, g.N, 32 * (cell0 + nxt));
                vt.load(Vb, a.Kd, g.N, 32 * (cell0 + nxt));
            }
            if ((bits.nz >> cur) & 1ull)
            {
                const int jbase = 32 * (cell0 + cur);
                float mv[16];
                if ((bits.gen >> cur) & 1ull)
                    mask_row16(mrow, g.N, jbase, h, mv);
                else
                {
#pragma unroll
                    for (int r = 0; r < 16; ++r) mv[r] = 0.0f;
                }
                const f32x16 s = score_chain<KP>(Ks[buf], qf, h, c);
                const f32x16 p = score_chain<KP>(Vs[buf], of, h, c);
                float w[16], wp[16];
#pragma unroll
                for (int r = 0; r < 16; ++r)
                {
                    const float sc = jbase + drow(r, h) < g.N ? a.alpha * s[r] + mv[r] : kNegInf;
                    w[r] = sc == kNegInf ? 0.0f : exp_neg(sc - mi) * linv;
                    wp[r] = w[r] * (a.alpha2 * p[r]);
                    racc += wp[r];
                }
                value_chain2<KP>(Ks[buf], wp, w, h, c, x, y);
            }
            if (nxt < 0) break;
            kt.store(Ks[buf ^ 1]);
            vt.store(Vs[buf ^ 1]);
            __syncthreads();
            buf ^= 1;
            cur = nxt;
            rest &= rest - 1;
        }
    }
    racc += __shfl_xor(racc, 32);
    if (line >= g.RT) return;
    if (g.NR == 1)
    {
        if (qi >= g.M) return;
        if (h == 0) a.R[(long)it.b * g.M + qi] = racc;
        float* dq = a.dQ + (long)it.b * a.K * g.M + qi;
#pragma unroll
        for (int u = 0; u < DU; ++u)
#pragma unroll
            for (int r = 0; r < 16; ++r)
            {
                const int d = DU * drow(r, h) + u;
                if (d < a.K) dq[(long)d * g.M] = a.alpha * (x[u][r] - racc * y[u][r]);
            }
        return;
    }
    const long pi = ((long)it.b * g.RT + line) * g.NR + it.rg;
    if (!bits.nz)
    {
        if (lane == 0) g.flag[pi] = 0;
        return;
    }
    float* pp = g.part + pi * g.pw;
    if (h == 0) pp[c] = racc;
#pragma unroll
    for (int u = 0; u < DU; ++u)
#pragma unroll
        for (int r = 0; r < 16; ++r)
        {
            pp[32 + (u * 16 + r) * 64 + lane] = x[u][r];
            pp[32 + ((DU + u) * 16 + r) * 64 + lane] = y[u][r];
        }
    if (lane == 0) g.flag[pi] = 1;
}

template <int KP>
__global__ __launch_bounds__(64) void k_flash_bwd_rows_combine(FlashBwdArgs a, FlashGeo g)
{
    constexpr int DU = KP / 32;
    const int lane = threadIdx.x, h = lane >> 5, c = lane & 31;
    const long lidx = blockIdx.x;
    const int b = static_cast<int>(lidx / g.RT), line = static_cast<int>(lidx % g.RT), qi = line * 32 + c;
    float racc = 0.0f;
    f32x16 x[DU], y[DU];
#pragma unroll
    for (int u = 0; u < DU; ++u)
    {
        x[u] = zero16();
        y[u] = zero16();
    }
    for (int rg = 0; rg < g.NR; ++rg)
    {
        const long pi = lidx * g.NR + rg;
        if (!g.flag[pi]) continue;
        const float* pp = g.part + pi * g.pw;
        racc += pp[c];
#pragma unroll
        for (int u = 0; u < DU; ++u)
#pragma unroll
            for (int r = 0; r < 16; ++r)
            {
                x[u][r] += pp[32 + (u * 16 + r) * 64 + lane];
                y[u][r] += pp[32 + ((DU + u) * 16 + r) * 64 + lane];
            }
    }
    if (qi >= g.M) return;
    if (h == 0) a.R[(long)b * g.M + qi] = racc;
    float* dq = a.dQ + (long)b * a.K * g.M + qi;
#pragma unroll
    for (int u = 0; u < DU; ++u)
#pragma unroll
        for (int r = 0; r < 16; ++r)
        {
            const int d = DU * drow(r, h) + u;
            if (d < a.K) dq[(long)d * g.M] = a.alpha * (x[u][r] - racc * y[u][r]);
        }
}

// Loads the query-side tiles of one cell of the key-line kernel into registers:
// Q and dO (transposed), G rows, and m, 1/l, R of the 32 queries (threads 0-95).
template <int KP>
__device__ __forceinline__ void stage_cols(TTile<KP>& qt, TTile<KP>& ot, RTile<KP>& gt, float& st, const float* Qb,
                                           const float* Ob, const float* Gb, const float* mb, const float* lb,
                                           const float* Rb, const FlashBwdArgs& a, int M, int i0)
{
    qt.load(Qb, a.K, M, i0);
    ot.load(Ob, a.Kd, M, i0);
    gt.load(Gb, a.ldg, a.K, M, i0);
    if (threadIdx.x < 96)
    {
        const int i = i0 + static_cast<int>(threadIdx.x & 31), which = threadIdx.x >> 5;
        float v = 0.0f;
        if (i < M) v = which == 0 ? mb[i] : which == 1 ? lb[i] : Rb[i];
        st = which == 1 ? (v != 0.0f ? 1.0f / v : 0.0f) : v;
    }
}

// ── backward over key lines: dK and dV ─────────────────────────────────────
template <int KP>
__global__ __launch_bounds__(64 * kWaves, 2) void k_flash_bwd_cols(FlashBwdArgs a, FlashGeo g)
{
    constexpr int DU = KP / 32;
    __shared__ __align__(16) float Qs[2][32][KP + 4];   // query tile [query][dim]
    __shared__ __align__(16) float Os[2][32][KP + 4];   // dO tile [query][dim]
    __shared__ __align__(16) float Gs[2][32][KP + 4];   // G tile [query][dim]
    __shared__ float St[2][3][32];                      // m, 1/l, R of the tile's queries
    __shared__ unsigned long long nz_s[kWaves];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, h = lane >> 5, c = lane & 31;
    const Item it = item_of(g);
    const int line = it.grp * kWaves + wave, kj = line * 32 + c;
    const int cell0 = it.rg * g.R, ncell = min(g.R, g.RT - cell0);
    const Bits bits = line_bits(g, false, line, cell0, ncell);
    if (lane == 0) nz_s[wave] = bits.nz;
    __syncthreads();
    const unsigned long long any = nz_s[0] | nz_s[1] | nz_s[2] | nz_s[3];

    f32x16 dk[DU], dv[DU];
#pragma unroll
    for (int u = 0; u < DU; ++u)
    {
        dk[u] = zero16();
        dv[u] = zero16();
    }
    if (any)
    {
        const float* Qb = a.Q + (long)it.b * a.K * g.M;
        const float* Kb = a.Kt + (long)it.b * a.K * g.N;
        const float* Ob = a.dO + (long)it.b * a.Kd * g.M;
        const float* Vb = a.Vp + (long)it.b * a.Kd * g.N;
        const float* Gb = a.G + (long)it.b * g.M * a.ldg;
        const float* mb = a.m + (long)it.b * g.M;
        const float* lb = a.l + (long)it.b * g.M;
        const float* Rb = a.R + (long)it.b * g.M;
        TTile<KP> qt, ot;
        RTile<KP> gt;
        float st = 0.0f;
        int cur = __builtin_ctzll(any);
        unsigned long long rest = any & (any - 1);
        stage_cols(qt, ot, gt, st, Qb, Ob, Gb, mb, lb, Rb, a, g.M, 32 * (cell0 + cur));
        float kf[KP / 2], vf[KP / 2];
        line_operand<KP>(Kb, a.K, g.N, kj, h, kf);
        line_operand<KP>(Vb, a.Kd, g.N, kj, h, vf);
        const int jc = min(kj, g.N - 1);
        qt.store(Qs[0]);
        ot.store(Os[0]);
        gt.store(Gs[0]);
        if (threadIdx.x < 96) St[0][threadIdx.x >> 5][threadIdx.x & 31] = st;
        __syncthreads();
        int buf = 0;
        while (true)
        {
            const int nxt = rest ? __builtin_ctzll(rest) : -1;
            if (nxt >= 0) stage_cols(qt, ot, gt, st, Qb, Ob, Gb, mb, lb, Rb, a, g.M, 32 * (cell0 + nxt));
            if ((bits.nz >> cur) & 1ull)
            {
                const int ibase = 32 * (cell0 + cur);
                float mv[16];
                if ((bits.gen >> cur) & 1ull)
                {
#pragma unroll
                    for (int r = 0; r < 16; ++r) mv[r] = a.mask[(long)min(ibase + drow(r, h), g.M - 1) * g.N + jc];
                }
                else
                {
#pragma unroll
                    for (int r = 0; r < 16; ++r) mv[r] = 0.0f;
                }
                const f32x16 s = score_chain<KP>(Qs[buf], kf, h, c);
                const f32x16 p = score_chain<KP>(Os[buf], vf, h, c);
                float w[16], ds[16];
#pragma unroll
                for (int r = 0; r < 16; ++r)
                {
                    const int ii = drow(r, h);
                    const bool ok = ibase + ii < g.M && kj < g.N;
                    const float sc = ok ? a.alpha * s[r] + mv[r] : kNegInf;
                    w[r] = sc == kNegInf ? 0.0f : exp_neg(sc - St[buf][0][ii]) * St[buf][1][ii];
                    ds[r] = w[r] * (a.alpha2 * p[r] - St[buf][2][ii]);
                }
                value_chain<KP>(Gs[buf], w, h, c, dv);
                value_chain<KP>(Qs[buf], ds, h, c, dk);
            }
            if (nxt < 0) break;
            qt.store(Qs[buf ^ 1]);
            ot.store(Os[buf ^ 1]);
            gt.store(Gs[buf ^ 1]);
            if (threadIdx.x < 96) St[buf ^ 1][threadIdx.x >> 5][threadIdx.x & 31] = st;
            __syncthreads();
            buf ^= 1;
            cur = nxt;
            rest &= rest - 1;
        }
    }
    if (line >= g.CT) return;
    if (g.NR == 1)
    {
        if (kj >= g.N) return;
        float* dkb = a.dK + (long)it.b * a.K * g.N + kj;
        float* dvb = a.dV + (long)it.b * a.K * g.N + kj;
#pragma unroll
        for (int u = 0; u < DU; ++u)
#pragma unroll
            for (int r = 0; r < 16; ++r)
            {
                const int d = DU * drow(r, h) + u;
                if (d < a.K)
                {
                    dkb[(long)d * g.N] = a.alpha * dk[u][r];
                    dvb[(long)d * g.N] = dv[u][r];
                }
            }
        return;
    }
    const long pi = ((long)it.b * g.CT + line) * g.NR + it.rg;
    if (!bits.nz)
    {
        if (lane == 0) g.flag[pi] = 0;
        return;
    }
    float* pp = g.part + pi * g.pw;
#pragma unroll
    for (int u = 0; u < DU; ++u)
#pragma unroll
        for (int r = 0; r < 16; ++r)
        {
            pp[(u * 16 + r) * 64 + lane] = dk[u][r];
            pp[((DU + u) * 16 + r) * 64 + lane] = dv[u][r];
        }
    if (lane == 0) g.flag[pi] = 1;
}

template <int KP>
__global__ __launch_bounds__(64) void k_flash_bwd_cols_combine(FlashBwdArgs a, FlashGeo g)
{
    constexpr int DU = KP / 32;
    const int lane = threadIdx.x, h = lane >> 5, c = lane & 31;
    const long lidx = blockIdx.x;
    const int b = static_cast<int>(lidx / g.CT), line = static_cast<int>(lidx % g.CT), kj = line * 32 + c;
    f32x16 dk[DU], dv[DU];
#pragma unroll
    for (int u = 0; u < DU; ++u)
    {
        dk[u] = zero16();
        dv[u] = zero16();
    }
    for (int rg = 0; rg < g.NR; ++rg)
    {
        const long pi = lidx * g.NR + rg;
        if (!g.flag[pi]) continue;
        const float* pp = g.part + pi * g.pw;
#pragma unroll
        for (int u = 0; u < DU; ++u)
#pragma unroll
            for (int r = 0; r < 16; ++r)
            {
                dk[u][r] += pp[(u * 16 + r) * 64 + lane];
                dv[u][r] += pp[((DU + u) * 16 + r) * 64 + lane];
            }
    }
    if (kj >= g.N) return;
    float* dkb = a.dK + (long)b * a.K * g.N + kj;
    float* dvb = a.dV + (long)b * a.K * g.N + kj;
#pragma unroll
    for (int u = 0; u < DU; ++u)
#pragma unroll
        for (int r = 0; r < 16; ++r)
        {
            const int d = DU * drow(r, h) + u;
            if (d < a.K)
            {
                dkb[(long)d * g.N] = a.alpha * dk[u][r];
                dvb[(long)d * g.N] = dv[u][r];
            }
        }
}

// Mask cell classes: 0 all -inf, 1 all zero, 2 general.
__global__ __launch_bounds__(256) void k_flash_classify(const float* __restrict__ mask, int M, int N, int CT,
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
    if (threadIdx.x == 0) cls[(long)ib * CT + jb] = !finite ? 0 : (nonzero ? 2 : 1);
}

// ── host side ────────────────────────────────────────────────────────────────
size_t align256(size_t x) { return (x + 255) / 256 * 256; }

int pad32(size_t x) { return x <= 32 ? 32 : 64; }

// Ranges per line: one range when there are enough workgroups to fill the GPU
// twice over, else lines are cut (at most 64 cells per range, at least 8).
void ranges(size_t items, int cells, int& R, int& NR)
{
    int nr = (cells + kMaxRange - 1) / kMaxRange;
    if (items < 512)
    {
        const int want = static_cast<int>((1024 + items - 1) / items);
        const int cap = (cells + 7) / 8;
        nr = std::max(nr, std::min(want, cap));
    }
    nr = std::max(nr, 1);
    R = (cells + nr - 1) / nr;
    NR = (cells + R - 1) / R;
}

struct Plan
{
    FlashGeo rows, cols;
    size_t cls_off, flag_off, part_off, bytes;
};

Plan plan(size_t batch, size_t M, size_t N, int fwd_pw, int rows_pw, int cols_pw, bool backward)
{
    Plan p{};
    const int RT = static_cast<int>((M + 31) / 32), CT = static_cast<int>((N + 31) / 32);
    auto geo = [&](bool rows_side, int pw) {
        FlashGeo g{};
        g.M = static_cast<int>(M);
        g.N = static_cast<int>(N);
        g.RT = RT;
        g.CT = CT;
        const int lines = rows_side ? RT : CT, cells = rows_side ? CT : RT;
        g.G = (lines + kWaves - 1) / kWaves;
        ranges(batch * g.G, cells, g.R, g.NR);
        g.pw = pw;
        return g;
    };
    p.rows = geo(true, backward ? rows_pw : fwd_pw);
    p.cols = geo(false, cols_pw);
    p.cls_off = 0;
    p.flag_off = align256(static_cast<size_t>(RT) * CT);
    size_t flags = batch * RT * static_cast<size_t>(p.rows.NR), part = 0;
    if (p.rows.NR > 1) part = batch * RT * static_cast<size_t>(p.rows.NR) * p.rows.pw;
    if (backward)
    {
        flags = std::max(flags, batch * CT * static_cast<size_t>(p.cols.NR));
        if (p.cols.NR > 1) part = std::max(part, batch * CT * static_cast<size_t>(p.cols.NR) * p.cols.pw);
    }
    p.part_off = p.flag_off + align256(flags * sizeof(int));
    p.bytes = p.part_off + align256(part * sizeof(float));
    return p;
}

void bind(FlashGeo& g, const Plan& p, void* ws, bool masked)
{
    auto* base = static_cast<unsigned char*>(ws);
    g.cls = masked ? base + p.cls_off : nullptr;
    g.flag = reinterpret_cast<int*>(base + p.flag_off);
    g.part = reinterpret_cast<float*>(base + p.part_off);
}

int classify(const float* mask, const FlashGeo& g, void* ws, hipStream_t s)
{
    if (!mask) return 0;
    hipLaunchKernelGGL(k_flash_classify, dim3(g.CT, g.RT), dim3(256), 0, s, mask, g.M, g.N, g.CT,
                       static_cast<unsigned char*>(ws));
    return launch_status();
}

unsigned grid_of(const FlashGeo& g, size_t batch)
{
    return static_cast<unsigned>(batch * static_cast<size_t>(g.G) * g.NR);
}

int fwd_pw(int DP) { return 64 + 32 * DP; }
int rows_pw(int KP) { return 32 + 64 * KP; }
int cols_pw(int KP) { return 64 * KP; }

template <int KP, int DP, bool WITH_O>
int launch_fwd(const FlashFwdArgs& a, FlashGeo g, size_t batch, hipStream_t s)
{
    hipLaunchKernelGGL((k_flash_fwd<KP, DP, WITH_O>), dim3(grid_of(g, batch)), dim3(64 * kWaves), 0, s, a, g);
    if (int rc = launch_status()) return rc;
    if (g.NR == 1) return 0;
    hipLaunchKernelGGL((k_flash_fwd_combine<DP, WITH_O>), dim3(static_cast<unsigned>(batch * g.RT)), dim3(64), 0, s,
                       a, g);
    return launch_status();
}

template <int KP>
int launch_bwd(const FlashBwdArgs& a, FlashGeo gr, FlashGeo gc, size_t batch, hipStream_t s)
{
    hipLaunchKernelGGL((k_flash_bwd_rows<KP>), dim3(grid_of(gr, batch)), dim3(64 * kWaves), 0, s, a, gr);
    if (int rc = launch_status()) return rc;
    if (gr.NR > 1)
    {
        hipLaunchKernelGGL((k_flash_bwd_rows_combine<KP>), dim3(static_cast<unsigned>(batch * gr.RT)), dim3(64), 0,
                           s, a, gr);
        if (int rc = launch_status()) return rc;
    }
    hipLaunchKernelGGL((k_flash_bwd_cols<KP>), dim3(grid_of(gc, batch)), dim3(64 * kWaves), 0, s, a, gc);
    if (int rc = launch_status()) return rc;
    if (gc.NR == 1) return 0;
    hipLaunchKernelGGL((k_flash_bwd_cols_combine<KP>), dim3(static_cast<unsigned>(batch * gc.CT)), dim3(64), 0, s, a,
                       gc);
    return launch_status();
}

} // namespace

bool flash_supported(size_t batch, size_t M, size_t N, size_t K, size_t D)
{
    // Head dims up to 64 and value widths up to 64 in multiples of 4 (16-byte
    // value rows); grids of at most 2^31 workgroups; sizes that fit int.
    return batch >= 1 && M >= 1 && N >= 1 && K >= 1 && K <= 64 && D >= 1 && D <= 64 && D % 4 == 0 &&
           M <= (size_t{1} << 24) && N <= (size_t{1} << 24) && batch <= (size_t{1} << 20) &&
           batch * ((M + 31) / 32) * ((N + 31) / 32) <= (size_t{1} << 30);
}

size_t flash_workspace_bytes(size_t batch, size_t M, size_t N, size_t K, size_t D, bool backward)
{
    const int KP = pad32(K), DP = pad32(D);
    return plan(batch, M, N, fwd_pw(DP), rows_pw(KP), cols_pw(KP), backward).bytes;
}

int flash_forward(const FlashFwdArgs& a, size_t batch, void* ws, hipStream_t s)
{
    const int KP = pad32(static_cast<size_t>(a.K)), DP = a.O ? pad32(static_cast<size_t>(a.D)) : 32;
    Plan p = plan(batch, static_cast<size_t>(a.M), static_cast<size_t>(a.N), fwd_pw(DP), rows_pw(KP),
                  cols_pw(KP), false);
    bind(p.rows, p, ws, a.mask != nullptr);
    if (int rc = classify(a.mask, p.rows, ws, s)) return rc;
    if (!a.O) return KP == 32 ? launch_fwd<32, 32, false>(a, p.rows, batch, s) : launch_fwd<64, 32, false>(a, p.rows, batch, s);
    if (KP == 32) return DP == 32 ? launch_fwd<32, 32, true>(a, p.rows, batch, s) : launch_fwd<32, 64, true>(a, p.rows, batch, s);
    return DP == 32 ? launch_fwd<64, 32, true>(a, p.rows, batch, s) : launch_fwd<64, 64, true>(a, p.rows, batch, s);
}

int flash_backward(const FlashBwdArgs& a, size_t batch, void* ws, hipStream_t s)
{
    const int KP = pad32(static_cast<size_t>(std::max(a.K, a.Kd)));
    Plan p = plan(batch, static_cast<size_t>(a.M), static_cast<size_t>(a.N), fwd_pw(32), rows_pw(KP), cols_pw(KP),
                  true);
    bind(p.rows, p, ws, a.mask != nullptr);
    bind(p.cols, p, ws, a.mask != nullptr);
    if (int rc = classify(a.mask, p.rows, ws, s)) return rc;
    return KP == 32 ? launch_bwd<32>(a, p.rows, p.cols, batch, s) : launch_bwd<64>(a, p.rows, p.cols, batch, s);
}

} // namespace nnhip

// ── C-ABI (include/nnhip_kernels.h) ─────────────────────────────────────────
extern "C" int nnhip_flash_supported(size_t batch, size_t M, size_t N, size_t K, size_t D)
{
    return nnhip::flash_supported(batch, M, N, K, D) ? 1 : 0;
}

extern "C" size_t nnhip_flash_workspace_bytes(size_t batch, size_t M, size_t N, size_t K, size_t D, int backward)
{
    return nnhip::flash_workspace_bytes(batch, M, N, K, D, backward != 0);
}

extern "C" int nnhip_flash_forward(const float* Q, const float* Kt, const float* V, const float* mask, float* m,
                                   float* l, float* O, size_t batch, size_t M, size_t N, size_t K, size_t D,
                                   float alpha, void* workspace, void* stream)
{
    if (!Q || !Kt || !m || !l || !workspace || (O && !V)) return -1;
    if (!nnhip::flash_supported(batch, M, N, K, O ? D : 4)) return -3;
    nnhip::FlashFwdArgs a{Q, Kt, V, mask, m, l, O, static_cast<int>(M), static_cast<int>(N), static_cast<int>(K),
                          static_cast<int>(O ? D : 4), alpha};
    return nnhip::flash_forward(a, batch, workspace, static_cast<hipStream_t>(stream));
}

extern "C" int nnhip_flash_backward(const float* Q, const float* Kt, const float* dO, const float* Vp, const float* G,
                                    size_t ldg, const float* mask, const float* m, const float* l, float* R,
                                    float* dQ, float* dK, float* dV, size_t batch, size_t M, size_t N, size_t K,
                                    size_t Kd, float alpha, float alpha2, void* workspace, void* stream)
{
    if (!Q || !Kt || !dO || !Vp || !G || !m || !l || !R || !dQ || !dK || !dV || !workspace) return -1;
    if (!nnhip::flash_supported(batch, M, N, K > Kd ? K : Kd, 4) || K % 4 != 0 || ldg < K || ldg % 4 != 0) return -3;
    nnhip::FlashBwdArgs a{Q, Kt, dO, Vp, G, mask, m, l, R, dQ, dK, dV, static_cast<int>(M), static_cast<int>(N),
                          static_cast<int>(K), static_cast<int>(Kd), static_cast<int>(ldg), alpha, alpha2};
    return nnhip::flash_backward(a, batch, workspace, static_cast<hipStream_t>(stream));
}
