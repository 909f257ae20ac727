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
#include <cstdint>
#include <type_traits>

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
// v_max_f32; for the finite and -inf scores here the same as (a < b ? b : a).
__device__ __forceinline__ float fmax_f(float a, float b) { return __builtin_fmaxf(a, b); }

// Buffer loads with the hardware range check: a load whose byte offset is at
// or past the resource's size returns 0 without touching memory, so padding
// elements (offset kOob) are zero with no branch around the load. A resource
// covers one batch entry's array, below 2 GiB (flash_supported). Word 3 sets
// the 32-bit data format that untyped loads need on gfx9-family parts.
using Rsrc = __amdgpu_buffer_rsrc_t;
constexpr unsigned kOob = 0x80000000u;
__device__ __forceinline__ Rsrc rsrc(const float* base, long floats)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, static_cast<int>(floats * 4), 0x00020000);
}
// off when sgn >= 0, else an out-of-range offset (bit 31 set; resources are
// below 2 GiB). Integer arithmetic only: a select here can be turned into a
// branch around the load, with a wait for every load in flight inside it.
__device__ __forceinline__ unsigned oob_if_neg(unsigned off, int sgn)
{
    return off | (static_cast<unsigned>(sgn) & kOob);
}
__device__ __forceinline__ float bload(Rsrc r, unsigned off)
{
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
__device__ __forceinline__ float4 bload4(Rsrc r, unsigned off)
{
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
}

// Workgroups are dispatched round-robin over the 8 XCDs (one L2 each); this
// gives each XCD a contiguous run of work items, so the items of one batch
// entry, which re-read its tiles, share an L2. Within an XCD the k-th and the
// (k + n/2)-th workgroups end up on the same CU, so the second half of the run
// is taken in reverse: with items ordered heaviest first, each CU then gets
// one heavy and one light item (measured: 93 -> 70 us on a causal T = 512
// forward).
__device__ __forceinline__ int xcd_item(int bid, int nb)
{
    const int x = bid % 8, q = nb / 8, r = nb % 8, n = q + (x < r ? 1 : 0), half = (n + 1) / 2;
    int k = bid / 8;
    if (k >= half) k = n - 1 - (k - half);
    return x * q + min(x, r) + k;
}

struct Item
{
    int b, grp, rg;
};
// Batch entry, line group and range of this workgroup. With an order table
// (k_flash_order: items by cell count, laid out so that each CU's resident
// workgroups add up to about the same work) the workgroup takes the item the
// table names; an entry outside the grid is never used (identity instead).
// Without one, groups run heaviest first within each batch entry (with causal
// masks later groups have more cells).
__device__ __forceinline__ Item item_of(const FlashGeo& g)
{
    int it = xcd_item(blockIdx.x, gridDim.x);
    if (g.order)
    {
        const int o = g.order[blockIdx.x];
        it = (o >= 0 && o < static_cast<int>(gridDim.x)) ? o : static_cast<int>(blockIdx.x);
    }
    const int per = g.G * g.NR;
    Item r;
    r.b = it / per;
    const int rem = it % per;
    r.grp = g.G - 1 - rem / g.NR;
    r.rg = rem % g.NR;
    return r;
}

// Arguments and cell tables of the row that batch entry b (uniform over the
// workgroup) belongs to: the row's arguments are pre-offset, so b indexes them.
template <class Args>
__device__ __forceinline__ Args row_args(const FlashSet<Args>& t, FlashGeo& g, int b)
{
    const int row = __builtin_amdgcn_readfirstlane(b / t.hpr);
    g.cls = t.cls[row];
    return t.a[row];
}

// This range's cells of a line (ballots: bit x <-> cell rg*R + x, non-empty /
// general) and which of the line's ranges are non-empty. R is a power of two
// <= 64, so every range lies inside one 64-cell ballot; lines are scanned one
// 64-cell chunk per lane load. rows: the line is a query tile and cells run
// along keys; else a key tile, cells along queries.
struct LineWork
{
    unsigned long long nz, gen, ranges;
    int nne;
};
__device__ __forceinline__ LineWork line_work(const FlashGeo& g, bool rows, int b, int line, int rg)
{
    LineWork w{0ull, 0ull, 0ull, 0};
    if (line >= (rows ? g.RT : g.CT)) return w;
    const int cells = rows ? g.CT : g.RT, lane = threadIdx.x & 63;
    const unsigned char* cls = g.cls ? g.cls + (long)b * g.cls_bs : nullptr;
    const unsigned long long lowR = g.R >= 64 ? ~0ull : ((1ull << g.R) - 1);
    for (int x0 = 0; x0 < cells; x0 += 64)
    {
        const int x = x0 + lane;
        int cl = 0;
        if (x < cells) cl = !cls ? 1 : (rows ? cls[(long)line * g.CT + x] : cls[(long)x * g.CT + line]);
        const unsigned long long nz = __ballot(cl != 0), gen = __ballot(cl == 2);
        const int r_end = min(g.NR, (x0 + 64) / g.R);
        for (int r = x0 / g.R; r < r_end; ++r)
        {
            const int sh = r * g.R - x0;
            const unsigned long long bits = (nz >> sh) & lowR;
            if (bits) w.ranges |= 1ull << r;
            if (r == rg)
            {
                w.nz = bits;
                w.gen = (gen >> sh) & lowR;
            }
        }
    }
    w.nne = __popcll(w.ranges);
    return w;
}
// Who writes a line's outputs: with one non-empty range its workgroup writes
// them directly (range 0 when the line has none); with several, each writes a
// partial and the combine kernel merges them.
__device__ __forceinline__ bool direct_writer(const LineWork& w, int rg)
{
    return w.nne == 1 ? w.nz != 0 : (w.nne == 0 && rg == 0);
}

// A 32-token x KP-dim tile of a (dims, T) [dim][token] array, staged
// transposed as [token][dim]. Thread t holds token t%32, dim quads t/32 + 8s.
template <int KP>
struct TTile
{
    static constexpr int NQ = KP / 32;
    float4 r[NQ];
    __device__ __forceinline__ void load(const float* base, int dims, int T, int t0, int tid)
    {
        const Rsrc rs = rsrc(base, (long)dims * T);
        const int tok = tid & 31, q0 = tid >> 5, t = t0 + tok;
#pragma unroll
        for (int s = 0; s < NQ; ++s)
        {
            const int d0 = 4 * (q0 + 8 * s);
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)   // dims past the array fall past the resource by themselves
                v[e] = bload(rs, oob_if_neg(4u * static_cast<unsigned>((d0 + e) * T + t), T - 1 - t));
            r[s] = make_float4(v[0], v[1], v[2], v[3]);
        }
    }
    __device__ __forceinline__ void store(float (*lds)[KP + 4], int tid) const
    {
        const int tok = tid & 31, q0 = tid >> 5;
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
    __device__ __forceinline__ void load(const float* base, int ld, int ncols, int T, int t0, int tid)
    {
        const Rsrc rs = rsrc(base, (long)T * ld);
#pragma unroll
        for (int s = 0; s < NQ; ++s)
        {
            const int idx = tid + 256 * s, tok = idx / QPR, q = idx % QPR;
            r[s] = bload4(rs, oob_if_neg(4u * static_cast<unsigned>((t0 + tok) * ld + 4 * q),
                                         (T - 1 - t0 - tok) | (ncols - 1 - 4 * q)));
        }
    }
    __device__ __forceinline__ void store(float (*lds)[DP + 4], int tid) const
    {
#pragma unroll
        for (int s = 0; s < NQ; ++s)
        {
            const int idx = tid + 256 * s, tok = idx / QPR, q = idx % QPR;
            *reinterpret_cast<float4*>(&lds[tok][4 * q]) = r[s];
        }
    }
};

// A row of an (M, N) array of one batch entry: the entry's resource and the
// row's byte offset.
struct MRow
{
    Rsrc rs;
    unsigned row;
};
__device__ __forceinline__ MRow mrow_of(const float* batch_base, int M, int N, int row)
{
    return MRow{rsrc(batch_base, (long)M * N), 4u * static_cast<unsigned>(row) * static_cast<unsigned>(N)};
}

// X(row, jbase + drow(r, h)) for r = 0..15 (zero past column N).
__device__ __forceinline__ void mask_row16(const MRow& x, int N, int jbase, int h, float* mv)
{
    if ((N & 3) == 0)
    {
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4)
        {
            const int j = jbase + 8 * g4 + 4 * h;
            const float4 v = bload4(x.rs, oob_if_neg(x.row + 4u * j, N - 1 - j));
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
            mv[r] = bload(x.rs, oob_if_neg(x.row + 4u * j, N - 1 - j));
        }
    }
}

// Score chain: D[token drow(r,h)][line token c] = sum_k tile[c][k] * reg[k] over KP dims.
// Scheduling fence after a chain's LDS reads when PRE: only VALU, SALU and
// transcendental instructions may move across it, so the reads are all issued
// before the first MFMA and the chain runs without waiting on LDS (costs the
// registers of the whole A operand).
template <bool PRE>
__device__ __forceinline__ void operands_first()
{
    if constexpr (PRE) __builtin_amdgcn_sched_barrier(0x0406);
}

template <int KP, bool PRE = false>
__device__ __forceinline__ f32x16 score_chain(const float (*tile)[KP + 4], const float* reg, int h, int c)
{
    constexpr int KH = KP / 2;
    float4 a[KH / 4];
#pragma unroll
    for (int q4 = 0; q4 < KH / 4; ++q4) a[q4] = *reinterpret_cast<const float4*>(&tile[c][KH * h + 4 * q4]);
    operands_first<PRE>();
    f32x16 s = zero16();
#pragma unroll
    for (int q4 = 0; q4 < KH / 4; ++q4)
    {
        s = mfma(a[q4].x, reg[4 * q4 + 0], s);
        s = mfma(a[q4].y, reg[4 * q4 + 1], s);
        s = mfma(a[q4].z, reg[4 * q4 + 2], s);
        s = mfma(a[q4].w, reg[4 * q4 + 3], s);
    }
    return s;
}

// acc[u] += tile^T (dims DU*c + u, tokens drow(r,h)) x w (tokens drow(r,h), line token c).
template <int DP, bool PRE = false>
__device__ __forceinline__ void value_chain(const float (*tile)[DP + 4], const float* w, int h, int c, f32x16* acc)
{
    constexpr int DU = DP / 32;
    if constexpr (DU == 2)
    {
        float2 a[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) a[r] = *reinterpret_cast<const float2*>(&tile[drow(r, h)][2 * c]);
        operands_first<PRE>();
#pragma unroll
        for (int r = 0; r < 16; ++r)
        {
            acc[0] = mfma(a[r].x, w[r], acc[0]);
            acc[1] = mfma(a[r].y, w[r], acc[1]);
        }
    }
    else
    {
        float a[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) a[r] = tile[drow(r, h)][c];
        operands_first<PRE>();
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[0] = mfma(a[r], w[r], acc[0]);
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
// Writes m, l (and O / l) of one query line, or its range partial: m, l, unnormalised O.
template <int DP, bool WITH_O>
__device__ __forceinline__ void fwd_store(const FlashFwdArgs& a, const FlashGeo& g, const LineWork& lw, int b,
                                          int line, int rg, float mrun, float lrun, const f32x16* o)
{
    constexpr int DU = DP / 32;
    const int lane = threadIdx.x & 63, h = lane >> 5, c = lane & 31, qi = line * 32 + c;
    if (line >= g.RT) return;
    if (direct_writer(lw, rg))
    {
        if (qi >= g.M) return;
        const long row = (long)b * g.M + qi;
        if (h == 0)
        {
            a.m[row] = mrun;
            a.l[row] = lrun;
        }
        if constexpr (WITH_O)
        {
            const float inv = lrun > 0.0f ? 1.0f / lrun : 0.0f;
            if (a.o_dm)
            {
                float* ocol = a.O + (long)b * a.D * g.M + qi;   // O per batch (D, M)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                {
                    const int d0 = DU * drow(r, h);
                    if (d0 >= a.D) continue;
#pragma unroll
                    for (int u = 0; u < DU; ++u) ocol[(long)(d0 + u) * g.M] = o[u][r] * inv;
                }
                return;
            }
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
    if (lw.nne <= 1 || !lw.nz) return;
    float* pp = g.part + (((long)b * g.RT + line) * g.NR + rg) * g.pw;
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
}

// Scores of one cell for this lane's query (16 keys drow(r,h) of the cell):
// alpha * dot + mask, -inf for keys past N. Returns the cell's row maximum.
template <bool FULL, bool MASKED>
__device__ __forceinline__ float cell_scores(const f32x16& s, float alpha, const MRow& mrow, int N, int jbase, int h,
                                             float* x)
{
    float mv[16];
    if constexpr (MASKED) mask_row16(mrow, N, jbase, h, mv);
#pragma unroll
    for (int r = 0; r < 16; ++r)
    {
        float v = alpha * s[r];
        if constexpr (MASKED) v += mv[r];
        if constexpr (!FULL) v = jbase + drow(r, h) < N ? v : kNegInf;
        x[r] = v;
    }
    // Pairwise tree: 4 levels of independent v_max instead of a 16-long chain.
    float t8[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) t8[r] = fmax_f(x[r], x[r + 8]);
#pragma unroll
    for (int r = 0; r < 4; ++r) t8[r] = fmax_f(t8[r], t8[r + 4]);
    return fmax_f(kLowest, fmax_f(fmax_f(t8[0], t8[2]), fmax_f(t8[1], t8[3])));
}

// Forward workgroup: 4 waves on 4 consecutive query lines (32 queries each)
// walking the non-empty cells of their range CPS (1 or 2) at a time. A step
// stages the key and value tiles of its cells in LDS (double-buffered, one
// barrier per step); each wave computes the scores of its active cells,
// updates its online max / sum once per step (one cross-lane max, one
// rescale, skipped when no row maximum moved) and accumulates the weighted
// values.
template <int KP, int DP, bool WITH_O, bool VDM, int CPS>
__global__ __launch_bounds__(64 * kWaves, CPS == 1 ? 3 : 2) void k_flash_fwd(FlashFwdSet t, FlashGeo g)
{
    constexpr int DU = DP / 32;
    __shared__ __align__(16) float Ks[2][CPS][32][KP + 4];
    __shared__ __align__(16) float Vs[WITH_O ? 2 : 1][WITH_O ? CPS : 1][WITH_O ? 32 : 1][DP + 4];
    __shared__ unsigned long long nz_s[kWaves];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, h = lane >> 5, c = lane & 31;
    const Item it = item_of(g);
    const FlashFwdArgs a = row_args(t, g, it.b);
    const int line = it.grp * kWaves + wave, qi = line * 32 + c;
    const LineWork lw = line_work(g, true, it.b, line, it.rg);
    if (lane == 0) nz_s[wave] = lw.nz;
    __syncthreads();
    const unsigned long long any = nz_s[0] | nz_s[1] | nz_s[2] | nz_s[3];

    float mrun = kLowest, lrun = 0.0f;
    f32x16 o[DU];
#pragma unroll
    for (int u = 0; u < DU; ++u) o[u] = zero16();
    if (any)
    {
        const int cell0 = it.rg * g.R;
        const float* Qb = a.Q + (long)it.b * a.K * g.M;
        const float* Kb = a.Kt + (long)it.b * a.K * g.N;
        const float* Vb = WITH_O ? a.V + (long)it.b * g.N * a.D : nullptr;
        TTile<KP> kt[CPS];
        std::conditional_t<VDM, TTile<DP>, RTile<DP>> vt[CPS];   // V (D, N) or (N, D), staged [key][dim]
        unsigned long long rest = any;
        auto pop = [&]() {
            if (!rest) return -1;
            const int b = __builtin_ctzll(rest);
            rest &= rest - 1;
            return b;
        };
        auto load = [&](int c0, int c1) {
            const int cc[2] = {c0, c1};
#pragma unroll
            for (int t = 0; t < CPS; ++t)
                if (cc[t] >= 0)
                {
                    kt[t].load(Kb, a.K, g.N, 32 * (cell0 + cc[t]), threadIdx.x);
                    if constexpr (WITH_O && VDM) vt[t].load(Vb, a.D, g.N, 32 * (cell0 + cc[t]), threadIdx.x);
                    if constexpr (WITH_O && !VDM) vt[t].load(Vb, a.D, a.D, g.N, 32 * (cell0 + cc[t]), threadIdx.x);
                }
        };
        auto store = [&](int buf, int c0, int c1) {
            const int cc[2] = {c0, c1};
#pragma unroll
            for (int t = 0; t < CPS; ++t)
                if (cc[t] >= 0)
                {
                    kt[t].store(Ks[buf][t], threadIdx.x);
                    if constexpr (WITH_O) vt[t].store(Vs[buf][t], threadIdx.x);
                }
        };
        int c0 = pop(), c1 = CPS == 2 ? pop() : -1;
        load(c0, c1);
        float qf[KP / 2];
        line_operand<KP>(Qb, a.K, g.M, qi, h, qf);
        const int qc = min(qi, g.M - 1);
        const MRow mrow = mrow_of(a.mask ? a.mask + it.b * a.mask_bs : a.Q, a.mask ? g.M : 0, g.N, qc);
        store(0, c0, c1);
        __syncthreads();
        int buf = 0;
        while (true)
        {
            const int n0 = pop(), n1 = CPS == 2 ? pop() : -1;
            if (n0 >= 0) load(n0, n1);
            const bool act0 = (lw.nz >> c0) & 1ull, act1 = c1 >= 0 && ((lw.nz >> c1) & 1ull);
            if (act0 || act1)
            {
                float x[CPS][16], cmax = kLowest;
                // Every active cell's score chain first: the matrix core works
                // on the second while the first one's scores are processed.
                f32x16 scs[CPS];
#pragma unroll
                for (int t = 0; t < CPS; ++t)
                    if (t ? act1 : act0) scs[t] = score_chain<KP, CPS == 2>(Ks[buf][t], qf, h, c);
#pragma unroll
                for (int t = 0; t < CPS; ++t)
                {
                    const int cell = t ? c1 : c0;
                    if (!(t ? act1 : act0))
                    {
#pragma unroll
                        for (int r = 0; r < 16; ++r) x[t][r] = kNegInf;
                        continue;
                    }
                    const int jbase = 32 * (cell0 + cell);
                    const f32x16& sc = scs[t];
                    const bool gen = (lw.gen >> cell) & 1ull, full = jbase + 32 <= g.N;
                    float cm;
                    if (full && !gen)
                        cm = cell_scores<true, false>(sc, a.alpha, mrow, g.N, jbase, h, x[t]);
                    else if (full)
                        cm = cell_scores<true, true>(sc, a.alpha, mrow, g.N, jbase, h, x[t]);
                    else if (!gen)
                        cm = cell_scores<false, false>(sc, a.alpha, mrow, g.N, jbase, h, x[t]);
                    else
                        cm = cell_scores<false, true>(sc, a.alpha, mrow, g.N, jbase, h, x[t]);
                    cmax = fmax_f(cmax, cm);
                    if (a.S)
                    {
                        // The cell's scores for the key-line pass, in this lane order.
                        float* blk = a.S + (((long)it.b * g.RT + line) * g.CT + (cell0 + cell)) * 1024 + lane;
#pragma unroll
                        for (int r = 0; r < 16; ++r) blk[r * 64] = x[t][r];
                    }
                }
                cmax = fmax_f(cmax, __shfl_xor(cmax, 32));
                const float mnew = fmax_f(mrun, cmax);
                if (__any(mnew != mrun))
                {
                    const float scale = exp_neg(mrun - mnew);
                    lrun *= scale;
                    if constexpr (WITH_O)
                    {
#pragma unroll
                        for (int u = 0; u < DU; ++u) o[u] *= scale;
                    }
                    mrun = mnew;
                }
                // Rows still without an allowed key keep lowest() and only -inf scores.
                const float mb = mrun == kLowest ? 0.0f : mrun * kLog2e;
#pragma unroll
                for (int t = 0; t < CPS; ++t)
                {
                    if (!(t ? act1 : act0)) continue;
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                    {
                        x[t][r] = __builtin_amdgcn_exp2f(__builtin_fmaf(x[t][r], kLog2e, -mb));
                        lrun += x[t][r];
                    }
                    if constexpr (WITH_O) value_chain<DP, CPS == 2>(Vs[buf][t], x[t], h, c, o);
                }
            }
            if (n0 < 0) break;
            store(buf ^ 1, n0, n1);
            __syncthreads();
            buf ^= 1;
            c0 = n0;
            c1 = n1;
        }
    }
    lrun += __shfl_xor(lrun, 32);
    fwd_store<DP, WITH_O>(a, g, lw, it.b, line, it.rg, mrun, lrun, o);
}

// Merges of lines cut into several ranges (the k_flash_*_combine kernels):
// one workgroup per line. Wave w takes rows r = w, w+4, w+8, w+12 of the
// f32x16 lane layout (every u), so each partial is read by all four waves at
// once in 256-byte rows; every element is still merged in range order.
template <int DP, bool WITH_O>
__global__ __launch_bounds__(256) void k_flash_fwd_combine(FlashFwdSet t, FlashGeo g)
{
    constexpr int DU = DP / 32;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, h = lane >> 5, c = lane & 31;
    const long lidx = blockIdx.x;
    const int b = static_cast<int>(lidx / g.RT), line = static_cast<int>(lidx % g.RT);
    const FlashFwdArgs a = row_args(t, g, b);
    const LineWork lw = line_work(g, true, b, line, 0);
    if (lw.nne <= 1) return;
    float m = kLowest, l = 0.0f;
    float o[DU][4];
#pragma unroll
    for (int u = 0; u < DU; ++u)
#pragma unroll
        for (int k = 0; k < 4; ++k) o[u][k] = 0.0f;
    for (unsigned long long rs = lw.ranges; rs; rs &= rs - 1)
    {
        const float* pp = g.part + (lidx * g.NR + __builtin_ctzll(rs)) * g.pw;
        const float mr = pp[c], lr = pp[32 + c];
        float t[DU][4];
        if constexpr (WITH_O)
        {
#pragma unroll
            for (int u = 0; u < DU; ++u)
#pragma unroll
                for (int k = 0; k < 4; ++k) t[u][k] = pp[64 + (u * 16 + wave + 4 * k) * 64 + lane];
        }
        const float mn = fmax_f(m, mr);
        const float sa = exp_neg(m - mn), sb = exp_neg(mr - mn);
        l = l * sa + lr * sb;
        m = mn;
        if constexpr (WITH_O)
        {
#pragma unroll
            for (int u = 0; u < DU; ++u)
#pragma unroll
                for (int k = 0; k < 4; ++k) o[u][k] = o[u][k] * sa + t[u][k] * sb;
        }
    }
    const int qi = line * 32 + c;
    if (qi >= g.M) return;
    const long row = (long)b * g.M + qi;
    if (wave == 0 && h == 0)
    {
        a.m[row] = m;
        a.l[row] = l;
    }
    if constexpr (WITH_O)
    {
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
        for (int k = 0; k < 4; ++k)
        {
            const int d0 = DU * drow(wave + 4 * k, h);
            if (d0 >= a.D) continue;
            if (a.o_dm)
            {
                float* ocol = a.O + (long)b * a.D * g.M + qi;   // O per batch (D, M)
#pragma unroll
                for (int u = 0; u < DU; ++u) ocol[(long)(d0 + u) * g.M] = o[u][k] * inv;
            }
            else if constexpr (DU == 2)
                *reinterpret_cast<float2*>(a.O + row * a.D + d0) = make_float2(o[0][k] * inv, o[1][k] * inv);
            else
                a.O[row * a.D + d0] = o[0][k] * inv;
        }
    }
}

// ── backward over query lines: R and dQ ────────────────────────────────────
template <int KP>
__device__ __forceinline__ void rows_store(const FlashBwdArgs& a, const FlashGeo& g, const LineWork& lw, int b,
                                           int line, int rg, float racc, const f32x16* x, const f32x16* y)
{
    constexpr int DU = KP / 32;
    const int lane = threadIdx.x & 63, h = lane >> 5, c = lane & 31, qi = line * 32 + c;
    if (line >= g.RT) return;
    if (direct_writer(lw, rg))
    {
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
        return;
    }
    if (lw.nne <= 1 || !lw.nz) return;
    float* pp = g.part + (((long)b * g.RT + line) * g.NR + rg) * g.pw;
    if (h == 0) pp[c] = racc;
#pragma unroll
    for (int u = 0; u < DU; ++u)
#pragma unroll
        for (int r = 0; r < 16; ++r)
        {
            pp[32 + (u * 16 + r) * 64 + lane] = x[u][r];
            pp[32 + ((DU + u) * 16 + r) * 64 + lane] = y[u][r];
        }
}

template <int KP>
__device__ __forceinline__ void rows_group(const FlashBwdArgs& a, const FlashGeo& g, int b, int grp, int rg,
                                           float (*Ks)[32][KP + 4], float (*Vs)[32][KP + 4],
                                           unsigned long long* nz_s)
{
    constexpr int DU = KP / 32;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, h = lane >> 5, c = lane & 31;
    const int line = grp * kWaves + wave, qi = line * 32 + c;
    const LineWork lw = line_work(g, true, b, line, rg);
    if (lane == 0) nz_s[wave] = lw.nz;
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
        const int cell0 = rg * g.R;
        const float* Qb = a.Q + (long)b * a.K * g.M;
        const float* Kb = a.Kt + (long)b * a.K * g.N;
        const float* Ob = a.dO + (long)b * a.Kd * g.M;
        const float* Vb = a.Vp + (long)b * a.Kd * g.N;
        TTile<KP> kt, vt;
        int cur = __builtin_ctzll(any);
        unsigned long long rest = any & (any - 1);
        kt.load(Kb, a.K, g.N, 32 * (cell0 + cur), threadIdx.x);
        vt.load(Vb, a.Kd, g.N, 32 * (cell0 + cur), threadIdx.x);
        float qf[KP / 2], of[KP / 2];
        line_operand<KP>(Qb, a.K, g.M, qi, h, qf);
        line_operand<KP>(Ob, a.Kd, g.M, qi, h, of);
        const int qc = min(qi, g.M - 1);
        const long srow = (long)b * g.M + qc;
        const float mi = a.m[srow], li = a.l[srow];
        const float linv = li != 0.0f ? 1.0f / li : 0.0f;
        const float mb = mi == kLowest ? 0.0f : mi * kLog2e;   // a row without allowed keys has only -inf scores
        const MRow mrow = mrow_of(a.mask ? a.mask + b * a.mask_bs : a.Q, a.mask ? g.M : 0, g.N, qc);
        kt.store(Ks[0], threadIdx.x);
        vt.store(Vs[0], threadIdx.x);
        __syncthreads();
        int buf = 0;
        while (true)
        {
            const int nxt = rest ? __builtin_ctzll(rest) : -1;
            if (nxt >= 0)
            {
                kt.load(Kb, a.K, g.N, 32 * (cell0 + nxt), threadIdx.x);
                vt.load(Vb, a.Kd, g.N, 32 * (cell0 + nxt), threadIdx.x);
            }
            if ((lw.nz >> cur) & 1ull)
            {
                const int jbase = 32 * (cell0 + cur);
                const f32x16 s = score_chain<KP>(Ks[buf], qf, h, c);
                const f32x16 pp = score_chain<KP>(Vs[buf], of, h, c);
                float w[16], wp[16];
                const bool gen = (lw.gen >> cur) & 1ull, full = jbase + 32 <= g.N;
                if (full && !gen)
                    cell_scores<true, false>(s, a.alpha, mrow, g.N, jbase, h, w);
                else if (full)
                    cell_scores<true, true>(s, a.alpha, mrow, g.N, jbase, h, w);
                else if (!gen)
                    cell_scores<false, false>(s, a.alpha, mrow, g.N, jbase, h, w);
                else
                    cell_scores<false, true>(s, a.alpha, mrow, g.N, jbase, h, w);
#pragma unroll
                for (int r = 0; r < 16; ++r)
                {
                    w[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(w[r], kLog2e, -mb)) * linv;
                    wp[r] = w[r] * (a.alpha2 * pp[r]);
                    racc += wp[r];
                }
                value_chain2<KP>(Ks[buf], wp, w, h, c, x, y);
            }
            if (nxt < 0) break;
            kt.store(Ks[buf ^ 1], threadIdx.x);
            vt.store(Vs[buf ^ 1], threadIdx.x);
            __syncthreads();
            buf ^= 1;
            cur = nxt;
            rest &= rest - 1;
        }
    }
    racc += __shfl_xor(racc, 32);
    rows_store<KP>(a, g, lw, b, line, rg, racc, x, y);
}

template <int KP>
__global__ __launch_bounds__(64 * kWaves, 2) void k_flash_bwd_rows(FlashBwdSet t, FlashGeo g)
{
    __shared__ __align__(16) float Ks[2][32][KP + 4];   // key tile [key][dim]
    __shared__ __align__(16) float Vs[2][32][KP + 4];   // V' tile [key][dim]
    __shared__ unsigned long long nz_s[kWaves];
    const Item it = item_of(g);
    const FlashBwdArgs a = row_args(t, g, it.b);
    rows_group<KP>(a, g, it.b, it.grp, it.rg, Ks, Vs, nz_s);
}

template <int KP>
__global__ __launch_bounds__(256) void k_flash_bwd_rows_combine(FlashBwdSet t, FlashGeo g)
{
    constexpr int DU = KP / 32;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, h = lane >> 5, c = lane & 31;
    const long lidx = blockIdx.x;
    const int b = static_cast<int>(lidx / g.RT), line = static_cast<int>(lidx % g.RT);
    const FlashBwdArgs a = row_args(t, g, b);
    const LineWork lw = line_work(g, true, b, line, 0);
    if (lw.nne <= 1) return;
    float racc = 0.0f;
    float x[DU][4], y[DU][4];
#pragma unroll
    for (int u = 0; u < DU; ++u)
#pragma unroll
        for (int k = 0; k < 4; ++k) x[u][k] = y[u][k] = 0.0f;
    for (unsigned long long rs = lw.ranges; rs; rs &= rs - 1)
    {
        const float* pp = g.part + (lidx * g.NR + __builtin_ctzll(rs)) * g.pw;
        float tx[DU][4], ty[DU][4];
        const float rr = pp[c];
#pragma unroll
        for (int u = 0; u < DU; ++u)
#pragma unroll
            for (int k = 0; k < 4; ++k)
            {
                tx[u][k] = pp[32 + (u * 16 + wave + 4 * k) * 64 + lane];
                ty[u][k] = pp[32 + ((DU + u) * 16 + wave + 4 * k) * 64 + lane];
            }
        racc += rr;
#pragma unroll
        for (int u = 0; u < DU; ++u)
#pragma unroll
            for (int k = 0; k < 4; ++k)
            {
                x[u][k] += tx[u][k];
                y[u][k] += ty[u][k];
            }
    }
    const int qi = line * 32 + c;
    if (qi >= g.M) return;
    if (wave == 0 && h == 0) a.R[(long)b * g.M + qi] = racc;
    float* dq = a.dQ + (long)b * a.K * g.M + qi;
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int u = 0; u < DU; ++u)
        {
            const int d = DU * drow(wave + 4 * k, h) + u;
            if (d < a.K) dq[(long)d * g.M] = a.alpha * (x[u][k] - racc * y[u][k]);
        }
}

// Loads the query-side tiles of one cell of the key-line kernel into registers:
// Q and dO (transposed), G rows, and m, 1/l, R of the 32 queries (threads 0-95).
template <int KP, bool GDO>
__device__ __forceinline__ void stage_cols(TTile<KP>& qt, TTile<KP>& ot, RTile<KP>& gt, float& st, const float* Qb,
                                           const float* Ob, const float* Gb, const float* mb, const float* lb,
                                           const float* Rb, const FlashBwdArgs& a, int M, int i0)
{
    qt.load(Qb, a.K, M, i0, threadIdx.x);
    ot.load(Ob, a.Kd, M, i0, threadIdx.x);
    if constexpr (!GDO) gt.load(Gb, a.ldg, a.K, M, i0, threadIdx.x);
    if (threadIdx.x < 96)
    {
        const int i = i0 + static_cast<int>(threadIdx.x & 31), which = threadIdx.x >> 5;
        float v = 0.0f;
        if (i < M) v = which == 0 ? mb[i] : which == 1 ? lb[i] : Rb[i];
        // m * log2(e) (0 for a row without allowed keys), 1 / l (0 for l = 0), R.
        st = which == 0 ? (v == kLowest ? 0.0f : v * kLog2e) : which == 1 ? (v != 0.0f ? 1.0f / v : 0.0f) : v;
    }
}

// Scores of one cell of the key-line kernel for this lane's key (16 queries
// drow(r,h)): alpha * dot + mask, -inf outside the (M, N) plane.
template <bool FULL, bool MASKED>
__device__ __forceinline__ void col_scores(const f32x16& s, const FlashBwdArgs& a, const float* mask, int ibase,
                                           int jc, int kj, int h, int M, int N, float* x)
{
    // Mask loads are issued 8 at a time (clamped indices, no branch), then used.
#pragma unroll
    for (int r0 = 0; r0 < 16; r0 += 8)
    {
        float mv[8];
        if constexpr (MASKED)
        {
#pragma unroll
            for (int r = 0; r < 8; ++r) mv[r] = mask[(long)min(ibase + drow(r0 + r, h), M - 1) * N + jc];
        }
#pragma unroll
        for (int r = 0; r < 8; ++r)
        {
            const int i = ibase + drow(r0 + r, h);
            float v = a.alpha * s[r0 + r];
            if constexpr (MASKED) v += mv[r];
            if constexpr (!FULL) v = (i < M && kj < N) ? v : kNegInf;
            x[r0 + r] = v;
        }
    }
}

// ── backward over key lines: dK and dV ─────────────────────────────────────
template <int KP>
__device__ __forceinline__ void cols_store(const FlashBwdArgs& a, const FlashGeo& g, const LineWork& lw, int b,
                                           int line, int rg, const f32x16* dk, const f32x16* dv)
{
    constexpr int DU = KP / 32;
    const int lane = threadIdx.x & 63, h = lane >> 5, c = lane & 31, kj = line * 32 + c;
    if (line >= g.CT) return;
    if (direct_writer(lw, rg))
    {
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
        return;
    }
    if (lw.nne <= 1 || !lw.nz) return;
    float* pp = g.part + (((long)b * g.CT + line) * g.NR + rg) * g.pw;
#pragma unroll
    for (int u = 0; u < DU; ++u)
#pragma unroll
        for (int r = 0; r < 16; ++r)
        {
            pp[(u * 16 + r) * 64 + lane] = dk[u][r];
            pp[((DU + u) * 16 + r) * 64 + lane] = dv[u][r];
        }
}

template <int KP, bool GDO, bool WDS, bool SST>
__device__ __forceinline__ void cols_group(const FlashBwdArgs& a, const FlashGeo& g, int b, int grp, int rg,
                                           float (*Qs)[32][KP + 4], float (*Os)[32][KP + 4],
                                           float (*Gs)[32][KP + 4], float (*St)[3][32], unsigned long long* nz_s)
{
    constexpr int DU = KP / 32;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, h = lane >> 5, c = lane & 31;
    const int line = grp * kWaves + wave, kj = line * 32 + c;
    const LineWork lw = line_work(g, false, b, line, rg);
    if (lane == 0) nz_s[wave] = lw.nz;
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
        const int cell0 = rg * g.R;
        const float* Qb = a.Q + (long)b * a.K * g.M;
        const float* Kb = a.Kt + (long)b * a.K * g.N;
        const float* Ob = a.dO + (long)b * a.Kd * g.M;
        const float* Vb = a.Vp + (long)b * a.Kd * g.N;
        const float* Gb = a.G + (long)b * g.M * a.ldg;
        const float* mb = a.m + (long)b * g.M;
        const float* lb = a.l + (long)b * g.M;
        const float* Rb = a.R + (long)b * g.M;
        TTile<KP> qt, ot;
        RTile<KP> gt;
        float st = 0.0f;
        int cur = __builtin_ctzll(any);
        unsigned long long rest = any & (any - 1);
        stage_cols<KP, GDO>(qt, ot, gt, st, Qb, Ob, Gb, mb, lb, Rb, a, g.M, 32 * (cell0 + cur));
        float kf[SST ? 1 : KP / 2], vf[KP / 2];
        if constexpr (!SST) line_operand<KP>(Kb, a.K, g.N, kj, h, kf);
        line_operand<KP>(Vb, a.Kd, g.N, kj, h, vf);
        // SST: this lane's key c in the forward's score blocks (r 64 + h 32 + q with drow(r, h) = c).
        const float* sl = SST ? a.S + ((long)b * g.RT * g.CT + line) * 1024 + (4 * (c >> 3) + (c & 3)) * 64 +
                                    ((c >> 2) & 1) * 32 + 4 * h
                              : nullptr;
        const int jc = min(kj, g.N - 1);
        const float* mk = a.mask ? a.mask + b * a.mask_bs : nullptr;
        // SST: block (query tile cell0 + x, key tile line), queries drow(r, h), 4 at a time;
        // a cell's block is loaded one cell ahead of its chains.
        auto score_block = [&](int x, float* w) {
            const float* blk = sl + (long)(cell0 + x) * g.CT * 1024;
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4)
            {
                const float4 v = *reinterpret_cast<const float4*>(blk + 8 * g4);
                w[4 * g4 + 0] = v.x;
                w[4 * g4 + 1] = v.y;
                w[4 * g4 + 2] = v.z;
                w[4 * g4 + 3] = v.w;
            }
        };
        float sw[SST ? 16 : 1];
        if constexpr (SST)
            if ((lw.nz >> cur) & 1ull) score_block(cur, sw);
        qt.store(Qs[0], threadIdx.x);
        ot.store(Os[0], threadIdx.x);
        if constexpr (!GDO) gt.store(Gs[0], threadIdx.x);
        if (threadIdx.x < 96) St[0][threadIdx.x >> 5][threadIdx.x & 31] = st;
        __syncthreads();
        int buf = 0;
        while (true)
        {
            const int nxt = rest ? __builtin_ctzll(rest) : -1;
            if (nxt >= 0) stage_cols<KP, GDO>(qt, ot, gt, st, Qb, Ob, Gb, mb, lb, Rb, a, g.M, 32 * (cell0 + nxt));
            float swn[SST ? 16 : 1];
            if constexpr (SST)
                if (nxt >= 0 && ((lw.nz >> nxt) & 1ull)) score_block(nxt, swn);
            if ((lw.nz >> cur) & 1ull)
            {
                const int ibase = 32 * (cell0 + cur);
                float w[16], ds[16];
                const bool gen = (lw.gen >> cur) & 1ull, full = ibase + 32 <= g.M && (line + 1) * 32 <= g.N;
                if constexpr (SST)
                {
#pragma unroll
                    for (int r = 0; r < 16; ++r) w[r] = sw[r];
                    if (!full)
                    {
#pragma unroll
                        for (int r = 0; r < 16; ++r)
                            w[r] = (ibase + drow(r, h) < g.M && kj < g.N) ? w[r] : kNegInf;
                    }
                }
                const f32x16 p = score_chain<KP>(Os[buf], vf, h, c);
                if constexpr (!SST)
                {
                    const f32x16 s = score_chain<KP>(Qs[buf], kf, h, c);
                    if (full && !gen)
                        col_scores<true, false>(s, a, mk, ibase, jc, kj, h, g.M, g.N, w);
                    else if (full)
                        col_scores<true, true>(s, a, mk, ibase, jc, kj, h, g.M, g.N, w);
                    else if (!gen)
                        col_scores<false, false>(s, a, mk, ibase, jc, kj, h, g.M, g.N, w);
                    else
                        col_scores<false, true>(s, a, mk, ibase, jc, kj, h, g.M, g.N, w);
                }
#pragma unroll
                for (int r = 0; r < 16; ++r)
                {
                    const int ii = drow(r, h);
                    w[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(w[r], kLog2e, -St[buf][0][ii])) * St[buf][1][ii];
                    ds[r] = w[r] * (a.alpha2 * p[r] - St[buf][2][ii]);
                }

                if constexpr (GDO)
                    value_chain<KP>(Os[buf], w, h, c, dv);
                else
                    value_chain<KP>(Gs[buf], w, h, c, dv);
                value_chain<KP>(Qs[buf], ds, h, c, dk);
                if constexpr (WDS)
                {
                    // dS of the cell, for the query-line pass (row i, key kj).
                    float* dsb = a.dS + (long)b * g.M * g.N + kj;
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                    {
                        const int i = ibase + drow(r, h);
                        if (i < g.M && kj < g.N) dsb[(long)i * g.N] = ds[r];
                    }
                }
            }
            if (nxt < 0) break;
            if constexpr (SST)
            {
#pragma unroll
                for (int r = 0; r < 16; ++r) sw[r] = swn[r];
            }
            qt.store(Qs[buf ^ 1], threadIdx.x);
            ot.store(Os[buf ^ 1], threadIdx.x);
            if constexpr (!GDO) gt.store(Gs[buf ^ 1], threadIdx.x);
            if (threadIdx.x < 96) St[buf ^ 1][threadIdx.x >> 5][threadIdx.x & 31] = st;
            __syncthreads();
            buf ^= 1;
            cur = nxt;
            rest &= rest - 1;
        }
    }
    cols_store<KP>(a, g, lw, b, line, rg, dk, dv);
}

template <int KP, bool GDO, bool WDS, bool SST = false>
__global__ __launch_bounds__(64 * kWaves, 2) void k_flash_bwd_cols(FlashBwdSet t, FlashGeo g)
{
    __shared__ __align__(16) float Qs[2][32][KP + 4];   // query tile [query][dim]
    __shared__ __align__(16) float Os[2][32][KP + 4];   // dO tile [query][dim]
    __shared__ __align__(16) float Gs[GDO ? 1 : 2][32][KP + 4];   // G tile [query][dim] (GDO: the dO tile)
    __shared__ float St[2][3][32];                      // m, 1/l, R of the tile's queries
    __shared__ unsigned long long nz_s[kWaves];
    const Item it = item_of(g);
    const FlashBwdArgs a = row_args(t, g, it.b);
    cols_group<KP, GDO, WDS, SST>(a, g, it.b, it.grp, it.rg, Qs, Os, Gs, St, nz_s);
}

template <int KP>
__global__ __launch_bounds__(256) void k_flash_bwd_cols_combine(FlashBwdSet t, FlashGeo g)
{
    constexpr int DU = KP / 32;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, h = lane >> 5, c = lane & 31;
    const long lidx = blockIdx.x;
    const int b = static_cast<int>(lidx / g.CT), line = static_cast<int>(lidx % g.CT);
    const FlashBwdArgs a = row_args(t, g, b);
    const LineWork lw = line_work(g, false, b, line, 0);
    if (lw.nne <= 1) return;
    float dk[DU][4], dv[DU][4];
#pragma unroll
    for (int u = 0; u < DU; ++u)
#pragma unroll
        for (int k = 0; k < 4; ++k) dk[u][k] = dv[u][k] = 0.0f;
    for (unsigned long long rs = lw.ranges; rs; rs &= rs - 1)
    {
        const float* pp = g.part + (lidx * g.NR + __builtin_ctzll(rs)) * g.pw;
        float tk[DU][4], tv[DU][4];
#pragma unroll
        for (int u = 0; u < DU; ++u)
#pragma unroll
            for (int k = 0; k < 4; ++k)
            {
                tk[u][k] = pp[(u * 16 + wave + 4 * k) * 64 + lane];
                tv[u][k] = pp[((DU + u) * 16 + wave + 4 * k) * 64 + lane];
            }
#pragma unroll
        for (int u = 0; u < DU; ++u)
#pragma unroll
            for (int k = 0; k < 4; ++k)
            {
                dk[u][k] += tk[u][k];
                dv[u][k] += tv[u][k];
            }
    }
    const int kj = line * 32 + c;
    if (kj >= g.N) return;
    float* dkb = a.dK + (long)b * a.K * g.N + kj;
    float* dvb = a.dV + (long)b * a.K * g.N + kj;
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int u = 0; u < DU; ++u)
        {
            const int d = DU * drow(wave + 4 * k, h) + u;
            if (d < a.K)
            {
                dkb[(long)d * g.N] = a.alpha * dk[u][k];
                dvb[(long)d * g.N] = dv[u][k];
            }
        }
}

// dQ of one query line from the dq pass, dQ = alpha x: written directly, or
// x as the range's partial (pw = 32 KP floats) for k_flash_bwd_dq_combine.
template <int KP>
__device__ __forceinline__ void dq_store(const FlashBwdArgs& a, const FlashGeo& g, const LineWork& lw, int b,
                                         int line, int rg, const f32x16* x)
{
    constexpr int DU = KP / 32;
    const int lane = threadIdx.x & 63, h = lane >> 5, c = lane & 31, qi = line * 32 + c;
    if (line >= g.RT) return;
    if (direct_writer(lw, rg))
    {
        if (qi >= g.M) return;
        float* dq = a.dQ + (long)b * a.K * g.M + qi;
#pragma unroll
        for (int u = 0; u < DU; ++u)
#pragma unroll
            for (int r = 0; r < 16; ++r)
            {
                const int d = DU * drow(r, h) + u;
                if (d < a.K) dq[(long)d * g.M] = a.alpha * x[u][r];
            }
        return;
    }
    if (lw.nne <= 1 || !lw.nz) return;
    float* pp = g.part + (((long)b * g.RT + line) * g.NR + rg) * g.pw;
#pragma unroll
    for (int u = 0; u < DU; ++u)
#pragma unroll
        for (int r = 0; r < 16; ++r) pp[(u * 16 + r) * 64 + lane] = x[u][r];
}

template <int KP>
__global__ __launch_bounds__(256) void k_flash_bwd_dq_combine(FlashBwdSet t, FlashGeo g)
{
    constexpr int DU = KP / 32;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, h = lane >> 5, c = lane & 31;
    const long lidx = blockIdx.x;
    const int b = static_cast<int>(lidx / g.RT), line = static_cast<int>(lidx % g.RT);
    const FlashBwdArgs a = row_args(t, g, b);
    const LineWork lw = line_work(g, true, b, line, 0);
    if (lw.nne <= 1) return;
    float x[DU][4];
#pragma unroll
    for (int u = 0; u < DU; ++u)
#pragma unroll
        for (int k = 0; k < 4; ++k) x[u][k] = 0.0f;
    for (unsigned long long rs = lw.ranges; rs; rs &= rs - 1)
    {
        const float* pp = g.part + (lidx * g.NR + __builtin_ctzll(rs)) * g.pw;
        float t[DU][4];
#pragma unroll
        for (int u = 0; u < DU; ++u)
#pragma unroll
            for (int k = 0; k < 4; ++k) t[u][k] = pp[(u * 16 + wave + 4 * k) * 64 + lane];
#pragma unroll
        for (int u = 0; u < DU; ++u)
#pragma unroll
            for (int k = 0; k < 4; ++k) x[u][k] += t[u][k];
    }
    const int qi = line * 32 + c;
    if (qi >= g.M) return;
    float* dq = a.dQ + (long)b * a.K * g.M + qi;
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int u = 0; u < DU; ++u)
        {
            const int d = DU * drow(wave + 4 * k, h) + u;
            if (d < a.K) dq[(long)d * g.M] = a.alpha * x[u][k];
        }
}

// dQ from the stored dS: dQ_i = alpha sum_j dS_ij k_j over the non-empty cells
// of the line's range, with the rows kernel's lines and ranges.
template <int KP>
__global__ __launch_bounds__(64 * kWaves, 3) void k_flash_bwd_dq(FlashBwdSet t, FlashGeo g)
{
    constexpr int DU = KP / 32;
    __shared__ __align__(16) float Ks[2][32][KP + 4];   // key tile [key][dim]
    __shared__ unsigned long long nz_s[kWaves];
    const Item it = item_of(g);
    const FlashBwdArgs a = row_args(t, g, it.b);
    const int b = it.b, rg = it.rg;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, h = lane >> 5, c = lane & 31;
    const int line = it.grp * kWaves + wave, qi = line * 32 + c;
    const LineWork lw = line_work(g, true, b, line, rg);
    if (lane == 0) nz_s[wave] = lw.nz;
    __syncthreads();
    const unsigned long long any = nz_s[0] | nz_s[1] | nz_s[2] | nz_s[3];
    f32x16 x[DU];
#pragma unroll
    for (int u = 0; u < DU; ++u) x[u] = zero16();
    if (any)
    {
        const int cell0 = rg * g.R;
        const float* Kb = a.Kt + (long)b * a.K * g.N;
        const MRow dsrow = mrow_of(a.dS + (long)b * g.M * g.N, g.M, g.N, min(qi, g.M - 1));
        TTile<KP> kt;
        int cur = __builtin_ctzll(any);
        unsigned long long rest = any & (any - 1);
        kt.load(Kb, a.K, g.N, 32 * (cell0 + cur), threadIdx.x);
        // This line's dS of a cell is loaded one cell ahead of its chain.
        float w[16];
        if ((lw.nz >> cur) & 1ull) mask_row16(dsrow, g.N, 32 * (cell0 + cur), h, w);
        kt.store(Ks[0], threadIdx.x);
        __syncthreads();
        int buf = 0;
        while (true)
        {
            const int nxt = rest ? __builtin_ctzll(rest) : -1;
            float wn[16];
            if (nxt >= 0)
            {
                kt.load(Kb, a.K, g.N, 32 * (cell0 + nxt), threadIdx.x);
                if ((lw.nz >> nxt) & 1ull) mask_row16(dsrow, g.N, 32 * (cell0 + nxt), h, wn);
            }
            if ((lw.nz >> cur) & 1ull) value_chain<KP>(Ks[buf], w, h, c, x);
            if (nxt < 0) break;
#pragma unroll
            for (int r = 0; r < 16; ++r) w[r] = wn[r];
            kt.store(Ks[buf ^ 1], threadIdx.x);
            __syncthreads();
            buf ^= 1;
            cur = nxt;
            rest &= rest - 1;
        }
    }
    dq_store<KP>(a, g, lw, b, line, rg, x);
}

// Work order of a flash launch (one workgroup of 1024 threads). The weight of
// an item (batch entry, line group, range) is the number of cells of its range
// that at least one of its 4 lines has to visit (mask cell class != 0); the
// kernel time is set by the most loaded CU, so items are sorted heaviest first
// (counting sort, weights 0..R) and sorted position p is given to workgroup
//   p < resident:  ncu r + (r even ? q : n_r - 1 - q),  r = p / ncu, q = p % ncu
//   p >= resident: p
// (n_r: items in round r, ncu unless it is the last, partial round)
// (ncu = CUs; resident = workgroups per CU x ncu). Workgroups are dispatched
// round-robin over the CUs, so round r of resident workgroups runs together and
// the serpentine gives every CU one heavy and one light item per pair of
// rounds; later workgroups backfill CUs as they free up, heaviest first. Items
// of equal weight may be placed in any order (only the timing depends on it).
constexpr int kOrderThreads = 1024;
// Cell tables of the rows of a launch (pre-offset like FlashSet::cls).
struct FlashCls
{
    const unsigned char* cls[kFlashMaxRows];
    int hpr;
};
__global__ __launch_bounds__(kOrderThreads) void k_flash_order(FlashGeo g, FlashCls tab, int rows, int nitems,
                                                               int ncu, int resident, int* __restrict__ order,
                                                               unsigned char* __restrict__ weight)
{
    __shared__ int count[65], cursor[65];
    const int t = threadIdx.x, lines = rows ? g.RT : g.CT, cells = rows ? g.CT : g.RT, per = g.G * g.NR;
    if (t < 65) count[t] = 0;
    __syncthreads();
    for (int it = t; it < nitems; it += kOrderThreads)
    {
        const int b = it / per, rem = it % per, grp = g.G - 1 - rem / g.NR, rg = rem % g.NR;
        const unsigned char* cls = tab.cls[b / tab.hpr] + (long)b * g.cls_bs;
        const int x0 = rg * g.R, x1 = min(x0 + g.R, cells), l0 = grp * kWaves;
        int w = 0;
        if ((g.CT & 3) == 0)
        {
            // 32-bit reads (the table and every row start at multiples of 4 bytes): rows: 4 cells of
            // one line per word, OR over the 4 lines; columns: the 4 lines of one cell per word.
            if (rows)
            {
                for (int x = x0; x < x1; x += 4)
                {
                    unsigned u = 0;
#pragma unroll
                    for (int k = 0; k < kWaves; ++k)
                        if (l0 + k < lines) u |= *reinterpret_cast<const unsigned*>(cls + (long)(l0 + k) * g.CT + x);
                    w += ((u & 0xffu) != 0) + ((u & 0xff00u) != 0) + ((u & 0xff0000u) != 0) + ((u >> 24) != 0);
                }
            }
            else
            {
                const int valid = min(kWaves, lines - l0);
                const unsigned keep = valid >= 4 ? ~0u : (1u << (8 * valid)) - 1u;
                for (int x = x0; x < x1; ++x)
                    w += (*reinterpret_cast<const unsigned*>(cls + (long)x * g.CT + l0) & keep) != 0;
            }
        }
        else
        {
            for (int x = x0; x < x1; ++x)
            {
                bool any = false;
                for (int k = 0; k < kWaves; ++k)
                {
                    const int line = l0 + k;
                    if (line < lines)
                        any = any || (rows ? cls[(long)line * g.CT + x] : cls[(long)x * g.CT + line]) != 0;
                }
                w += any ? 1 : 0;
            }
        }
        weight[it] = static_cast<unsigned char>(w);
        atomicAdd(&count[w], 1);
    }
    __syncthreads();
    if (t == 0)
    {
        int acc = 0;
        for (int w = 64; w >= 0; --w)
        {
            cursor[w] = acc;
            acc += count[w];
        }
    }
    __syncthreads();
    for (int it = t; it < nitems; it += kOrderThreads)
    {
        const int p = atomicAdd(&cursor[weight[it]], 1);
        int bid = p;
        if (p < resident)
        {
            // a last, partial round is reversed within its own n items: bid stays below nitems
            const int r = p / ncu, q = p % ncu, n = min(ncu, nitems - r * ncu);
            bid = r * ncu + ((r & 1) ? n - 1 - q : q);
        }
        order[bid] = it;
    }
}

// R_i = alpha2 sum_d dO(d, i) O(d, i): dO per batch (Kd, M) dim-major; O the
// same, or (M, Kd) query-major when o_qm. A workgroup takes 64 rows (one per
// lane); wave w sums dims [w q, (w+1) q), q = Kd / 4 <= 16, in two chains
// (even and odd dims), and wave 0 adds the four partials in wave order.
// Query-major O rows are contiguous: the workgroup's 64 Kd floats are staged
// through LDS. Loops run a fixed 16 steps over clamped addresses, so every
// load is in flight at once. blockIdx.y: the row of a multi-row launch (its
// own dO, O and R, `total` entries each).
struct RowdotSet
{
    const float* dO[kFlashMaxRows];
    const float* O[kFlashMaxRows];
    float* R[kFlashMaxRows];
};
__global__ __launch_bounds__(256) void k_flash_rowdot(RowdotSet set, int M, int Kd, long total, float alpha2, int o_qm)
{
    __shared__ float part[4][64];
    __shared__ float Ot[64][65];
    const float* __restrict__ dO = set.dO[blockIdx.y];
    const float* __restrict__ O = set.O[blockIdx.y];
    float* __restrict__ R = set.R[blockIdx.y];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const long t0 = (long)blockIdx.x * 64, t = t0 + lane;
    const int q = Kd / 4, d0 = wave * q;
    if (o_qm)
    {
        // 64 rows x Kd floats, Kd / 4 per thread; past the last row reads 0.
        const long n = min(64L, total - t0) * Kd;
        const Rsrc rs = rsrc(O + t0 * Kd, n);
        float v[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) v[k] = bload(rs, 4u * static_cast<unsigned>(threadIdx.x + 256 * k));
#pragma unroll
        for (int k = 0; k < 16; ++k)
            if (k < q)
            {
                const unsigned e = threadIdx.x + 256u * k;
                Ot[e / static_cast<unsigned>(Kd)][e % static_cast<unsigned>(Kd)] = v[k];
            }
        __syncthreads();
    }
    float acc[2] = {0.0f, 0.0f};
    if (t < total)
    {
        const long b = t / M, i = t % M;
        const float* p = dO + (b * Kd + d0) * M + i;
        const float* od = O + (b * Kd + d0) * M + i;
        float pv[16], ov[16];
#pragma unroll
        for (int k = 0; k < 16; ++k)
        {
            const int kc = min(k, q - 1);
            pv[k] = p[(long)kc * M];
            ov[k] = o_qm ? Ot[lane][d0 + kc] : od[(long)kc * M];
        }
#pragma unroll
        for (int k = 0; k < 16; ++k)
            if (k < q) acc[k & 1] = __builtin_fmaf(pv[k], ov[k], acc[k & 1]);
    }
    part[wave][lane] = acc[0] + acc[1];
    __syncthreads();
    if (wave == 0 && t < total) R[t] = alpha2 * (((part[0][lane] + part[1][lane]) + part[2][lane]) + part[3][lane]);
}

// Mask cell classes: 0 all -inf, 1 all zero, 2 general. blockIdx.z: which mask.
__global__ __launch_bounds__(256) void k_flash_classify(const float* __restrict__ mask, long mask_bs, int M, int N,
                                                        int CT, unsigned char* __restrict__ cls)
{
    const int jb = blockIdx.x, ib = blockIdx.y;
    mask += blockIdx.z * mask_bs;
    cls += (long)blockIdx.z * gridDim.y * CT;
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

// Ranges per line: R cells each, R a power of two in [8, 64] and at most 64
// ranges per line. One range when there are enough workgroups to fill the GPU
// twice over, else lines are cut until there are about four times as many
// workgroups as CUs.
void ranges(size_t items, int cells, int& R, int& NR)
{
    R = 64;
    if (items < 512)
    {
        const size_t want = (1024 + items - 1) / items;
        while (R > 8 && static_cast<size_t>((cells + R - 1) / R) < want) R /= 2;
    }
    NR = (cells + R - 1) / R;
}

// Geometry of a row kernel (lines = query tiles) or a column kernel (lines = key tiles);
// per_batch_cls: every batch entry has its own cell table.
FlashGeo geo(size_t batch, size_t M, size_t N, bool rows, int pw, const unsigned char* cls, void* ws,
             bool per_batch_cls = false)
{
    FlashGeo g{};
    g.M = static_cast<int>(M);
    g.N = static_cast<int>(N);
    g.RT = static_cast<int>((M + 31) / 32);
    g.CT = static_cast<int>((N + 31) / 32);
    const int lines = rows ? g.RT : g.CT, cells = rows ? g.CT : g.RT;
    g.G = (lines + kWaves - 1) / kWaves;
    ranges(batch * g.G, cells, g.R, g.NR);
    g.pw = pw;
    g.cls = cls;
    g.cls_bs = per_batch_cls ? static_cast<long>(g.RT) * g.CT : 0;
    g.part = static_cast<float*>(ws);
    g.order = nullptr;
    return g;
}

size_t part_bytes(const FlashGeo& g, size_t batch, bool rows)
{
    if (g.NR == 1) return 0;
    return align256(batch * static_cast<size_t>(rows ? g.RT : g.CT) * g.NR * g.pw * sizeof(float));
}

unsigned grid_of(const FlashGeo& g, size_t batch)
{
    return static_cast<unsigned>(batch * static_cast<size_t>(g.G) * g.NR);
}

// One order table: the workgroup -> item map, then the item weights.
size_t order_table_bytes(const FlashGeo& g, size_t batch)
{
    const size_t n = grid_of(g, batch);
    return align256(n * sizeof(int)) + align256(n);
}

// Pointer p moved back by `elems` elements (null stays null): row r of a
// multi-row launch passes its arrays shifted by r * hpr batch entries, so the
// kernels' launch-wide entry index b addresses them.
template <class T>
T* shifted(T* p, size_t elems)
{
    return p ? reinterpret_cast<T*>(reinterpret_cast<std::uintptr_t>(p) - elems * sizeof(T)) : nullptr;
}

size_t blocks_per_entry(size_t M, size_t N) { return ((M + 31) / 32) * ((N + 31) / 32) * 1024; }

// The rows' cell tables (null rows: no mask), shifted by their first entries.
FlashCls cls_table(const unsigned char* const* cells, int rows, size_t hpr, long cls_bs)
{
    FlashCls t{};
    t.hpr = static_cast<int>(hpr);
    for (int r = 0; r < rows; ++r) t.cls[r] = shifted(cells[r], static_cast<size_t>(r) * hpr * cls_bs);
    return t;
}

FlashFwdSet fwd_set(const FlashFwdArgs* a, const unsigned char* const* cells, int rows, size_t hpr, long cls_bs)
{
    FlashFwdSet t{};
    t.hpr = static_cast<int>(hpr);
    t.rows = rows;
    for (int r = 0; r < rows; ++r)
    {
        FlashFwdArgs x = a[r];
        const size_t b0 = static_cast<size_t>(r) * hpr, M = x.M, N = x.N, K = x.K, D = x.D;
        x.Q = shifted(x.Q, b0 * K * M);
        x.Kt = shifted(x.Kt, b0 * K * N);
        x.V = shifted(x.V, b0 * N * D);
        x.mask = shifted(x.mask, b0 * static_cast<size_t>(x.mask_bs));
        x.m = shifted(x.m, b0 * M);
        x.l = shifted(x.l, b0 * M);
        x.O = shifted(x.O, b0 * M * D);
        x.S = shifted(x.S, b0 * blocks_per_entry(M, N));
        t.a[r] = x;
        t.cls[r] = x.mask ? shifted(cells[r], b0 * cls_bs) : nullptr;
    }
    return t;
}

FlashBwdSet bwd_set(const FlashBwdArgs* a, const unsigned char* const* cells, int rows, size_t hpr, long cls_bs)
{
    FlashBwdSet t{};
    t.hpr = static_cast<int>(hpr);
    t.rows = rows;
    for (int r = 0; r < rows; ++r)
    {
        FlashBwdArgs x = a[r];
        const size_t b0 = static_cast<size_t>(r) * hpr, M = x.M, N = x.N, K = x.K, Kd = x.Kd;
        x.Q = shifted(x.Q, b0 * K * M);
        x.Kt = shifted(x.Kt, b0 * K * N);
        x.dO = shifted(x.dO, b0 * Kd * M);
        x.Vp = shifted(x.Vp, b0 * Kd * N);
        x.G = shifted(x.G, b0 * M * static_cast<size_t>(x.ldg));
        x.mask = shifted(x.mask, b0 * static_cast<size_t>(x.mask_bs));
        x.m = shifted(x.m, b0 * M);
        x.l = shifted(x.l, b0 * M);
        x.R = shifted(x.R, b0 * M);
        x.dQ = shifted(x.dQ, b0 * K * M);
        x.dK = shifted(x.dK, b0 * K * N);
        x.dV = shifted(x.dV, b0 * K * N);
        x.dS = shifted(x.dS, b0 * M * N);
        x.S = shifted(x.S, b0 * blocks_per_entry(M, N));
        t.a[r] = x;
        t.cls[r] = x.mask ? shifted(cells[r], b0 * cls_bs) : nullptr;
    }
    return t;
}

// Rows of one launch agree on every shape and layout the kernels take from row 0.
bool same_launch(const FlashFwdArgs& x, const FlashFwdArgs& y)
{
    return x.M == y.M && x.N == y.N && x.K == y.K && x.D == y.D && !x.mask == !y.mask && x.mask_bs == y.mask_bs &&
           x.v_dm == y.v_dm && x.o_dm == y.o_dm && !x.O == !y.O && !x.V == !y.V && !x.S == !y.S;
}
bool same_launch(const FlashBwdArgs& x, const FlashBwdArgs& y)
{
    return x.M == y.M && x.N == y.N && x.K == y.K && x.Kd == y.Kd && x.ldg == y.ldg && !x.mask == !y.mask &&
           x.mask_bs == y.mask_bs && x.g_do == y.g_do && !x.G == !y.G && !x.S == !y.S && !x.R == !y.R;
}

// Builds g's order table at `at` (order_table_bytes(g, batch) bytes); `resident`:
// workgroups of the kernel per CU.
int build_order(const FlashGeo& g, const FlashCls& tab, size_t batch, bool rows, int resident, char* at,
                hipStream_t s)
{
    const size_t n = grid_of(g, batch);
    if (n == 0) return 0;
    int* order = reinterpret_cast<int*>(at);
    unsigned char* weight = reinterpret_cast<unsigned char*>(at + align256(n * sizeof(int)));
    const int ncu = device_cus();
    hipLaunchKernelGGL(k_flash_order, dim3(1), dim3(kOrderThreads), 0, s, g, tab, rows ? 1 : 0, static_cast<int>(n),
                       ncu, resident * ncu, order, weight);
    return launch_status();
}

int fwd_pw(int DP) { return 64 + 32 * DP; }
int rows_pw(int KP) { return 32 + 64 * KP; }
int cols_pw(int KP) { return 64 * KP; }
int dq_pw(int KP) { return 32 * KP; }

template <int KP, int DP, bool WITH_O>
int launch_fwd(const FlashFwdSet& t, const FlashGeo& g0, size_t batch, const int* order, hipStream_t s)
{
    // Cells per step: one cell (3 workgroups per CU: 35 KB of LDS, <= 168
    // VGPRs) when a line range holds >= 32 cells, two (2 per CU) for shorter
    // ranges, where fewer barriers per cell pay more. Measured: causal
    // (96 x 1024)^2 58 -> 71 TFLOP/s with one; causal (128 x 512)^2 and the
    // document-masked rows 3-4 % faster with two.
    const dim3 grid(grid_of(g0, batch)), block(64 * kWaves);
    const bool one = std::min(g0.R, g0.CT) >= 32;
    FlashGeo g = g0;
    g.order = order;
    if (WITH_O && t.a[0].v_dm)
    {
        if (one) hipLaunchKernelGGL((k_flash_fwd<KP, DP, WITH_O, true, 1>), grid, block, 0, s, t, g);
        else hipLaunchKernelGGL((k_flash_fwd<KP, DP, WITH_O, true, 2>), grid, block, 0, s, t, g);
    }
    else
    {
        if (one) hipLaunchKernelGGL((k_flash_fwd<KP, DP, WITH_O, false, 1>), grid, block, 0, s, t, g);
        else hipLaunchKernelGGL((k_flash_fwd<KP, DP, WITH_O, false, 2>), grid, block, 0, s, t, g);
    }
    if (int rc = launch_status()) return rc;
    if (g.NR == 1) return 0;
    hipLaunchKernelGGL((k_flash_fwd_combine<DP, WITH_O>), dim3(static_cast<unsigned>(batch * g.RT)), dim3(256), 0, s,
                       t, g);
    return launch_status();
}

template <int KP>
int launch_bwd(const FlashBwdSet& t, const FlashGeo& gr0, const FlashGeo& gc0, size_t batch,
               const int* order_rows, const int* order_cols, hipStream_t s)
{
    FlashGeo gr = gr0, gc = gc0;
    gr.order = order_rows;
    gc.order = order_cols;
    hipLaunchKernelGGL((k_flash_bwd_rows<KP>), dim3(grid_of(gr, batch)), dim3(64 * kWaves), 0, s, t, gr);
    if (int rc = launch_status()) return rc;
    if (gr.NR > 1)
    {
        hipLaunchKernelGGL((k_flash_bwd_rows_combine<KP>), dim3(static_cast<unsigned>(batch * gr.RT)), dim3(256), 0,
                           s, t, gr);
        if (int rc = launch_status()) return rc;
    }
    if (t.a[0].g_do)
        hipLaunchKernelGGL((k_flash_bwd_cols<KP, true, false>), dim3(grid_of(gc, batch)), dim3(64 * kWaves), 0, s, t,
                           gc);
    else
        hipLaunchKernelGGL((k_flash_bwd_cols<KP, false, false>), dim3(grid_of(gc, batch)), dim3(64 * kWaves), 0, s, t,
                           gc);
    if (int rc = launch_status()) return rc;
    if (gc.NR == 1) return 0;
    hipLaunchKernelGGL((k_flash_bwd_cols_combine<KP>), dim3(static_cast<unsigned>(batch * gc.CT)), dim3(256), 0, s, t,
                       gc);
    return launch_status();
}

} // namespace

bool flash_supported(size_t batch, size_t M, size_t N, size_t K, size_t D)
{
    // Head dims up to 64 and value widths up to 64 in multiples of 4 (16-byte
    // value rows); sizes that fit int; at most 2^30 cells over all batches.
    // Lines of at most 64 ranges of 64 cells: M, N <= 131072.
    // One batch entry's (M, N) mask or score gradients below 2 GiB (32-bit
    // buffer offsets).
    return batch >= 1 && M >= 1 && N >= 1 && K >= 1 && K <= 64 && D >= 1 && D <= 64 && D % 4 == 0 &&
           M <= (size_t{1} << 17) && N <= (size_t{1} << 17) && batch <= (size_t{1} << 20) &&
           M * N < (size_t{1} << 29) &&
           batch * ((M + 31) / 32) * ((N + 31) / 32) <= (size_t{1} << 30);
}

size_t flash_cells_bytes(size_t M, size_t N) { return ((M + 31) / 32) * ((N + 31) / 32); }

int flash_classify(const float* mask, size_t masks, long mask_bs, size_t M, size_t N, void* cells, hipStream_t s)
{
    const unsigned RT = static_cast<unsigned>((M + 31) / 32), CT = static_cast<unsigned>((N + 31) / 32);
    hipLaunchKernelGGL(k_flash_classify, dim3(CT, RT, static_cast<unsigned>(masks)), dim3(256), 0, s, mask, mask_bs,
                       static_cast<int>(M), static_cast<int>(N), static_cast<int>(CT),
                       static_cast<unsigned char*>(cells));
    return launch_status();
}

size_t flash_workspace_bytes(size_t batch, size_t M, size_t N, size_t K, size_t D, bool backward)
{
    if (!backward) return part_bytes(geo(batch, M, N, true, fwd_pw(pad32(D)), nullptr, nullptr), batch, true);
    const int KP = pad32(K);
    return std::max(part_bytes(geo(batch, M, N, true, rows_pw(KP), nullptr, nullptr), batch, true),
                    part_bytes(geo(batch, M, N, false, cols_pw(KP), nullptr, nullptr), batch, false));
}

// Order tables (k_flash_order) for a call with a mask cell table: kind 0 the
// forward (one table), 1 the backward (query lines, then key lines), 2 the
// backward from the forward output (key lines, then the dQ pass). They depend
// on the cell table and (batch, M, N) only.
size_t flash_order_bytes(size_t batch, size_t M, size_t N, int kind)
{
    const FlashGeo gr = geo(batch, M, N, true, 0, nullptr, nullptr);
    if (kind == 0) return order_table_bytes(gr, batch);
    const FlashGeo gc = geo(batch, M, N, false, 0, nullptr, nullptr);
    return order_table_bytes(gr, batch) + order_table_bytes(gc, batch);
}

int flash_build_rows_order(const unsigned char* const* cells, int rows, size_t hpr, size_t M, size_t N,
                           bool per_batch_cls, int kind, void* out, hipStream_t s)
{
    if (rows < 1 || rows > kFlashMaxRows || hpr == 0) return -1;
    for (int r = 0; r < rows; ++r)
        if (!cells[r]) return -1;
    const size_t batch = static_cast<size_t>(rows) * hpr;
    char* at = static_cast<char*>(out);
    const FlashGeo gr = geo(batch, M, N, true, 0, cells[0], nullptr, per_batch_cls);
    const FlashGeo gc = geo(batch, M, N, false, 0, cells[0], nullptr, per_batch_cls);
    const FlashCls tab = cls_table(cells, rows, hpr, gr.cls_bs);
    if (kind == 0) return build_order(gr, tab, batch, true, std::min(gr.R, gr.CT) >= 32 ? 3 : 2, at, s);
    if (kind == 1)
    {
        if (int rc = build_order(gr, tab, batch, true, 2, at, s)) return rc;
        return build_order(gc, tab, batch, false, 2, at + order_table_bytes(gr, batch), s);
    }
    if (int rc = build_order(gc, tab, batch, false, 2, at, s)) return rc;
    return build_order(gr, tab, batch, true, 3, at + order_table_bytes(gc, batch), s);
}

int flash_build_order(const unsigned char* cells, size_t batch, size_t M, size_t N, bool per_batch_cls, int kind,
                      void* out, hipStream_t s)
{
    return flash_build_rows_order(&cells, 1, batch, M, N, per_batch_cls, kind, out, s);
}

int flash_forward_rows(const FlashFwdArgs* a, const unsigned char* const* cells, int rows, size_t hpr, void* ws,
                       const int* order, hipStream_t s)
{
    if (rows < 1 || rows > kFlashMaxRows || hpr == 0) return -1;
    const FlashFwdArgs& a0 = a[0];
    for (int r = 0; r < rows; ++r)
        if (!same_launch(a0, a[r]) || (a[r].mask && !cells[r])) return -1;
    const size_t batch = static_cast<size_t>(rows) * hpr;
    const int KP = pad32(static_cast<size_t>(a0.K)), DP = a0.O ? pad32(static_cast<size_t>(a0.D)) : 32;
    const FlashGeo g = geo(batch, static_cast<size_t>(a0.M), static_cast<size_t>(a0.N), true, fwd_pw(DP),
                           a0.mask ? cells[0] : nullptr, ws, a0.mask && a0.mask_bs != 0);
    if (g.NR > 1 && !ws) return -1;
    const FlashFwdSet t = fwd_set(a, cells, rows, hpr, g.cls_bs);
    const int* ow = a0.mask ? order : nullptr;
    if (!a0.O)
        return KP == 32 ? launch_fwd<32, 32, false>(t, g, batch, ow, s) : launch_fwd<64, 32, false>(t, g, batch, ow, s);
    if (KP == 32)
        return DP == 32 ? launch_fwd<32, 32, true>(t, g, batch, ow, s) : launch_fwd<32, 64, true>(t, g, batch, ow, s);
    return DP == 32 ? launch_fwd<64, 32, true>(t, g, batch, ow, s) : launch_fwd<64, 64, true>(t, g, batch, ow, s);
}

int flash_forward(const FlashFwdArgs& a, const unsigned char* cells, size_t batch, void* ws, const int* order,
                  hipStream_t s)
{
    return flash_forward_rows(&a, &cells, 1, batch, ws, order, s);
}

int flash_backward(const FlashBwdArgs& a, const unsigned char* cells, size_t batch, void* ws, const int* order,
                   hipStream_t s)
{
    const int KP = pad32(static_cast<size_t>(std::max(a.K, a.Kd)));
    const unsigned char* cl = a.mask ? cells : nullptr;
    const bool pb = a.mask && a.mask_bs != 0;
    const FlashGeo gr =
        geo(batch, static_cast<size_t>(a.M), static_cast<size_t>(a.N), true, rows_pw(KP), cl, ws, pb);
    const FlashGeo gc =
        geo(batch, static_cast<size_t>(a.M), static_cast<size_t>(a.N), false, cols_pw(KP), cl, ws, pb);
    if ((gr.NR > 1 || gc.NR > 1) && !ws) return -1;
    const int* orr = a.mask ? order : nullptr;
    const int* occ = orr ? reinterpret_cast<const int*>(reinterpret_cast<const char*>(orr) +
                                                         order_table_bytes(gr, batch))
                         : nullptr;
    const FlashBwdSet t = bwd_set(&a, &cl, 1, batch, gr.cls_bs);
    return KP == 32 ? launch_bwd<32>(t, gr, gc, batch, orr, occ, s) : launch_bwd<64>(t, gr, gc, batch, orr, occ, s);
}

size_t flash_ds_workspace_bytes(size_t batch, size_t M, size_t N, size_t K)
{
    const int KP = pad32(K);
    const size_t part = std::max(part_bytes(geo(batch, M, N, true, dq_pw(KP), nullptr, nullptr), batch, true),
                                 part_bytes(geo(batch, M, N, false, cols_pw(KP), nullptr, nullptr), batch, false));
    return align256(batch * M * N * sizeof(float)) + align256(batch * M * sizeof(float)) + part;
}

int flash_backward_ds_rows(const FlashBwdArgs* a, const float* const* O, int o_qm, const unsigned char* const* cells,
                           int rows, size_t hpr, void* ws, const int* order, hipStream_t s)
{
    if (!ws || rows < 1 || rows > kFlashMaxRows || hpr == 0) return -1;
    for (int r = 0; r < rows; ++r)
        if (!same_launch(a[0], a[r]) || a[r].K != a[r].Kd || !O[r] || (a[r].mask && !cells[r])) return -1;
    const size_t batch = static_cast<size_t>(rows) * hpr;
    const size_t M = static_cast<size_t>(a[0].M), N = static_cast<size_t>(a[0].N);
    // Workspace: dS of every entry, R where the caller keeps none, then the range partials.
    char* w = static_cast<char*>(ws);
    float* dS = reinterpret_cast<float*>(w);
    w += align256(batch * M * N * sizeof(float));
    float* Rw = reinterpret_cast<float*>(w);
    w += align256(batch * M * sizeof(float));
    FlashBwdArgs x[kFlashMaxRows];
    RowdotSet rd{};
    for (int r = 0; r < rows; ++r)
    {
        const size_t b0 = static_cast<size_t>(r) * hpr;
        x[r] = a[r];
        x[r].dS = dS + b0 * M * N;
        if (!x[r].R) x[r].R = Rw + b0 * M;
        x[r].g_do = 1;
        rd.dO[r] = x[r].dO;
        rd.O[r] = O[r];
        rd.R[r] = x[r].R;
    }
    const int KP = pad32(static_cast<size_t>(x[0].K));
    const unsigned char* cl0 = x[0].mask ? cells[0] : nullptr;
    const bool pb = x[0].mask && x[0].mask_bs != 0;
    FlashGeo gr = geo(batch, M, N, true, dq_pw(KP), cl0, w, pb);
    FlashGeo gc = geo(batch, M, N, false, cols_pw(KP), cl0, w, pb);
    if (x[0].mask && order)
    {
        gc.order = order;
        gr.order = reinterpret_cast<const int*>(reinterpret_cast<const char*>(order) + order_table_bytes(gc, batch));
    }
    const FlashBwdSet t = bwd_set(x, cells, rows, hpr, gr.cls_bs);
    const long total = static_cast<long>(hpr * M);
    hipLaunchKernelGGL(k_flash_rowdot, dim3(static_cast<unsigned>((total + 63) / 64), static_cast<unsigned>(rows)),
                       dim3(256), 0, s, rd, x[0].M, x[0].Kd, total, x[0].alpha2, o_qm ? 1 : 0);
    if (int rc = launch_status()) return rc;
    auto run = [&](auto kp) -> int {
        constexpr int P = decltype(kp)::value;
        if (x[0].S)
            hipLaunchKernelGGL((k_flash_bwd_cols<P, true, true, true>), dim3(grid_of(gc, batch)), dim3(64 * kWaves), 0,
                               s, t, gc);
        else
            hipLaunchKernelGGL((k_flash_bwd_cols<P, true, true>), dim3(grid_of(gc, batch)), dim3(64 * kWaves), 0, s,
                               t, gc);
        if (int rc = launch_status()) return rc;
        if (gc.NR > 1)
        {
            hipLaunchKernelGGL((k_flash_bwd_cols_combine<P>), dim3(static_cast<unsigned>(batch * gc.CT)), dim3(256),
                               0, s, t, gc);
            if (int rc = launch_status()) return rc;
        }
        hipLaunchKernelGGL((k_flash_bwd_dq<P>), dim3(grid_of(gr, batch)), dim3(64 * kWaves), 0, s, t, gr);
        if (int rc = launch_status()) return rc;
        if (gr.NR > 1)
        {
            hipLaunchKernelGGL((k_flash_bwd_dq_combine<P>), dim3(static_cast<unsigned>(batch * gr.RT)), dim3(256),
                               0, s, t, gr);
            if (int rc = launch_status()) return rc;
        }
        return 0;
    };
    return KP == 32 ? run(std::integral_constant<int, 32>{}) : run(std::integral_constant<int, 64>{});
}

int flash_backward_ds(const FlashBwdArgs& a, const float* O, int o_qm, const unsigned char* cells, size_t batch,
                      void* ws, const int* order, hipStream_t s)
{
    return flash_backward_ds_rows(&a, &O, o_qm, &cells, 1, batch, ws, order, s);
}

} // namespace nnhip

// ── C-ABI (include/nnhip_kernels.h) ─────────────────────────────────────────
extern "C" size_t nnhip_flash_ds_workspace_bytes(size_t batch, size_t M, size_t N, size_t K)
{
    return nnhip::flash_ds_workspace_bytes(batch, M, N, K);
}

extern "C" int nnhip_flash_backward_ds(const float* Q, const float* Kt, const float* dO, const float* Vp,
                                       const float* O, const float* mask, const void* cells, const float* m,
                                       const float* l, float* dQ, float* dK, float* dV, size_t batch, size_t M,
                                       size_t N, size_t K, float alpha, float alpha2, size_t mask_batch_stride,
                                       void* workspace, void* stream)
{
    return nnhip_flash_backward_ds_ordered(Q, Kt, dO, Vp, O, 0, mask, cells, m, l, nullptr, dQ, dK, dV, batch, M, N,
                                           K, alpha, alpha2, mask_batch_stride, nullptr, nullptr, workspace, stream);
}

extern "C" int nnhip_flash_backward_ds_ordered(const float* Q, const float* Kt, const float* dO, const float* Vp,
                                               const float* O, int o_query_major, const float* mask,
                                               const void* cells, const float* m, const float* l, float* R, float* dQ,
                                               float* dK, float* dV, size_t batch, size_t M, size_t N, size_t K,
                                               float alpha, float alpha2, size_t mask_batch_stride,
                                               const float* scores, const void* order, void* workspace, void* stream)
{
    if (!Q || !Kt || !dO || !Vp || !O || !m || !l || !dQ || !dK || !dV || !workspace || (mask && !cells)) return -1;
    if (mask && mask_batch_stride != 0 && mask_batch_stride < M * N) return -1;
    if (!nnhip::flash_supported(batch, M, N, K, 4) || K % 4 != 0) return -3;
    nnhip::FlashBwdArgs a{Q, Kt, dO, Vp, nullptr, mask, m, l, R, dQ, dK, dV, static_cast<int>(M),
                          static_cast<int>(N), static_cast<int>(K), static_cast<int>(K), static_cast<int>(K), alpha,
                          alpha2};
    a.mask_bs = mask ? static_cast<long>(mask_batch_stride) : 0;
    a.S = scores;
    return nnhip::flash_backward_ds(a, O, o_query_major, static_cast<const unsigned char*>(cells), batch, workspace,
                                    static_cast<const int*>(order), static_cast<hipStream_t>(stream));
}

extern "C" int nnhip_flash_supported(size_t batch, size_t M, size_t N, size_t K, size_t D)
{
    return nnhip::flash_supported(batch, M, N, K, D) ? 1 : 0;
}

extern "C" size_t nnhip_flash_cells_bytes(size_t M, size_t N) { return nnhip::flash_cells_bytes(M, N); }

extern "C" int nnhip_flash_classify(const float* mask, size_t M, size_t N, void* cells, void* stream)
{
    return nnhip_flash_classify_batched(mask, 1, 0, M, N, cells, stream);
}

extern "C" int nnhip_flash_classify_batched(const float* mask, size_t masks, size_t mask_batch_stride, size_t M,
                                            size_t N, void* cells, void* stream)
{
    if (!mask || !cells || M == 0 || N == 0 || masks == 0) return -1;
    if (masks > 1 && mask_batch_stride < M * N) return -1;
    if (M > (size_t{1} << 24) || N > (size_t{1} << 24) || masks > 65535) return -3;
    return nnhip::flash_classify(mask, masks, static_cast<long>(mask_batch_stride), M, N, cells,
                                 static_cast<hipStream_t>(stream));
}

extern "C" size_t nnhip_flash_workspace_bytes(size_t batch, size_t M, size_t N, size_t K, size_t D, int backward)
{
    return nnhip::flash_workspace_bytes(batch, M, N, K, D, backward != 0);
}

extern "C" int nnhip_flash_forward(const float* Q, const float* Kt, const float* V, const float* mask,
                                   const void* cells, float* m, float* l, float* O, size_t batch, size_t M, size_t N,
                                   size_t K, size_t D, float alpha, void* workspace, void* stream)
{
    return nnhip_flash_forward_layout(Q, Kt, V, mask, cells, m, l, O, batch, M, N, K, D, alpha, 0, 0, 0, workspace,
                                      stream);
}

extern "C" int nnhip_flash_forward_layout(const float* Q, const float* Kt, const float* V, const float* mask,
                                          const void* cells, float* m, float* l, float* O, size_t batch, size_t M,
                                          size_t N, size_t K, size_t D, float alpha, size_t mask_batch_stride,
                                          int v_dim_major, int o_dim_major, void* workspace, void* stream)
{
    return nnhip_flash_forward_ordered(Q, Kt, V, mask, cells, m, l, O, batch, M, N, K, D, alpha, mask_batch_stride,
                                       v_dim_major, o_dim_major, nullptr, nullptr, workspace, stream);
}

extern "C" int nnhip_flash_forward_ordered(const float* Q, const float* Kt, const float* V, const float* mask,
                                           const void* cells, float* m, float* l, float* O, size_t batch, size_t M,
                                           size_t N, size_t K, size_t D, float alpha, size_t mask_batch_stride,
                                           int v_dim_major, int o_dim_major, float* scores, const void* order,
                                           void* workspace, void* stream)
{
    if (!Q || !Kt || !m || !l || (O && !V) || (mask && !cells)) return -1;
    if (mask && mask_batch_stride != 0 && mask_batch_stride < M * N) return -1;
    if (!nnhip::flash_supported(batch, M, N, K, O ? D : 4)) return -3;
    nnhip::FlashFwdArgs a{Q, Kt, V, mask, m, l, O, static_cast<int>(M), static_cast<int>(N), static_cast<int>(K),
                          static_cast<int>(O ? D : 4), alpha};
    a.mask_bs = mask ? static_cast<long>(mask_batch_stride) : 0;
    a.v_dm = v_dim_major ? 1 : 0;
    a.o_dm = o_dim_major ? 1 : 0;
    a.S = scores;
    return nnhip::flash_forward(a, static_cast<const unsigned char*>(cells), batch, workspace,
                                static_cast<const int*>(order), static_cast<hipStream_t>(stream));
}

extern "C" int nnhip_flash_backward(const float* Q, const float* Kt, const float* dO, const float* Vp, const float* G,
                                    size_t ldg, const float* mask, const void* cells, const float* m, const float* l,
                                    float* R, float* dQ, float* dK, float* dV, size_t batch, size_t M, size_t N,
                                    size_t K, size_t Kd, float alpha, float alpha2, void* workspace, void* stream)
{
    if (!G) return -1;
    return nnhip_flash_backward_layout(Q, Kt, dO, Vp, G, ldg, mask, cells, m, l, R, dQ, dK, dV, batch, M, N, K, Kd,
                                       alpha, alpha2, 0, 0, workspace, stream);
}

extern "C" int nnhip_flash_backward_layout(const float* Q, const float* Kt, const float* dO, const float* Vp,
                                           const float* G, size_t ldg, const float* mask, const void* cells,
                                           const float* m, const float* l, float* R, float* dQ, float* dK, float* dV,
                                           size_t batch, size_t M, size_t N, size_t K, size_t Kd, float alpha,
                                           float alpha2, size_t mask_batch_stride, int g_is_do, void* workspace,
                                           void* stream)
{
    return nnhip_flash_backward_ordered(Q, Kt, dO, Vp, G, ldg, mask, cells, m, l, R, dQ, dK, dV, batch, M, N, K, Kd,
                                        alpha, alpha2, mask_batch_stride, g_is_do, nullptr, workspace, stream);
}

extern "C" int nnhip_flash_backward_ordered(const float* Q, const float* Kt, const float* dO, const float* Vp,
                                            const float* G, size_t ldg, const float* mask, const void* cells,
                                            const float* m, const float* l, float* R, float* dQ, float* dK,
                                            float* dV, size_t batch, size_t M, size_t N, size_t K, size_t Kd,
                                            float alpha, float alpha2, size_t mask_batch_stride, int g_is_do,
                                            const void* order, void* workspace, void* stream)
{
    if (!Q || !Kt || !dO || !Vp || (!G && !g_is_do) || !m || !l || !R || !dQ || !dK || !dV || (mask && !cells))
        return -1;
    if (mask && mask_batch_stride != 0 && mask_batch_stride < M * N) return -1;
    if (g_is_do && Kd != K) return -1;
    if (g_is_do) ldg = K;
    if (!nnhip::flash_supported(batch, M, N, K > Kd ? K : Kd, 4) || K % 4 != 0 || ldg < K || ldg % 4 != 0 ||
        M * ldg >= (size_t{1} << 29))
        return -3;
    nnhip::FlashBwdArgs a{Q, Kt, dO, Vp, G, mask, m, l, R, dQ, dK, dV, static_cast<int>(M), static_cast<int>(N),
                          static_cast<int>(K), static_cast<int>(Kd), static_cast<int>(ldg), alpha, alpha2};
    a.mask_bs = mask ? static_cast<long>(mask_batch_stride) : 0;
    a.g_do = g_is_do ? 1 : 0;
    return nnhip::flash_backward(a, static_cast<const unsigned char*>(cells), batch, workspace,
                                 static_cast<const int*>(order), static_cast<hipStream_t>(stream));
}

extern "C" size_t nnhip_flash_order_bytes(size_t batch, size_t M, size_t N, int kind)
{
    if (kind < 0 || kind > 2 || batch == 0 || M == 0 || N == 0) return 0;
    return nnhip::flash_order_bytes(batch, M, N, kind);
}

extern "C" int nnhip_flash_build_order(const void* cells, size_t batch, size_t M, size_t N, size_t mask_batch_stride,
                                       int kind, void* order, void* stream)
{
    if (!cells || !order || kind < 0 || kind > 2) return -1;
    if (!nnhip::flash_supported(batch, M, N, 1, 4)) return -3;
    return nnhip::flash_build_order(static_cast<const unsigned char*>(cells), batch, M, N, mask_batch_stride != 0,
                                    kind, order, static_cast<hipStream_t>(stream));
}

extern "C" int nnhip_flash_forward_rows(const nnhip_flash_fwd_row* rows, size_t nrows, size_t hpr, size_t M, size_t N,
                                        size_t K, size_t D, float alpha, int v_dim_major, int o_dim_major,
                                        const void* order, void* workspace, void* stream)
{
    if (!rows || nrows == 0 || nrows > static_cast<size_t>(nnhip::kFlashMaxRows) || hpr == 0) return -1;
    if (!nnhip::flash_supported(nrows * hpr, M, N, K, D)) return -3;
    nnhip::FlashFwdArgs a[nnhip::kFlashMaxRows];
    const unsigned char* cells[nnhip::kFlashMaxRows];
    for (size_t r = 0; r < nrows; ++r)
    {
        const nnhip_flash_fwd_row& x = rows[r];
        if (!x.Q || !x.Kt || !x.m || !x.l || (x.O && !x.V) || (x.mask && !x.cells)) return -1;
        a[r] = nnhip::FlashFwdArgs{x.Q, x.Kt, x.V, x.mask, x.m, x.l, x.O, static_cast<int>(M), static_cast<int>(N),
                                   static_cast<int>(K), static_cast<int>(x.O ? D : 4), alpha};
        a[r].v_dm = v_dim_major ? 1 : 0;
        a[r].o_dm = o_dim_major ? 1 : 0;
        a[r].S = x.scores;
        cells[r] = static_cast<const unsigned char*>(x.cells);
    }
    return nnhip::flash_forward_rows(a, cells, static_cast<int>(nrows), hpr, workspace, static_cast<const int*>(order),
                                     static_cast<hipStream_t>(stream));
}

extern "C" int nnhip_flash_backward_ds_rows(const nnhip_flash_bwd_row* rows, size_t nrows, size_t hpr, size_t M,
                                            size_t N, size_t K, float alpha, float alpha2, int o_query_major,
                                            const void* order, void* workspace, void* stream)
{
    if (!rows || nrows == 0 || nrows > static_cast<size_t>(nnhip::kFlashMaxRows) || hpr == 0 || !workspace) return -1;
    if (!nnhip::flash_supported(nrows * hpr, M, N, K, 4) || K % 4 != 0) return -3;
    nnhip::FlashBwdArgs a[nnhip::kFlashMaxRows];
    const float* O[nnhip::kFlashMaxRows];
    const unsigned char* cells[nnhip::kFlashMaxRows];
    for (size_t r = 0; r < nrows; ++r)
    {
        const nnhip_flash_bwd_row& x = rows[r];
        if (!x.Q || !x.Kt || !x.dO || !x.Vp || !x.O || !x.m || !x.l || !x.dQ || !x.dK || !x.dV || (x.mask && !x.cells))
            return -1;
        a[r] = nnhip::FlashBwdArgs{x.Q, x.Kt, x.dO, x.Vp, nullptr, x.mask, x.m, x.l, x.R, x.dQ, x.dK, x.dV,
                                   static_cast<int>(M), static_cast<int>(N), static_cast<int>(K), static_cast<int>(K),
                                   static_cast<int>(K), alpha, alpha2};
        a[r].S = x.scores;
        O[r] = x.O;
        cells[r] = static_cast<const unsigned char*>(x.cells);
    }
    return nnhip::flash_backward_ds_rows(a, O, o_query_major, cells, static_cast<int>(nrows), hpr, workspace,
                                         static_cast<const int*>(order), static_cast<hipStream_t>(stream));
}

extern "C" int nnhip_flash_build_rows_order(const void* const* cells, size_t nrows, size_t hpr, size_t M, size_t N,
                                            int kind, void* order, void* stream)
{
    if (!cells || !order || kind < 0 || kind > 2 || nrows == 0 || nrows > static_cast<size_t>(nnhip::kFlashMaxRows))
        return -1;
    if (!nnhip::flash_supported(nrows * hpr, M, N, 1, 4)) return -3;
    return nnhip::flash_build_rows_order(reinterpret_cast<const unsigned char* const*>(cells), static_cast<int>(nrows),
                                         hpr, M, N, false, kind, order, static_cast<hipStream_t>(stream));
}
