// k_attn_mfma.hip — the fused attention primitives on the fp32 matrix cores.
//
// Same semantics as the general path in k_attention.hip (CPU engine,
// cpu_engine.hpp:426-915), for head dims K <= 128 and value widths D <= 128:
//   s_ij = alpha * dot_k(Q(i,k), Kt(k,j)) + mask(i,j),  W_ij = exp(s_ij - m_i) / l_i  (0 where s_ij = -inf)
// with Q(i,k) = A_b(i,k) and Kt(k,j) = B_b(k,j) in the transpose conventions of
// ComputeEngine (compute_engine.hpp:217-276).
//
// Work decomposition. The (M, N) score plane of each batch is cut into 32x32
// cells. A work item is one wave (64 lanes, no block barriers) that owns a
// 32-wide line of cells (32 queries; 32 keys for backward_kv) and a range of
// kCells consecutive cells along it. Items cost at most kCells cells however
// the mask distributes the allowed pairs, and there are thousands of them, so
// causal and document masks balance over the 1024 SIMDs by themselves. A line
// with a single non-empty range writes its output directly; otherwise each
// item writes a partial result (maxima, sums, output rows) to the workspace and
// a combine kernel adds a line's partials in range order, so results do not
// depend on scheduling. (Combining inside the item kernel would need
// device-scope release/acquire between workgroups, i.e. a write-back of the
// whole L2 per item on this GPU: far slower than a second launch.)
//
// Per cell: one v_mfma_f32_32x32x2_f32 chain over k computes the score tile
// (transposed, S^T = Kt^T Q, in the query-line kernels: each lane then owns one
// query, and the score registers are already laid out as the B operand of the
// next MFMA, O^T = V^T W^T or dQ^T = Kt dS^T). Operands come straight from
// global memory (L2) into registers; the next cell's score operand is loaded
// while the current cell computes. The two operands that need a transpose (Kt
// for dQ, Q for dK) go through a wave-private LDS tile.
//
// MFMA 32x32x2 operand layout (lane l, h = l/32, c = l%32), step r of 2 k's:
//   A[row c][k h], B[k h][col c];  D register r <-> row drow(r,h), col c,
//   drow(r,h) = 8*(r/4) + 4*h + r%4.
// Feeding D registers as a B operand, step r consumes reduction indices
// drow(r,0) and drow(r,1): over r = 0..15 each of the 32 is used once, and the
// A operand is read with the same index map.
//
// Masks: a pre-pass classifies every cell of the shared (M,N) mask as all
// -inf (skipped), all zero (no mask read) or general.
#include "attn_mfma.hpp"
#include "common.hpp"

namespace nnhip
{
namespace
{

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr float kNegInf = -__builtin_huge_valf();
constexpr int kCells = 8;         // cells per work item along its line (a range)
constexpr int kStep = 2;          // cells staged per pipeline step
constexpr int kSteps = kCells / kStep;
constexpr int kMaxTiles = 1024;   // 32-wide tiles per axis: M, N <= 32768

enum { kRowMax = 0, kRowDenom = 1, kRowApply = 2, kRowR = 3, kRowDQ = 4 };

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

// Geometry and workspace of one call (identical for every item).
struct Work
{
    int RT, CT;                  // query tiles, key tiles
    int NR;                      // ranges per line: ceil(tiles along the line / kCells)
    const unsigned char* cls;    // RT x CT cell classes (unused without a mask: every cell is class 1)
    float* part;                 // partial results, pw floats per item
    int pw;
};

__global__ __launch_bounds__(256) void k_attn_classify(const float* __restrict__ mask, int M, int N, int CT,
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

// Workgroups are dispatched round-robin over the 8 XCDs, each with its own L2.
// Maps the 1-D workgroup id to a work item so that each XCD runs one
// contiguous run of items: the items of one batch entry (which re-read its
// query and key tiles) then share an L2.
__device__ __forceinline__ int xcd_item(int bid, int nb)
{
    const int x = bid % 8, k = bid / 8, q = nb / 8, r = nb % 8;
    return x * q + min(x, r) + k;
}

__device__ __forceinline__ int cell_class(const AttnArgs& d, const Work& w, int ib, int jb)
{
    return !d.mask ? 1 : w.cls[(long)ib * w.CT + jb];
}

// What an item knows about its line: its own non-empty / general cells (bit t
// = cell rg*kCells + t) and which ranges of the line are non-empty.
struct LineInfo
{
    unsigned mine_nz = 0, mine_gen = 0;
    int nne = 0;
    unsigned long long ranges[kMaxTiles / kCells / 64] = {};
};

// rows: the line is query tile `line`, cells run along keys; else key tile, cells along queries.
__device__ LineInfo line_info(const AttnArgs& d, const Work& w, bool rows, int line, int rg)
{
    static_assert(kCells == 8, "range packing below assumes 8 cells (one byte) per range");
    LineInfo li;
    const int nx = rows ? w.CT : w.RT;
    const int lane = threadIdx.x & 63;
    for (int x0 = 0; x0 < nx; x0 += 64)
    {
        const int x = x0 + lane;
        const int cl = x < nx ? (rows ? cell_class(d, w, line, x) : cell_class(d, w, x, line)) : 0;
        const unsigned long long nz = __ballot(cl != 0);
        const unsigned long long gen = __ballot(cl == 2);
        unsigned long long packed = 0;   // bit q: range x0/kCells + q is non-empty
#pragma unroll
        for (int q = 0; q < 64 / kCells; ++q) packed |= (((nz >> (kCells * q)) & 0xFFull) != 0 ? 1ull : 0ull) << q;
        li.nne += __popcll(packed);
        const int rb = x0 / kCells;
#pragma unroll
        for (int q = 0; q < kMaxTiles / kCells / 64; ++q)   // constant indices keep the words in registers
            if (rb / 64 == q) li.ranges[q] |= packed << (rb % 64);
        const int xb = rg * kCells;
        if (xb >= x0 && xb < x0 + 64)
        {
            li.mine_nz = static_cast<unsigned>((nz >> (xb - x0)) & 0xFF);
            li.mine_gen = static_cast<unsigned>((gen >> (xb - x0)) & 0xFF);
        }
    }
    return li;
}

// f(range) for each non-empty range of the line, in range order.
template <class F>
__device__ __forceinline__ void for_ranges(const LineInfo& li, int nr, F f)
{
#pragma unroll
    for (int q = 0; q < kMaxTiles / kCells / 64; ++q)
    {
        if (q * 64 >= nr) break;
        unsigned long long m = li.ranges[q];
        while (m)
        {
            const int t = __builtin_ctzll(m);
            m &= m - 1;
            f(q * 64 + t);
        }
    }
}

// Writes a query line's output tiles from the registers' (k = 32u + drow(r,h), query qi) layout:
// O[(b*M + qi)*D + k] (apply) or dQ[(b*K + k)*M + qi] = alpha * value.
template <bool APPLY, int NU>
__device__ __forceinline__ void store_row_tiles(const AttnArgs& d, float* out, int D, int b, int qi, int h,
                                                const f32x16* acc)
{
    if (qi >= d.M) return;
#pragma unroll
    for (int u = 0; u < NU; ++u)
#pragma unroll
        for (int r = 0; r < 16; ++r)
        {
            const int k = 32 * u + drow(r, h);
            if constexpr (APPLY)
            {
                if (k < D) out[((long)b * d.M + qi) * D + k] = acc[u][r];
            }
            else if (k < d.K)
                out[((long)b * d.K + k) * d.M + qi] = d.alpha * acc[u][r];
        }
}

// ── query-line kernel: forward row max / denominators / apply, backward R / dQ ──
// A workgroup is 4 waves = 4 consecutive query lines sharing one key range.
// The range is walked kStep cells at a time through two LDS buffers: the key
// (and value) tiles of the next step are loaded into registers while the
// current step's MFMAs run, then written to the other buffer (one barrier per
// step, as in the GEMM).
constexpr int kWaves = 4;

// Which steps of the range any wave of the workgroup has work in.
__device__ __forceinline__ unsigned steps_needed(unsigned need)
{
    unsigned m = 0;
#pragma unroll
    for (int s = 0; s < kSteps; ++s)
        if ((need >> (kStep * s)) & ((1u << kStep) - 1)) m |= 1u << s;
    return m;
}

template <int KP, int MODE, int DU>
__global__ __launch_bounds__(64 * kWaves) void k_attn_rows(AttnArgs d, Work w, const float* __restrict__ row_max,
                                                           const float* __restrict__ denom,
                                                           const float* __restrict__ V, int D,
                                                           const float* __restrict__ P,
                                                           const float* __restrict__ Rin, float* __restrict__ out)
{
    constexpr int NT = 64 * kWaves;
    constexpr bool APPLY = MODE == kRowApply, DQ = MODE == kRowDQ, USE_P = MODE == kRowR || MODE == kRowDQ;
    constexpr bool SCALAR = MODE == kRowMax || MODE == kRowDenom || MODE == kRowR;
    constexpr int NU = APPLY ? DU : (DQ ? KP / 32 : 1);   // 32-wide output subtiles held by a wave
    constexpr int VS = DU * 32 + 8;                       // value row stride: rows 4 apart use disjoint banks
    constexpr int PK = KP * 32 / NT, PV = APPLY ? 32 * DU * 32 / NT : 1;   // per thread, per staged cell
    static_assert(PK * NT == KP * 32 && (!APPLY || PV * NT == 32 * DU * 32), "staging covers each tile exactly");
    __shared__ float Ks[2][kStep][KP][33];                // Ks[buf][t][k][jj] = Kt(k, jbase_t + jj)
    __shared__ float Vs[APPLY ? 2 : 1][APPLY ? kStep : 1][APPLY ? 32 : 1][APPLY ? VS : 1];
    __shared__ unsigned need_s;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, h = lane >> 5, c = lane & 31;
    const int per = (w.RT + kWaves - 1) / kWaves * w.NR;
    const int item = xcd_item(blockIdx.x, gridDim.x), b = item / per, grp = item % per / w.NR, rg = item % w.NR;
    const int row = grp * kWaves + wave, qi = row * 32 + c;
    const LineInfo li = row < w.RT ? line_info(d, w, true, row, rg) : LineInfo{};
    if (threadIdx.x == 0) need_s = 0;
    __syncthreads();
    if (lane == 0 && li.mine_nz) atomicOr(&need_s, li.mine_nz);
    __syncthreads();
    const unsigned steps = steps_needed(need_s);   // steps of the range any wave computes

    // A line without any allowed pair still has outputs: lowest() maxima, zero sums and rows.
    auto write_empty_line = [&]() {
        if (li.nne != 0 || rg != 0 || row >= w.RT || qi >= d.M) return;
        if constexpr (SCALAR)
        {
            if (h == 0) out[(long)b * d.M + qi] = MODE == kRowMax ? kLowest : 0.0f;
        }
        else
        {
            const int width = APPLY ? D : d.K;
            for (int k = h; k < width; k += 2)
                out[APPLY ? ((long)b * d.M + qi) * D + k : ((long)b * d.K + k) * d.M + qi] = 0.0f;
        }
    };
    if (steps == 0)
    {
        write_empty_line();
        return;
    }

    const float* Ab = d.A + (long)b * d.M * d.K;
    const float* Bb = d.B + (long)b * d.K * d.N;
    const float* Vb = APPLY ? V + (long)b * d.N * D : nullptr;
    // Register staging of one step's tiles (clamped addresses; out-of-range values are zeroed when stored).
    float kr[kStep][PK], vr[kStep][PV];
    auto load_step = [&](int st) {
#pragma unroll
        for (int t = 0; t < kStep; ++t)
        {
            const int jbase = 32 * (rg * kCells + st * kStep + t);
#pragma unroll
            for (int u = 0; u < PK; ++u)
            {
                const int e = threadIdx.x + u * NT;
                const int k = d.tB ? e % KP : e / 32, jj = d.tB ? e / KP : e % 32;
                kr[t][u] = kt_at(d, Bb, min(k, d.K - 1), min(jbase + jj, d.N - 1));
            }
            if constexpr (APPLY)
            {
#pragma unroll
                for (int u = 0; u < PV; ++u)
                {
                    const int e = threadIdx.x + u * NT, jj = e / (DU * 32), k = e % (DU * 32);
                    vr[t][u] = Vb[(long)min(jbase + jj, d.N - 1) * D + min(k, D - 1)];
                }
            }
        }
    };
    auto store_step = [&](int st, int buf) {
#pragma unroll
        for (int t = 0; t < kStep; ++t)
        {
            const int jbase = 32 * (rg * kCells + st * kStep + t);
#pragma unroll
            for (int u = 0; u < PK; ++u)
            {
                const int e = threadIdx.x + u * NT;
                const int k = d.tB ? e % KP : e / 32, jj = d.tB ? e / KP : e % 32;
                Ks[buf][t][k][jj] = (k < d.K && jbase + jj < d.N) ? kr[t][u] : 0.0f;
            }
            if constexpr (APPLY)
            {
#pragma unroll
                for (int u = 0; u < PV; ++u)
                {
                    const int e = threadIdx.x + u * NT, jj = e / (DU * 32), k = e % (DU * 32);
                    Vs[buf][t][jj][k] = (k < D && jbase + jj < d.N) ? vr[t][u] : 0.0f;
                }
            }
        }
    };
    auto next_step = [&](int st) {
        while (st < kSteps && !((steps >> st) & 1u)) ++st;
        return st;
    };
    int st = next_step(0);
    load_step(st);

    // This wave's queries: B operand of S^T, Q(qi, 2kk + h).
    const int qc = min(qi, d.M - 1);
    float qf[KP / 2];
#pragma unroll
    for (int kk = 0; kk < KP / 2; ++kk)
    {
        const int k = 2 * kk + h;
        const float x = q_at(d, Ab, qc, min(k, d.K - 1));
        qf[kk] = (qi < d.M && k < d.K) ? x : 0.0f;
    }
    float m_i = 0.0f, inv_l = 0.0f, r_i = 0.0f;
    if constexpr (MODE != kRowMax) m_i = row_max[(long)b * d.M + qc];
    if constexpr (MODE != kRowMax && MODE != kRowDenom) inv_l = 1.0f / denom[(long)b * d.M + qc];
    if constexpr (DQ) r_i = Rin[(long)b * d.M + qc];
    const float* prow = USE_P ? P + ((long)b * d.M + qc) * d.N : nullptr;
    const float* mrow = d.mask ? d.mask + (long)qc * d.N : nullptr;

    float red = MODE == kRowMax ? kLowest : 0.0f;
    f32x16 acc[NU];
#pragma unroll
    for (int u = 0; u < NU; ++u) acc[u] = zero16();

    int buf = 0;
    store_step(st, buf);
    __syncthreads();
    while (true)
    {
        const int nxt = next_step(st + 1);
        if (nxt < kSteps) load_step(nxt);   // in flight during this step's MFMAs
#pragma unroll
        for (int t = 0; t < kStep; ++t)
        {
            const int cell = st * kStep + t;
            if (!((li.mine_nz >> cell) & 1u)) continue;
            const int jbase = 32 * (rg * kCells + cell);
            // Side operands (consumed after the score chain).
            float mv[16], pv[USE_P ? 16 : 1];
            if ((li.mine_gen >> cell) & 1u)
            {
#pragma unroll
                for (int r = 0; r < 16; ++r) mv[r] = mrow[min(jbase + drow(r, h), d.N - 1)];
            }
            else
            {
#pragma unroll
                for (int r = 0; r < 16; ++r) mv[r] = 0.0f;
            }
            if constexpr (USE_P)
            {
#pragma unroll
                for (int r = 0; r < 16; ++r) pv[r] = prow[min(jbase + drow(r, h), d.N - 1)];
            }
            f32x16 sacc = zero16();
#pragma unroll
            for (int kk = 0; kk < KP / 2; ++kk) sacc = mfma(Ks[buf][t][2 * kk + h][c], qf[kk], sacc);
            float sv[16];
#pragma unroll
            for (int r = 0; r < 16; ++r)
                sv[r] = (jbase + drow(r, h) < d.N && qi < d.M) ? d.alpha * sacc[r] + mv[r] : kNegInf;
            if constexpr (MODE == kRowMax)
            {
#pragma unroll
                for (int r = 0; r < 16; ++r) red = fmax_std(red, sv[r]);
            }
            else if constexpr (MODE == kRowDenom)
            {
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (sv[r] != kNegInf) red += expf(sv[r] - m_i);
            }
            else
            {
                float wv[16];
#pragma unroll
                for (int r = 0; r < 16; ++r) wv[r] = sv[r] == kNegInf ? 0.0f : expf(sv[r] - m_i) * inv_l;
                if constexpr (MODE == kRowR)
                {
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        if (sv[r] != kNegInf) red += wv[r] * pv[r];
                }
                else if constexpr (APPLY)
                {
#pragma unroll
                    for (int u = 0; u < DU; ++u)
#pragma unroll
                        for (int r = 0; r < 16; ++r)
                            acc[u] = mfma(Vs[buf][t][drow(r, h)][32 * u + c], wv[r], acc[u]);
                }
                else   // dQ: A operand Kt(32u + c, jbase + drow(r,h)) read transposed from the staged tile
                {
#pragma unroll
                    for (int u = 0; u < KP / 32; ++u)
#pragma unroll
                        for (int r = 0; r < 16; ++r)
                            acc[u] = mfma(Ks[buf][t][32 * u + c][drow(r, h)], wv[r] * (pv[r] - r_i), acc[u]);
                }
            }
        }
        if (nxt >= kSteps) break;
        store_step(nxt, buf ^ 1);
        __syncthreads();
        buf ^= 1;
        st = nxt;
    }
    if (li.mine_nz == 0)
    {
        write_empty_line();
        return;
    }

    // Output: direct when the line has one non-empty range, else a partial for k_attn_combine_rows.
    const long line = (long)b * w.RT + row;
    if constexpr (SCALAR)
    {
        const float o = __shfl_xor(red, 32, 64);
        red = MODE == kRowMax ? fmax_std(red, o) : red + o;
        if (li.nne > 1)
        {
            if (h == 0) w.part[(line * w.NR + rg) * w.pw + c] = red;
        }
        else if (h == 0 && qi < d.M)
            out[(long)b * d.M + qi] = red;
    }
    else
    {
        if (li.nne > 1)
        {
            float* mine = w.part + (line * w.NR + rg) * w.pw;
#pragma unroll
            for (int u = 0; u < NU; ++u)
#pragma unroll
                for (int r = 0; r < 16; ++r) mine[(u * 16 + r) * 64 + lane] = acc[u][r];
        }
        else
            store_row_tiles<APPLY, NU>(d, out, D, b, qi, h, acc);
    }
}

// Sums (the row max: maxima of) the partials of every line with several non-empty ranges, in range order.
template <int MODE, int NU>
__global__ __launch_bounds__(64) void k_attn_combine_rows(AttnArgs d, Work w, int D, float* __restrict__ out)
{
    constexpr bool SCALAR = MODE == kRowMax || MODE == kRowDenom || MODE == kRowR;
    const int lane = threadIdx.x, h = lane >> 5, c = lane & 31;
    const int item = xcd_item(blockIdx.x, gridDim.x), row = item % w.RT, b = item / w.RT, qi = row * 32 + c;
    const LineInfo li = line_info(d, w, true, row, 0);
    if (li.nne <= 1) return;
    const long line = (long)b * w.RT + row;
    if constexpr (SCALAR)
    {
        float red = MODE == kRowMax ? kLowest : 0.0f;
        for_ranges(li, w.NR, [&](int q) {
            const float v = w.part[(line * w.NR + q) * w.pw + c];
            red = MODE == kRowMax ? fmax_std(red, v) : red + v;
        });
        if (h == 0 && qi < d.M) out[(long)b * d.M + qi] = red;
    }
    else
    {
        f32x16 acc[NU];
#pragma unroll
        for (int u = 0; u < NU; ++u) acc[u] = zero16();
        for_ranges(li, w.NR, [&](int q) {
            const float* pp = w.part + (line * w.NR + q) * w.pw;
            float t[NU * 16];   // all loads of a partial in flight before the sums
#pragma unroll
            for (int e = 0; e < NU * 16; ++e) t[e] = pp[e * 64 + lane];
#pragma unroll
            for (int u = 0; u < NU; ++u)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[u][r] += t[u * 16 + r];
        });
        store_row_tiles<MODE == kRowApply, NU>(d, out, D, b, qi, h, acc);
    }
}

// Writes a key line's dK / dV from the registers' (k = 32u + drow(r,h), key kj) layout.
template <int NU>
__device__ __forceinline__ void store_col_tiles(const AttnArgs& d, float* dK, float* dV, int b, int kj, int h,
                                                const f32x16* acck, const f32x16* accv)
{
    if (kj >= d.N) return;
#pragma unroll
    for (int u = 0; u < NU; ++u)
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

// ── key-line kernel: backward_kv ─────────────────────────────────────────────
//   dK[k][j] = alpha sum_i Q(i,k) W (P - R_i),  dV[k][j] = sum_i G(i,k) W
// A workgroup is 4 waves = 4 consecutive key lines sharing one query range,
// walked kStep query cells at a time through two LDS buffers (as k_attn_rows).
template <int KP>
__global__ __launch_bounds__(64 * kWaves) void k_attn_cols(AttnArgs d, Work w, const float* __restrict__ P,
                                                           const float* __restrict__ G, int D,
                                                           const float* __restrict__ R,
                                                           const float* __restrict__ row_max,
                                                           const float* __restrict__ denom, float* __restrict__ dK,
                                                           float* __restrict__ dV)
{
    constexpr int NT = 64 * kWaves;
    constexpr int NU = KP / 32;
    constexpr int GS = KP + 8;   // G row stride: rows 4 apart use disjoint banks
    constexpr int PQ = 32 * KP / NT;   // per thread, per staged cell
    static_assert(PQ * NT == 32 * KP, "staging covers each tile exactly");
    __shared__ float Qs[2][kStep][32][KP + 1];   // Qs[buf][t][ii][k] = Q(ibase_t + ii, k)
    __shared__ float Gs[2][kStep][32][GS];       // Gs[buf][t][ii][k] = G(ibase_t + ii, k)
    __shared__ float St[2][kStep][3][32];        // row max, denominator, R of the staged queries
    __shared__ unsigned need_s;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, h = lane >> 5, c = lane & 31;
    const int per = (w.CT + kWaves - 1) / kWaves * w.NR;
    const int item = xcd_item(blockIdx.x, gridDim.x), b = item / per, grp = item % per / w.NR, rg = item % w.NR;
    const int col = grp * kWaves + wave, kj = col * 32 + c;
    const LineInfo li = col < w.CT ? line_info(d, w, false, col, rg) : LineInfo{};
    if (threadIdx.x == 0) need_s = 0;
    __syncthreads();
    if (lane == 0 && li.mine_nz) atomicOr(&need_s, li.mine_nz);
    __syncthreads();
    const unsigned steps = steps_needed(need_s);
    auto write_empty_line = [&]() {   // a key line without any allowed pair: zero gradients
        if (li.nne != 0 || rg != 0 || col >= w.CT || kj >= d.N) return;
        for (int k = h; k < d.K; k += 2)
        {
            dK[((long)b * d.K + k) * d.N + kj] = 0.0f;
            dV[((long)b * d.K + k) * d.N + kj] = 0.0f;
        }
    };
    if (steps == 0)
    {
        write_empty_line();
        return;
    }

    const float* Ab = d.A + (long)b * d.M * d.K;
    const float* Bb = d.B + (long)b * d.K * d.N;
    const float* Gb = G + (long)b * d.M * D;
    float qr[kStep][PQ], gr[kStep][PQ], sr[kStep];
    auto load_step = [&](int st) {
#pragma unroll
        for (int t = 0; t < kStep; ++t)
        {
            const int ibase = 32 * (rg * kCells + st * kStep + t);
#pragma unroll
            for (int u = 0; u < PQ; ++u)
            {
                const int e = threadIdx.x + u * NT;
                const int ii = d.tA ? e % 32 : e / KP, k = d.tA ? e / 32 : e % KP;
                qr[t][u] = q_at(d, Ab, min(ibase + ii, d.M - 1), min(k, d.K - 1));
                const int gi = e / KP, gk = e % KP;
                gr[t][u] = Gb[(long)min(ibase + gi, d.M - 1) * D + min(gk, d.K - 1)];
            }
            const long si = (long)b * d.M + min(ibase + static_cast<int>(threadIdx.x % 32), d.M - 1);
            const int which = threadIdx.x / 32;   // threads 0-95 load the statistics
            sr[t] = which == 0 ? row_max[si] : which == 1 ? denom[si] : which == 2 ? R[si] : 0.0f;
        }
    };
    auto store_step = [&](int st, int buf) {
#pragma unroll
        for (int t = 0; t < kStep; ++t)
        {
            const int ibase = 32 * (rg * kCells + st * kStep + t);
#pragma unroll
            for (int u = 0; u < PQ; ++u)
            {
                const int e = threadIdx.x + u * NT;
                const int ii = d.tA ? e % 32 : e / KP, k = d.tA ? e / 32 : e % KP;
                Qs[buf][t][ii][k] = (ibase + ii < d.M && k < d.K) ? qr[t][u] : 0.0f;
                const int gi = e / KP, gk = e % KP;
                Gs[buf][t][gi][gk] = (ibase + gi < d.M && gk < d.K) ? gr[t][u] : 0.0f;
            }
            if (threadIdx.x < 96)
            {
                const int ii = threadIdx.x % 32, which = threadIdx.x / 32;
                St[buf][t][which][ii] = ibase + ii < d.M ? sr[t] : (which == 1 ? 1.0f : 0.0f);
            }
        }
    };
    auto next_step = [&](int st) {
        while (st < kSteps && !((steps >> st) & 1u)) ++st;
        return st;
    };
    int st = next_step(0);
    load_step(st);

    const int jc = min(kj, d.N - 1);
    float kf[KP / 2];   // B operand of S = Q Kt: Kt(2kk + h, kj)
#pragma unroll
    for (int kk = 0; kk < KP / 2; ++kk)
    {
        const int k = 2 * kk + h;
        const float x = kt_at(d, Bb, min(k, d.K - 1), jc);
        kf[kk] = (kj < d.N && k < d.K) ? x : 0.0f;
    }
    f32x16 acck[NU], accv[NU];
#pragma unroll
    for (int u = 0; u < NU; ++u)
    {
        acck[u] = zero16();
        accv[u] = zero16();
    }
    int buf = 0;
    store_step(st, buf);
    __syncthreads();
    while (true)
    {
        const int nxt = next_step(st + 1);
        if (nxt < kSteps) load_step(nxt);
#pragma unroll
        for (int t = 0; t < kStep; ++t)
        {
            const int cell = st * kStep + t;
            if (!((li.mine_nz >> cell) & 1u)) continue;
            const int ibase = 32 * (rg * kCells + cell);
            float pv[16], mv[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) pv[r] = P[((long)b * d.M + min(ibase + drow(r, h), d.M - 1)) * d.N + jc];
            if ((li.mine_gen >> cell) & 1u)
            {
#pragma unroll
                for (int r = 0; r < 16; ++r) mv[r] = d.mask[(long)min(ibase + drow(r, h), d.M - 1) * d.N + jc];
            }
            else
            {
#pragma unroll
                for (int r = 0; r < 16; ++r) mv[r] = 0.0f;
            }
            f32x16 sacc = zero16();
#pragma unroll
            for (int kk = 0; kk < KP / 2; ++kk) sacc = mfma(Qs[buf][t][c][2 * kk + h], kf[kk], sacc);
            float wv[16], ds[16];
#pragma unroll
            for (int r = 0; r < 16; ++r)
            {
                const int ii = drow(r, h);
                const bool ok = ibase + ii < d.M && kj < d.N;
                const float xs = ok ? d.alpha * sacc[r] + mv[r] : kNegInf;
                wv[r] = xs == kNegInf ? 0.0f : expf(xs - St[buf][t][0][ii]) / St[buf][t][1][ii];
                ds[r] = wv[r] * ((ok ? pv[r] : 0.0f) - St[buf][t][2][ii]);
            }
#pragma unroll
            for (int u = 0; u < NU; ++u)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                {
                    acck[u] = mfma(Qs[buf][t][drow(r, h)][32 * u + c], ds[r], acck[u]);
                    accv[u] = mfma(Gs[buf][t][drow(r, h)][32 * u + c], wv[r], accv[u]);
                }
        }
        if (nxt >= kSteps) break;
        store_step(nxt, buf ^ 1);
        __syncthreads();
        buf ^= 1;
        st = nxt;
    }
    if (li.mine_nz == 0)
    {
        write_empty_line();
        return;
    }

    const long line = (long)b * w.CT + col;
    if (li.nne > 1)   // partial for k_attn_combine_cols
    {
        float* mine = w.part + (line * w.NR + rg) * w.pw;
#pragma unroll
        for (int u = 0; u < NU; ++u)
#pragma unroll
            for (int r = 0; r < 16; ++r)
            {
                mine[(u * 16 + r) * 64 + lane] = acck[u][r];
                mine[((NU + u) * 16 + r) * 64 + lane] = accv[u][r];
            }
    }
    else
        store_col_tiles<NU>(d, dK, dV, b, kj, h, acck, accv);
}

template <int NU>
__global__ __launch_bounds__(64) void k_attn_combine_cols(AttnArgs d, Work w, float* __restrict__ dK,
                                                          float* __restrict__ dV)
{
    const int lane = threadIdx.x, h = lane >> 5, c = lane & 31;
    const int item = xcd_item(blockIdx.x, gridDim.x), col = item % w.CT, b = item / w.CT, kj = col * 32 + c;
    const LineInfo li = line_info(d, w, false, col, 0);
    if (li.nne <= 1) return;
    const long line = (long)b * w.CT + col;
    f32x16 acck[NU], accv[NU];
#pragma unroll
    for (int u = 0; u < NU; ++u)
    {
        acck[u] = zero16();
        accv[u] = zero16();
    }
    for_ranges(li, w.NR, [&](int q) {
        const float* pp = w.part + (line * w.NR + q) * w.pw;
        float t[2 * NU * 16];   // all loads of a partial in flight before the sums
#pragma unroll
        for (int e = 0; e < 2 * NU * 16; ++e) t[e] = pp[e * 64 + lane];
#pragma unroll
        for (int u = 0; u < NU; ++u)
#pragma unroll
            for (int r = 0; r < 16; ++r)
            {
                acck[u][r] += t[u * 16 + r];
                accv[u][r] += t[(NU + u) * 16 + r];
            }
    });
    store_col_tiles<NU>(d, dK, dV, b, kj, h, acck, accv);
}

// ── host side ────────────────────────────────────────────────────────────────
struct Layout
{
    int RT, CT, NRr, NRc, KP, DP;
    size_t cls_off, part_off, bytes;
};

size_t align256(size_t x) { return (x + 255) / 256 * 256; }

Layout layout(size_t batch, size_t M, size_t N, size_t K, size_t D)
{
    Layout L{};
    L.RT = static_cast<int>((M + 31) / 32);
    L.CT = static_cast<int>((N + 31) / 32);
    L.NRr = (L.CT + kCells - 1) / kCells;
    L.NRc = (L.RT + kCells - 1) / kCells;
    L.KP = K <= 64 ? 64 : 128;
    L.DP = static_cast<int>((D + 31) / 32 * 32);
    if (L.DP > 128) L.DP = 128;
    L.cls_off = 0;
    L.part_off = align256(static_cast<size_t>(L.RT) * L.CT);
    const size_t pw_rows = static_cast<size_t>(L.KP > L.DP ? L.KP : L.DP) * 32;
    const size_t pw_cols = static_cast<size_t>(2 * L.KP) * 32;
    const size_t rows = batch * L.RT * L.NRr * pw_rows, cols = batch * L.CT * L.NRc * pw_cols;
    L.bytes = L.part_off + align256((rows > cols ? rows : cols) * sizeof(float));
    return L;
}

int prep(const AttnArgs& d, const Layout& L, void* ws, hipStream_t s)
{
    if (!d.mask) return 0;
    hipLaunchKernelGGL(k_attn_classify, dim3(L.CT, L.RT), dim3(256), 0, s, d.mask, d.M, d.N, L.CT,
                       static_cast<unsigned char*>(ws) + L.cls_off);
    return launch_status();
}

Work work_of(const Layout& L, void* ws, bool rows, int pw)
{
    auto* base = static_cast<unsigned char*>(ws);
    Work w{};
    w.RT = L.RT;
    w.CT = L.CT;
    w.NR = rows ? L.NRr : L.NRc;
    w.cls = base + L.cls_off;
    w.part = reinterpret_cast<float*>(base + L.part_off);
    w.pw = pw;
    return w;
}

template <int KP, int MODE, int DU>
int launch_rows(const AttnArgs& d, const Work& w, size_t batch, const float* row_max, const float* denom,
                const float* V, int D, const float* P, const float* Rin, float* out, hipStream_t s)
{
    const unsigned groups = static_cast<unsigned>((w.RT + kWaves - 1) / kWaves);
    hipLaunchKernelGGL((k_attn_rows<KP, MODE, DU>), dim3(groups * w.NR * static_cast<unsigned>(batch)),
                       dim3(64 * kWaves), 0, s, d, w, row_max, denom, V, D, P, Rin, out);
    if (int rc = launch_status()) return rc;
    if (w.NR == 1) return 0;   // every line wrote its output directly
    constexpr int NU = MODE == kRowApply ? DU : (MODE == kRowDQ ? KP / 32 : 1);
    hipLaunchKernelGGL((k_attn_combine_rows<MODE, NU>), dim3(static_cast<unsigned>(w.RT) * static_cast<unsigned>(batch)),
                       dim3(64), 0, s, d, w, D, out);
    return launch_status();
}

template <int KP, int MODE>
int rows_by_width(const AttnArgs& d, const Work& w, size_t batch, const float* row_max, const float* denom,
                  const float* V, int D, const float* P, const float* Rin, float* out, hipStream_t s)
{
    if constexpr (MODE == kRowApply)
    {
        switch ((D + 31) / 32)
        {
        case 1: return launch_rows<KP, MODE, 1>(d, w, batch, row_max, denom, V, D, P, Rin, out, s);
        case 2: return launch_rows<KP, MODE, 2>(d, w, batch, row_max, denom, V, D, P, Rin, out, s);
        case 3: return launch_rows<KP, MODE, 3>(d, w, batch, row_max, denom, V, D, P, Rin, out, s);
        default: return launch_rows<KP, MODE, 4>(d, w, batch, row_max, denom, V, D, P, Rin, out, s);
        }
    }
    else
        return launch_rows<KP, MODE, 1>(d, w, batch, row_max, denom, V, D, P, Rin, out, s);
}

template <int MODE>
int rows_kernel(const AttnArgs& d, const Work& w, size_t batch, const float* row_max, const float* denom,
                const float* V, int D, const float* P, const float* Rin, float* out, hipStream_t s)
{
    return d.K <= 64 ? rows_by_width<64, MODE>(d, w, batch, row_max, denom, V, D, P, Rin, out, s)
                     : rows_by_width<128, MODE>(d, w, batch, row_max, denom, V, D, P, Rin, out, s);
}

} // namespace

size_t attn_workspace_bytes(size_t batch, size_t M, size_t N, size_t K, size_t D)
{
    return layout(batch, M, N, K, D).bytes;
}

bool attn_mfma_supported(size_t batch, size_t M, size_t N, size_t K)
{
    constexpr size_t span = 32 * kMaxTiles;
    const size_t cells = ((M + 31) / 32) * ((N + 31) / 32);   // bounds the 1-D grids of work items
    return K >= 1 && K <= 128 && batch >= 1 && batch <= 65535 && M >= 1 && N >= 1 && M <= span && N <= span &&
           cells * batch <= (size_t{1} << 30);
}

int attn_mfma_forward(const AttnArgs& d, size_t batch, int mode, const float* row_max, const float* denom,
                      const float* V, size_t D, float* out, void* workspace, hipStream_t s)
{
    if (mode == kFwdApply && (D == 0 || D > 128)) return -3;
    const Layout L = layout(batch, d.M, d.N, d.K, mode == kFwdApply ? D : 1);
    if (int rc = prep(d, L, workspace, s)) return rc;
    const int Di = static_cast<int>(D);
    switch (mode)
    {
    case kFwdMax:
        return rows_kernel<kRowMax>(d, work_of(L, workspace, true, 32), batch, nullptr, nullptr, nullptr, 0,
                                    nullptr, nullptr, out, s);
    case kFwdDenom:
        return rows_kernel<kRowDenom>(d, work_of(L, workspace, true, 32), batch, row_max, nullptr, nullptr,
                                      0, nullptr, nullptr, out, s);
    default:
        return rows_kernel<kRowApply>(d, work_of(L, workspace, true, 32 * L.DP), batch, row_max, denom, V,
                                      Di, nullptr, nullptr, out, s);
    }
}

int attn_mfma_backward(const AttnArgs& d, size_t batch, bool kv, const float* P, const float* G, size_t D,
                       const float* R_in, const float* row_max, const float* denom, float* o1, float* o2,
                       void* workspace, hipStream_t s)
{
    const Layout L = layout(batch, d.M, d.N, d.K, 1);
    if (int rc = prep(d, L, workspace, s)) return rc;
    if (!kv)
    {
        // R first (into o2), then dQ (o1).
        if (int rc = rows_kernel<kRowR>(d, work_of(L, workspace, true, 32), batch, row_max, denom, nullptr,
                                        0, P, nullptr, o2, s))
            return rc;
        return rows_kernel<kRowDQ>(d, work_of(L, workspace, true, 32 * L.KP), batch, row_max, denom, nullptr,
                                   0, P, o2, o1, s);
    }
    const Work w = work_of(L, workspace, false, 2 * 32 * L.KP);
    const dim3 grid(static_cast<unsigned>((L.CT + kWaves - 1) / kWaves * L.NRc) * static_cast<unsigned>(batch));
    const dim3 lines(static_cast<unsigned>(L.CT) * static_cast<unsigned>(batch));
    if (d.K <= 64)
        hipLaunchKernelGGL(k_attn_cols<64>, grid, dim3(64 * kWaves), 0, s, d, w, P, G, static_cast<int>(D), R_in, row_max,
                           denom, o1, o2);
    else
        hipLaunchKernelGGL(k_attn_cols<128>, grid, dim3(64 * kWaves), 0, s, d, w, P, G, static_cast<int>(D), R_in,
                           row_max, denom, o1, o2);
    if (int rc = launch_status()) return rc;
    if (w.NR == 1) return 0;
    if (d.K <= 64)
        hipLaunchKernelGGL(k_attn_combine_cols<2>, lines, dim3(64), 0, s, d, w, o1, o2);
    else
        hipLaunchKernelGGL(k_attn_combine_cols<4>, lines, dim3(64), 0, s, d, w, o1, o2);
    return launch_status();
}

} // namespace nnhip
