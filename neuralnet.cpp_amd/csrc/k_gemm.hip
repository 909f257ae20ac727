// k_gemm.hip — fp32 GEMM on the gfx950 matrix cores (v_mfma_f32_32x32x2_f32).
//
// Computes C_b = alpha * op(A_b) op(B_b) for `batch` row blocks, covering
// ComputeEngine::matmul (compute_engine.hpp:182-184) and ::batched_matmul
// (:195-199; cpu_engine.hpp:335-419 applies alpha after the product, so does
// the epilogue here). All four transpose combinations are handled at the
// global->LDS staging step: both operands are kept k-major in LDS
// (As[k][m], Bs[k][n]) so every MFMA fragment read is 32 consecutive floats.
//
// Tiling: a workgroup of WM x WN waves owns a (32*FM*WM) x (32*FN*WN) tile of
// C; each wave owns FM x FN MFMA 32x32 blocks (64 x 64 or 32 x 64).
// K advances 16 at a time through two LDS buffers: the next stage's global
// loads are issued into registers before the current stage's MFMAs and
// written to the other buffer afterwards (one barrier per stage). Tile ids are
// remapped so that each XCD (own L2) works on a contiguous, row-grouped slab.
// Small output grids with long K (weight gradients) split K across
// workgroups; the partial tiles are summed in order (deterministic).
//
// MFMA 32x32x2 f32 operand layout (per lane l, k-step of 2):
//   A: A[i = l%32][k = l/32],  B: B[k = l/32][j = l%32],
//   D: 16 values, value r at row 8*(r/4) + 4*(l/32) + r%4, column l%32.
#include <cmath>
#include <mutex>

#include "common.hpp"
#include "nnhip_kernels.h"

namespace nnhip
{
namespace
{

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int PAD = 4;

// Tile id for workgroup `bid` of `nt` tiles (tiles_m x tiles_n). Workgroups are
// dispatched round-robin over the 8 XCDs, each with its own L2: the remap
// gives every XCD a contiguous slab of tile ids, and the slab is walked in
// groups of kGroupM tile rows so that neighbours share A and B panels.
constexpr int kGroupM = 8;
__device__ __forceinline__ void tile_coords(int bid, int nt, int tiles_m, int tiles_n, int& tm, int& tn)
{
    int t = bid;
    if ((nt & 7) == 0) t = (bid & 7) * (nt >> 3) + (bid >> 3);
    const int per_group = kGroupM * tiles_n;
    const int g = t / per_group, first_m = g * kGroupM;
    const int gsize = min(tiles_m - first_m, kGroupM);
    const int r = t - g * per_group;
    tm = first_m + r % gsize;
    tn = r / gsize;
}

typedef float f4 __attribute__((ext_vector_type(4)));

// Up to four products of one shape (the attention's q, k, v projections of
// one input; the weight gradients of its four Linears): workgroup batch z takes
// member z / nb, batch z % nb of that member, whose B is B[member] when set
// and the launch's B otherwise. With KSEG instead: up to three products of one
// shape summed into one C (the q, k, v input gradients), k running through
// segment i = k / klen of A[i] and B[i] in turn.
//
// SEG: operands stored by sequence, as the attention's heads' layout holds a
// (rows, B * T) matrix: column c of the operand at (c / T) * step + c % T, its
// rows T apart. Member i's A has its k columns so (aT[i] = T, aS[i] = step;
// 0: plain), its B its n columns (untransposed B) or k columns (transposed).
// A tile (n) or stage (k) never straddles two sequences (T a multiple of the
// tile width and of BK), so this is an offset per tile or per stage.
constexpr int kGroupMax = 4;
struct GemmGroup
{
    const float* A[kGroupMax];
    float* C[kGroupMax];
    const float* bias[kGroupMax];
    int nb;
    const float* B[kGroupMax];
    int klen;
    int aT[kGroupMax], bT[kGroupMax];
    long aS[kGroupMax], bS[kGroupMax];
};

// RSUM: the row sums of A over k as well (Linear::backward's bias gradient
// grad_b += row_reduce_sum(G) beside grad_w += G Xᵀ, whose A is G): the
// workgroups of tile column 0 add up the A values they stage, per row, in the
// order they stage them; member i's sums go to dst[i] (added to it when acc),
// or, with split K, to part[(slice * members + i) * M + row] for the reduce.
struct RowSums
{
    float* dst[kGroupMax];
    float* part;
    int acc;
};

// WM x WN waves; each wave owns (32*FM) x (32*FN) of C as FM x FN MFMA 32x32 blocks.
// STATS: besides C, each workgroup writes the column softmax statistics of its
// BM rows of C (as stored, bias included): part[tile_m * N + n] = max over the
// rows, part[(tiles_m + tile_m) * N + n] = sum of exp(c - max) over them. The
// sparse cross-entropy that follows the product (the GPT's lm_head logits)
// merges these instead of reading C once more for them. Needs splits == 1.
template <int WM, int WN, int FM, int FN, int BK, bool TA, bool TB, bool GUARD, bool STATS = false, bool GRP = false,
          bool KSEG = false, bool RSUM = false, bool SEG = false>
__global__ __launch_bounds__(64 * WM * WN) void k_gemm(const float* __restrict__ A, const float* __restrict__ B,
                                                       float* __restrict__ C, int M, int N, int K, long lda, long ldb,
                                                       long strideA, long strideB, long strideC, float alpha,
                                                       int tiles_m, int tiles_n, int k_split, float* __restrict__ part,
                                                       const float* __restrict__ bias, int accum, GemmGroup grp,
                                                       RowSums rs = {})
{
    static_assert(!RSUM || (GRP && !TA), "row sums of an untransposed A in grouped launches");
    static_assert(!SEG || (!GUARD && !STATS), "operands by sequence in whole tiles only");
    constexpr int NT = 64 * WM * WN;
    constexpr int BM = 32 * FM * WM, BN = 32 * FN * WN;
    constexpr int LA = BM * BK / 4 / NT;   // float4 per thread per stage for A
    constexpr int LB = BN * BK / 4 / NT;
    static_assert(LA * 4 * NT == BM * BK && LB * 4 * NT == BN * BK, "tile not divisible by the workgroup");
    // An A contiguous in k (untransposed) is staged as it lies, [m][k] (one
    // 16-byte LDS write per float4); a transposed A and B are staged k-major.
    // Within a stage the MFMA steps take k in the order k = 8 * (lane / 32) +
    // step, so a lane's eight k of one row of A are adjacent (two 16-byte LDS
    // reads); B uses the same order. Measured on the GPT-step products (d 768,
    // 8192 tokens): NN 101 -> 105 and 113 -> 117 TFLOP/s; staging a transposed
    // B as [n][k] as well was 3-5 % slower on the weight-gradient (NT) products.
    constexpr bool AK = !TA;
    constexpr int KROW = BK + 4;   // [m][k] row stride: 8 rows cover all 32 banks
    constexpr int A_R = AK ? BM : BK, A_C = AK ? KROW : BM + PAD;
    __shared__ __attribute__((aligned(16))) float As[2][A_R][A_C];
    __shared__ __attribute__((aligned(16))) float Bs[2][BK][BN + PAD];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    int tmi, tni;
    tile_coords(blockIdx.x, tiles_m * tiles_n, tiles_m, tiles_n, tmi, tni);
    const int m0 = tmi * BM, n0 = tni * BN;
    const long bz = blockIdx.z;
    if constexpr (GRP)
    {
        const int gi = static_cast<int>(bz / grp.nb);
        const long bb = bz % grp.nb;
        A = grp.A[gi];
        B = (grp.B[gi] ? grp.B[gi] : B) + bb * strideB;
        C = grp.C[gi] + bb * strideC;
        bias = grp.bias[gi];
    }
    else
    {
        A += bz * strideA;
        B += bz * strideB;
        C += bz * strideC;
    }
    // Split-K: workgroup row y covers k in [y*k_split, min(K, (y+1)*k_split)) and,
    // when there are several, writes its partial tile to part[y][batch][M][N].
    const int k_lo = blockIdx.y * k_split;
    const int k_hi = min(K, k_lo + k_split);
    if (!STATS && gridDim.y > 1) C = part + ((long)blockIdx.y * gridDim.z + bz) * strideC;
    // SEG: the member's sequence layouts (extra offset per sequence: step - T)
    int sa_t = 0, sb_t = 0;
    long sa_d = 0, sb_d = 0, b_off = 0;
    if constexpr (SEG)
    {
        const int gi = GRP ? static_cast<int>(bz / grp.nb) : 0;
        sa_t = grp.aT[gi];
        sb_t = grp.bT[gi];
        sa_d = grp.aS[gi] - sa_t;
        sb_d = grp.bS[gi] - sb_t;
        if (sa_t) lda = sa_t;   // rows of a sequence-stored operand are T apart
        if (sb_t) ldb = sb_t;
        if (!TB && sb_t) b_off = (long)(n0 / sb_t) * sb_d;
    }

    f4 ra[LA], rb[LB];   // native vectors: HIP's float4 struct kept these arrays in scratch

    // KSEG: the operands of the segment holding stage k0 (a stage never
    // straddles two: klen % BK == 0), addressed with k within the segment.
    auto seg_of = [&](int k0, const float* const* ops, const float* whole, int& kb) {
        if constexpr (KSEG)
        {
            const int sg = k0 / grp.klen;
            kb = k0 - sg * grp.klen;
            return ops[sg];
        }
        kb = k0;
        return whole;
    };
    // A_eff(m, k) = TA ? A[k*lda + m] : A[m*lda + k]
    auto load_a = [&](int k0) {
        int kb;
        const float* Ap = seg_of(k0, grp.A, A, kb);
        if constexpr (SEG && !TA)
            if (sa_t) Ap += (long)(kb / sa_t) * sa_d;
#pragma unroll
        for (int s = 0; s < LA; ++s)
        {
            const int idx = tid + NT * s;
            int m, k;
            if constexpr (TA) { k = idx / (BM / 4); m = (idx % (BM / 4)) * 4; }
            else { m = idx / (BK / 4); k = (idx % (BK / 4)) * 4; }
            const int gm = m0 + m, gk = kb + k, dk = k0 - kb;   // gk + dk: k over the whole sum
            if constexpr (!GUARD)
            {
                ra[s] = TA ? *reinterpret_cast<const f4*>(Ap + (long)gk * lda + gm)
                           : *reinterpret_cast<const f4*>(Ap + (long)gm * lda + gk);
            }
            else
            {
                float v[4];
#pragma unroll
                for (int q = 0; q < 4; ++q)
                {
                    const int mm = TA ? gm + q : gm, kk = TA ? gk : gk + q;
                    v[q] = (mm < M && kk + dk < k_hi) ? (TA ? Ap[(long)kk * lda + mm] : Ap[(long)mm * lda + kk])
                                                       : 0.0f;
                }
                ra[s] = f4{v[0], v[1], v[2], v[3]};
            }
        }
    };
    // B_eff(k, n) = TB ? B[n*ldb + k] : B[k*ldb + n]
    auto load_b = [&](int k0) {
        int kb;
        const float* Bp = seg_of(k0, grp.B, B, kb);
        if constexpr (SEG)
        {
            if (!TB) Bp += b_off;
            else if (sb_t) Bp += (long)(kb / sb_t) * sb_d;
        }
#pragma unroll
        for (int s = 0; s < LB; ++s)
        {
            const int idx = tid + NT * s;
            int n, k;
            if constexpr (!TB) { k = idx / (BN / 4); n = (idx % (BN / 4)) * 4; }
            else { n = idx / (BK / 4); k = (idx % (BK / 4)) * 4; }
            const int gn = n0 + n, gk = kb + k, dk = k0 - kb;
            if constexpr (!GUARD)
            {
                rb[s] = !TB ? *reinterpret_cast<const f4*>(Bp + (long)gk * ldb + gn)
                            : *reinterpret_cast<const f4*>(Bp + (long)gn * ldb + gk);
            }
            else
            {
                float v[4];
#pragma unroll
                for (int q = 0; q < 4; ++q)
                {
                    const int nn = !TB ? gn + q : gn, kk = !TB ? gk : gk + q;
                    v[q] = (nn < N && kk + dk < k_hi) ? (!TB ? Bp[(long)kk * ldb + nn] : Bp[(long)nn * ldb + kk])
                                                       : 0.0f;
                }
                rb[s] = f4{v[0], v[1], v[2], v[3]};
            }
        }
    };
    float racc[RSUM ? LA : 1] = {};
    const bool rsum_here = RSUM && tni == 0;
    auto store_a = [&](int buf) {
        if constexpr (RSUM)
            if (rsum_here)
            {
#pragma unroll
                for (int s = 0; s < LA; ++s) racc[s] += (ra[s].x + ra[s].y) + (ra[s].z + ra[s].w);
            }
#pragma unroll
        for (int s = 0; s < LA; ++s)
        {
            const int idx = tid + NT * s;
            if constexpr (TA)
            {
                const int k = idx / (BM / 4), m = (idx % (BM / 4)) * 4;
                *reinterpret_cast<f4*>(&As[buf][k][m]) = ra[s];
            }
            else
            {
                const int m = idx / (BK / 4), k = (idx % (BK / 4)) * 4;
                *reinterpret_cast<f4*>(&As[buf][m][k]) = ra[s];
            }
        }
    };
    auto store_b = [&](int buf) {
#pragma unroll
        for (int s = 0; s < LB; ++s)
        {
            const int idx = tid + NT * s;
            if constexpr (!TB)
            {
                const int k = idx / (BN / 4), n = (idx % (BN / 4)) * 4;
                *reinterpret_cast<f4*>(&Bs[buf][k][n]) = rb[s];
            }
            else
            {
                const int n = idx / (BK / 4), k = (idx % (BK / 4)) * 4;
                Bs[buf][k + 0][n] = rb[s].x;
                Bs[buf][k + 1][n] = rb[s].y;
                Bs[buf][k + 2][n] = rb[s].z;
                Bs[buf][k + 3][n] = rb[s].w;
            }
        }
    };

    floatx16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    const int kt_n = (k_hi - k_lo + BK - 1) / BK;
    if (kt_n > 0)
    {
        load_a(k_lo);
        load_b(k_lo);
        store_a(0);
        store_b(0);
        __syncthreads();
    }
    const int am = wm * 32 * FM + (lane & 31), bn = wn * 32 * FN + (lane & 31), kl = lane >> 5;
    for (int kt = 0; kt < kt_n; ++kt)
    {
        const int buf = kt & 1;
        const bool more = kt + 1 < kt_n;
        if (more)
        {
            load_a(k_lo + (kt + 1) * BK);
            load_b(k_lo + (kt + 1) * BK);
        }
        static_assert(BK == 16, "k order assumes 8 MFMA steps per stage");
#pragma unroll
        for (int kk = 0; kk < 8; ++kk)
        {
            const int k = 8 * kl + kk;
            float a[FM], b[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i) a[i] = AK ? As[buf][am + 32 * i][k] : As[buf][k][am + 32 * i];
#pragma unroll
            for (int j = 0; j < FN; ++j) b[j] = Bs[buf][k][bn + 32 * j];
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        if (more)
        {
            store_a(buf ^ 1);
            store_b(buf ^ 1);
        }
        __syncthreads();
    }

    // Epilogue: C = alpha * acc, then + bias[row] and / or + C (each rounded
    // as the separate broadcast / add call would round it); a split-K partial
    // is written unscaled and the reduce applies all of that.
    const int col_l = lane & 31, row_l = 4 * (lane >> 5);
    const bool plain = STATS || gridDim.y > 1 || (!bias && !accum);
    if constexpr (STATS)
    {
        // acc becomes C as stored (alpha * acc, + bias[row] rounded as the
        // separate add); the stores below then write it unchanged.
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r)
            {
                const int gm = m0 + wm * 32 * FM + i * 32 + 8 * (r / 4) + row_l + (r % 4);
                const float bv = (bias && (!GUARD || gm < M)) ? bias[gm] : 0.0f;
#pragma unroll
                for (int j = 0; j < FN; ++j)
                {
#pragma clang fp contract(off)
                    float v = alpha * acc[i][j][r];
                    if (bias) v = v + bv;
                    acc[i][j][r] = v;
                }
            }
        float* sm = &Bs[0][0][0];    // [WM][BN] maxima, then [WM][BN] sums (the stages are done)
        float* ss = sm + WM * BN;
#pragma unroll
        for (int j = 0; j < FN; ++j)
        {
            float mx = -__builtin_huge_valf();
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                {
                    const int gm = m0 + wm * 32 * FM + i * 32 + 8 * (r / 4) + row_l + (r % 4);
                    if (!GUARD || gm < M) mx = fmaxf(mx, acc[i][j][r]);
                }
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));   // lanes l and l ^ 32 hold one column's other rows
            float sum = 0.0f;
            if (mx > -__builtin_huge_valf())
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                    {
                        const int gm = m0 + wm * 32 * FM + i * 32 + 8 * (r / 4) + row_l + (r % 4);
                        if (!GUARD || gm < M) sum += __expf(acc[i][j][r] - mx);
                    }
            sum += __shfl_xor(sum, 32, 64);
            if (lane < 32)
            {
                sm[wm * BN + wn * 32 * FN + j * 32 + col_l] = mx;
                ss[wm * BN + wn * 32 * FN + j * 32 + col_l] = sum;
            }
        }
        __syncthreads();
        for (int c = tid; c < BN; c += NT)
        {
            const int gn = n0 + c;
            if (GUARD && gn >= N) continue;
            float m = sm[c], t = ss[c];
            for (int w = 1; w < WM; ++w)   // merge the waves' row bands in row order
            {
                const float m2 = sm[w * BN + c], t2 = ss[w * BN + c];
                if (m2 > m)
                {
                    t = t * __expf(m - m2) + t2;
                    m = m2;
                }
                else if (m2 > -__builtin_huge_valf())
                    t = t + t2 * __expf(m2 - m);
            }
            part[(long)tmi * N + gn] = m;
            part[(long)(tiles_m + tmi) * N + gn] = t;
        }
    }
    // Global loads and stores share one in-order counter, so a bias load
    // issued after a store would wait for the store as well: the tile's BM
    // bias values are staged in LDS (free after the last stage's barrier) and
    // read from there.
    const float* bsh = nullptr;
    if (!plain && bias)
    {
        float* bl = &As[0][0][0];
        for (int m = tid; m < BM; m += NT) bl[m] = (!GUARD || m0 + m < M) ? bias[m0 + m] : 0.0f;
        __syncthreads();
        bsh = bl;
    }
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
        {
            const int gn = n0 + wn * 32 * FN + j * 32 + col_l;
#pragma unroll
            for (int r = 0; r < 16; ++r)
            {
                const int ml = wm * 32 * FM + i * 32 + 8 * (r / 4) + row_l + (r % 4), gm = m0 + ml;
                if (GUARD && !(gm < M && gn < N)) continue;
                float* c = C + (long)gm * N + gn;
                if (plain)
                {
                    *c = STATS ? acc[i][j][r] : (gridDim.y > 1 ? 1.0f : alpha) * acc[i][j][r];
                    continue;
                }
                {
#pragma clang fp contract(off)
                    float v = alpha * acc[i][j][r];
                    if (bias) v = v + bsh[ml];
                    if (accum) v = *c + v;
                    *c = v;
                }
            }
        }
    if constexpr (RSUM)
        if (rsum_here)
        {
            // the BK / 4 threads that stage one row's float4s of a stage are adjacent lanes
            static_assert(BK / 4 == 4 && NT % 64 == 0, "row-sum lanes");
            const long gi = bz / grp.nb;
#pragma unroll
            for (int s = 0; s < LA; ++s)
            {
                float v = racc[s];
                v += __shfl_xor(v, 1, 64);
                v += __shfl_xor(v, 2, 64);
                const int gm = m0 + (tid + NT * s) / (BK / 4);
                if ((tid & 3) != 0 || gm >= M) continue;
                if (gridDim.y > 1)
                    rs.part[((long)blockIdx.y * gridDim.z + bz) * M + gm] = v;
                else
                {
#pragma clang fp contract(off)
                    float* d = rs.dst[gi] + gm;
                    *d = rs.acc ? *d + v : v;
                }
            }
        }
}

// C = alpha * sum_s part[s], summed in split order (deterministic); then
// + bias[row] (rows of N) and / or + C when given, rounded as the separate calls.
__global__ __launch_bounds__(256) void k_splitk_reduce_ep(const float* __restrict__ part, float* __restrict__ C,
                                                          long n, int splits, float alpha, const float* bias, long N,
                                                          int accum, int vec)
{
#pragma clang fp contract(off)
    const long stride = (long)gridDim.x * 256;
    if (vec)
    {
        // N % 4 == 0 and C 16-byte aligned: four consecutive elements share a row.
        const long n4 = n / 4;
        const float4* p4 = reinterpret_cast<const float4*>(part);
        float4* c4 = reinterpret_cast<float4*>(C);
        for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n4; i += stride)
        {
            float4 a = p4[i];
            for (int s = 1; s < splits; ++s)
            {
                const float4 b = p4[(long)s * n4 + i];
                a.x += b.x;
                a.y += b.y;
                a.z += b.z;
                a.w += b.w;
            }
            float4 v = make_float4(alpha * a.x, alpha * a.y, alpha * a.z, alpha * a.w);
            if (bias)
            {
                const float bv = bias[(4 * i) / N];
                v = make_float4(v.x + bv, v.y + bv, v.z + bv, v.w + bv);
            }
            if (accum)
            {
                const float4 c = c4[i];
                v = make_float4(c.x + v.x, c.y + v.y, c.z + v.z, c.w + v.w);
            }
            c4[i] = v;
        }
        return;
    }
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += stride)
    {
        float a = part[i];
        for (int s = 1; s < splits; ++s) a += part[(long)s * n + i];
        float v = alpha * a;
        if (bias) v = v + bias[i / N];
        if (accum) v = C[i] + v;
        C[i] = v;
    }
}

// The split-K partials of a grouped launch (members of mn elements each,
// part[s][member][mn]) into each member's C: C_i = alpha * sum_s part (+ C_i
// when accum), summed in split order; mn % 4 == 0, every C_i 16-byte aligned.
__global__ __launch_bounds__(256) void k_splitk_reduce_grp(const float* __restrict__ part, GemmGroup g, long mn,
                                                           int members, int splits, float alpha, int accum, RowSums rs,
                                                           int M)
{
#pragma clang fp contract(off)
    const long n4 = (long)members * mn / 4, stride = (long)gridDim.x * 256;
    if (rs.part)
    {
        // the row sums (RowSums), summed in slice order
        const long rows = (long)members * M;
        for (long r = (long)blockIdx.x * 256 + threadIdx.x; r < rows; r += stride)
        {
            float a = rs.part[r];
            for (int s = 1; s < splits; ++s) a += rs.part[(long)s * rows + r];
            const long mi = r / M;
            float* d = rs.dst[mi] + (r - mi * M);
            *d = rs.acc ? *d + a : a;
        }
    }
    const float4* p4 = reinterpret_cast<const float4*>(part);
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n4; i += stride)
    {
        float4 a = p4[i];
        for (int s = 1; s < splits; ++s)
        {
            const float4 b = p4[(long)s * n4 + i];
            a.x += b.x;
            a.y += b.y;
            a.z += b.z;
            a.w += b.w;
        }
        const long e = 4 * i, mi = e / mn;
        float4* c = reinterpret_cast<float4*>(g.C[mi] + (e - mi * mn));
        float4 v = make_float4(alpha * a.x, alpha * a.y, alpha * a.z, alpha * a.w);
        if (accum)
        {
            const float4 o = *c;
            v = make_float4(o.x + v.x, o.y + v.y, o.z + v.z, o.w + v.w);
        }
        *c = v;
    }
}

// C = alpha * sum_s part[s], summed in split order (deterministic).
__global__ __launch_bounds__(256) void k_splitk_reduce(const float* __restrict__ part, float* __restrict__ C,
                                                       long n, int splits, float alpha, int vec)
{
    const long stride = (long)gridDim.x * 256;
    if (vec)
    {
        const long n4 = n / 4;
        const float4* p4 = reinterpret_cast<const float4*>(part);
        for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n4; i += stride)
        {
            float4 a = p4[i];
            for (int s = 1; s < splits; ++s)
            {
                const float4 b = p4[(long)s * n4 + i];
                a.x += b.x;
                a.y += b.y;
                a.z += b.z;
                a.w += b.w;
            }
            reinterpret_cast<float4*>(C)[i] = make_float4(alpha * a.x, alpha * a.y, alpha * a.z, alpha * a.w);
        }
    }
    else
    {
        for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += stride)
        {
            float a = part[i];
            for (int s = 1; s < splits; ++s) a += part[(long)s * n + i];
            C[i] = alpha * a;
        }
    }
}

// Launch plan for one GEMM: tile configuration and split-K factor.
enum Cfg { kTall, kSquare, kSkinnyN, kThinWaves, kThinWavesM64 };
struct Plan
{
    Cfg cfg;
    int bm, bn, splits, k_split;
};

// Tile choice, from sweeps of the config-3 and config-4 shapes on MI355X.
// The work is balanced over the 1024 SIMDs first: a 768 x 8192 output makes
// only 192 tiles of 256 x 128, and any tiling with 64 x 64 per wave leaves
// either idle CUs or 1.5 waves per SIMD; 32 x 64 per wave (128 x 64 tiles of
// 4 waves: 768 workgroups, 3 waves on every SIMD) took those products from
// 69-80 to 87-98 TF/s and the 64-row attention products from 48-61 to 70-85.
//   * M <= 64: 64 x 128 tiles of 4 waves with 32 x 64 each;
//   * N <= 64: 256 x 64;
//   * at least 512 tiles of 256 x 128: 256 x 128 over 8 waves;
//   * K >= 4096 with a workspace: 256 x 128 (128 x 128 below 128 tiles) with
//     K split into slices (weight gradients, K = tokens: measured faster than
//     the thin tiles there);
//   * otherwise 128 x 64 tiles of 4 waves with 32 x 64 each, K split when the
//     grid is small and K >= 1024.
// Split K: slices of >= 256 k for about three workgroups per CU, partial
// tiles summed in slice order by k_splitk_reduce (deterministic).
Plan plan_gemm(size_t M, size_t N, size_t K, size_t batch, bool allow_split)
{
    Plan p;
    p.splits = 1;
    p.k_split = static_cast<int>(K);
    auto tiles = [&](int bm, int bn) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn) * batch; };
    auto split = [&](size_t t) {
        size_t want = (768 + t - 1) / t;
        const size_t max_splits = K / 256;
        if (want > max_splits) want = max_splits;
        if (want > 64) want = 64;
        if (want > 1)
        {
            size_t ks = (K + want - 1) / want;
            ks = (ks + 31) / 32 * 32;   // whole BK stages per slice
            p.k_split = static_cast<int>(ks);
            p.splits = static_cast<int>((K + ks - 1) / ks);
        }
    };
    // Mid-sized outputs with K >= 2048: split K so that the workgroups make whole
    // rounds of 3 per CU (768 on MI355X); the first of 256x128, 128x128, 128x64
    // whose split leaves >= 1024 of K per slice (measured on the config-3/4
    // shapes: 6144x768 K8192 NT 110 -> 123, 768x3072 K8192 NT 105 -> 115,
    // 768x8192 K3072 NN 121 -> 124 TFLOP/s; round counts that are not whole lose
    // the fraction).
    if (M > 64 && N > 64 && allow_split && K >= 2048 && tiles(256, 128) < 512)
    {
        const size_t round = 3 * static_cast<size_t>(device_cus());
        const Cfg cs[3] = {kTall, kSquare, kThinWaves};
        const int bms[3] = {256, 128, 128}, bns[3] = {128, 128, 64};
        for (int i = 0; i < 3; ++i)
        {
            const size_t t = tiles(bms[i], bns[i]);
            size_t s = 1;
            while (s <= 64 && (t * s) % round != 0) ++s;
            if (s > 64) continue;
            const size_t ks = ((K + s - 1) / s + 31) / 32 * 32;
            if (ks < 1024) continue;
            p.cfg = cs[i];
            p.bm = bms[i];
            p.bn = bns[i];
            p.k_split = static_cast<int>(ks);
            p.splits = static_cast<int>((K + ks - 1) / ks);
            return p;
        }
    }
    if (M <= 64) { p.cfg = kThinWavesM64; p.bm = 64; p.bn = 128; }
    else if (N <= 64) { p.cfg = kSkinnyN; p.bm = 256; p.bn = 64; }
    else if (tiles(256, 128) >= 512)
    {
        p.cfg = kTall;
        p.bm = 256;
        p.bn = 128;
        // Under 4 resident rounds of 256x128 tiles the last, partial round
        // costs a whole round: take smaller tiles when their whole rounds win
        // clearly (per-tile efficiency 1 : 0.985 : 0.94 measured on the config-3/4
        // shapes; 8192x2304 K768: 576 tiles of 256x128, 94 -> 120 TFLOP/s as
        // 2304 of 128x64). Grids of >= 4 rounds (the lm_head product) keep 256x128.
        const double round = 3.0 * device_cus();
        if (static_cast<double>(tiles(256, 128)) < 4.0 * round)
        {
            auto est = [&](size_t t, double eff) {
                const double r = static_cast<double>(t) / round;
                return r / std::ceil(r) * eff;
            };
            const double eT = est(tiles(256, 128), 1.0), eS = est(tiles(128, 128), 0.985),
                         eN = est(tiles(128, 64), 0.94);
            if (eN > eT + 0.05 && eN >= eS) { p.cfg = kThinWaves; p.bm = 128; p.bn = 64; }
            else if (eS > eT + 0.05) { p.cfg = kSquare; p.bm = 128; p.bn = 128; }
        }
    }
    else if (allow_split && K >= 4096)
    {
        p.cfg = kTall;
        p.bm = 256;
        p.bn = 128;
        if (tiles(128, 128) < 128)
        {
            // Small outputs from long K (the 768 x 768 weight gradients over 8192
            // tokens, alone or as the q, k, v group): 128 x 64 tiles split to
            // about 1728 workgroups (q, k, v group 101 -> 111 TFLOP/s, the single
            // one unchanged at 95-97, against 128 x 128 tiles split to 768).
            p.cfg = kThinWaves;
            p.bm = 128;
            p.bn = 64;
            const size_t t = tiles(128, 64);
            size_t want = (1728 + t - 1) / t;
            if (want > K / 256) want = K / 256;
            if (want > 64) want = 64;
            if (want > 1)
            {
                const size_t ks = ((K + want - 1) / want + 31) / 32 * 32;
                p.k_split = static_cast<int>(ks);
                p.splits = static_cast<int>((K + ks - 1) / ks);
            }
            return p;
        }
        if (tiles(256, 128) < 128)
        {
            p.cfg = kSquare;
            p.bm = 128;
            p.bn = 128;
        }
        split(tiles(p.bm, p.bn));
        return p;
    }
    else { p.cfg = kThinWaves; p.bm = 128; p.bn = 64; }
    const size_t t = tiles(p.bm, p.bn);
    if (allow_split && t < 512 && K >= 1024) split(t);
    return p;
}

struct Epi
{
    const float* bias;                  // per output row, or null
    int accum;                          // C += result
    const GemmGroup* grp = nullptr;     // members of a grouped launch (no split, NN only)
    const GemmGroup* seg = nullptr;     // K segments summed into one C (TN only)
    const RowSums* rs = nullptr;        // grouped launches: the row sums of each member's A as well
    const GemmGroup* sq = nullptr;      // plain launches: member 0 gives the operands' sequence layouts
    bool by_seq = false;                // the group passed (grp, seg or sq) holds sequence layouts
};

template <int WM, int WN, int FM, int FN, int BK, bool TA, bool TB>
void launch_cfg(const float* A, const float* B, float* C, int M, int N, int K, long lda, long ldb, long sA, long sB,
                long sC, float alpha, int batch, bool vec_ok, int splits, int k_split, float* part, hipStream_t s,
                Epi e)
{
    constexpr int BM = 32 * FM * WM, BN = 32 * FN * WN;
    const int tm = (M + BM - 1) / BM, tn = (N + BN - 1) / BN;
    const bool guard = !vec_ok || (M % BM) || (N % BN) || (K % BK) || (k_split % BK);
    const dim3 grid(static_cast<unsigned>(tm * tn), static_cast<unsigned>(splits), static_cast<unsigned>(batch));
    const dim3 block(64 * WM * WN);
    if (e.by_seq)
    {
        if constexpr (TA && !TB)
            if (e.seg && !guard)
                hipLaunchKernelGGL((k_gemm<WM, WN, FM, FN, BK, TA, TB, false, false, false, true, false, true>), grid,
                                   block, 0, s, A, B, C, M, N, K, lda, ldb, sA, sB, sC, alpha, tm, tn, k_split, part,
                                   e.bias, e.accum, *e.seg);
        if constexpr (!TA && TB)
            if (e.grp && !guard)
            {
                if (e.rs)
                    hipLaunchKernelGGL((k_gemm<WM, WN, FM, FN, BK, TA, TB, false, false, true, false, true, true>), grid,
                                       block, 0, s, A, B, C, M, N, K, lda, ldb, sA, sB, sC, alpha, tm, tn, k_split,
                                       part, e.bias, e.accum, *e.grp, *e.rs);
                else
                    hipLaunchKernelGGL((k_gemm<WM, WN, FM, FN, BK, TA, TB, false, false, true, false, false, true>),
                                       grid, block, 0, s, A, B, C, M, N, K, lda, ldb, sA, sB, sC, alpha, tm, tn, k_split,
                                       part, e.bias, e.accum, *e.grp, RowSums{});
            }
        if constexpr (!TA && !TB)
            if (e.sq && !guard)
                hipLaunchKernelGGL((k_gemm<WM, WN, FM, FN, BK, TA, TB, false, false, false, false, false, true>), grid,
                                   block, 0, s, A, B, C, M, N, K, lda, ldb, sA, sB, sC, alpha, tm, tn, k_split, part,
                                   e.bias, e.accum, *e.sq, RowSums{});
        return;
    }
    if constexpr (TA && !TB)
        if (e.seg)
        {
            if (guard)
                hipLaunchKernelGGL((k_gemm<WM, WN, FM, FN, BK, TA, TB, true, false, false, true>), grid, block, 0, s, A,
                                   B, C, M, N, K, lda, ldb, sA, sB, sC, alpha, tm, tn, k_split, part, e.bias, e.accum,
                                   *e.seg);
            else
                hipLaunchKernelGGL((k_gemm<WM, WN, FM, FN, BK, TA, TB, false, false, false, true>), grid, block, 0, s,
                                   A, B, C, M, N, K, lda, ldb, sA, sB, sC, alpha, tm, tn, k_split, part, e.bias,
                                   e.accum, *e.seg);
            return;
        }
    if constexpr (!TA)
        if (e.grp && e.rs)
        {
            if (guard)
                hipLaunchKernelGGL((k_gemm<WM, WN, FM, FN, BK, TA, TB, true, false, true, false, true>), grid, block, 0,
                                   s, A, B, C, M, N, K, lda, ldb, sA, sB, sC, alpha, tm, tn, k_split, part, e.bias,
                                   e.accum, *e.grp, *e.rs);
            else
                hipLaunchKernelGGL((k_gemm<WM, WN, FM, FN, BK, TA, TB, false, false, true, false, true>), grid, block,
                                   0, s, A, B, C, M, N, K, lda, ldb, sA, sB, sC, alpha, tm, tn, k_split, part, e.bias,
                                   e.accum, *e.grp, *e.rs);
            return;
        }
    if constexpr (!TA)
        if (e.grp)
        {
            if (guard)
                hipLaunchKernelGGL((k_gemm<WM, WN, FM, FN, BK, TA, TB, true, false, true>), grid, block, 0, s, A, B, C,
                                   M, N, K, lda, ldb, sA, sB, sC, alpha, tm, tn, k_split, part, e.bias, e.accum,
                                   *e.grp);
            else
                hipLaunchKernelGGL((k_gemm<WM, WN, FM, FN, BK, TA, TB, false, false, true>), grid, block, 0, s, A, B,
                                   C, M, N, K, lda, ldb, sA, sB, sC, alpha, tm, tn, k_split, part, e.bias, e.accum,
                                   *e.grp);
            return;
        }
    if (guard)
        hipLaunchKernelGGL((k_gemm<WM, WN, FM, FN, BK, TA, TB, true>), grid, block, 0, s, A, B, C, M, N, K, lda, ldb,
                           sA, sB, sC, alpha, tm, tn, k_split, part, e.bias, e.accum, GemmGroup{});
    else
        hipLaunchKernelGGL((k_gemm<WM, WN, FM, FN, BK, TA, TB, false>), grid, block, 0, s, A, B, C, M, N, K, lda, ldb,
                           sA, sB, sC, alpha, tm, tn, k_split, part, e.bias, e.accum, GemmGroup{});
}

template <bool TA, bool TB>
void launch_trans(const Plan& p, const float* A, const float* B, float* C, int M, int N, int K, long lda, long ldb,
                  long sA, long sB, long sC, float alpha, int batch, float* part, hipStream_t s, Epi e)
{
    const bool vec_ok = (lda % 4 == 0) && (ldb % 4 == 0) && (sA % 4 == 0) && (sB % 4 == 0) && aligned16(A) &&
                        aligned16(B);
    switch (p.cfg)
    {
    case kSkinnyN:
        launch_cfg<4, 1, 2, 2, 16, TA, TB>(A, B, C, M, N, K, lda, ldb, sA, sB, sC, alpha, batch, vec_ok, p.splits,
                                           p.k_split, part, s, e);
        break;
    case kThinWaves:
        launch_cfg<4, 1, 1, 2, 16, TA, TB>(A, B, C, M, N, K, lda, ldb, sA, sB, sC, alpha, batch, vec_ok, p.splits,
                                           p.k_split, part, s, e);
        break;
    case kThinWavesM64:
        launch_cfg<2, 2, 1, 2, 16, TA, TB>(A, B, C, M, N, K, lda, ldb, sA, sB, sC, alpha, batch, vec_ok, p.splits,
                                           p.k_split, part, s, e);
        break;
    case kTall:
        launch_cfg<4, 2, 2, 2, 16, TA, TB>(A, B, C, M, N, K, lda, ldb, sA, sB, sC, alpha, batch, vec_ok, p.splits,
                                           p.k_split, part, s, e);
        break;
    default:
        launch_cfg<2, 2, 2, 2, 16, TA, TB>(A, B, C, M, N, K, lda, ldb, sA, sB, sC, alpha, batch, vec_ok, p.splits,
                                           p.k_split, part, s, e);
        break;
    }
}

// ── matrix-vector products (N == 1 or M == 1) ───────────────────────────────
// Memory-bound: each matrix element is read once, so these bypass the MFMA
// tiles (a 64-wide tile would waste 63/64 of its work). The epilogue rounds as
// the split-K reduction does: v = alpha * sum, v += bias, v = C_old + v.
__device__ __forceinline__ float gemv_epilogue(float acc, float alpha, const float* bias, long brow, const float* y,
                                               int accum)
{
#pragma clang fp contract(off)
    float v = alpha * acc;
    if (bias) v = v + bias[brow];
    if (accum) v = *y + v;
    return v;
}

// y[i] = alpha * sum_k R[i][k] x[k] over rows of R (row stride ldr): one wave per output.
// A row is short (a few KB) and each wave reads one, so the time is the memory
// latency: a lane issues all its loads of up to U float4 pairs (K <= 256 U)
// before the first multiply, and adds them in the order of k (lane q holds
// float4 q, q + 64, ...; the wave then sums the lanes). U is the smallest of
// 4, 8, 16 that covers K, to keep the registers (and so the waves resident
// per SIMD) for many-row products such as the LM head.
template <bool VEC, int U>
__device__ __forceinline__ float gemv_row(const float* r, const float* xv, int K, unsigned lane)
{
    float acc = 0.0f;
    int k = 0;
    if constexpr (VEC)
    {
        const float4* r4 = reinterpret_cast<const float4*>(r);
        const float4* x4 = reinterpret_cast<const float4*>(xv);
        const int K4 = K / 4;
        for (int q0 = static_cast<int>(lane); q0 < K4; q0 += 64 * U)
        {
            float4 a[U], v[U];
#pragma unroll
            for (int u = 0; u < U; ++u)
                if (q0 + 64 * u < K4)
                {
                    a[u] = r4[q0 + 64 * u];
                    v[u] = x4[q0 + 64 * u];
                }
#pragma unroll
            for (int u = 0; u < U; ++u)
                if (q0 + 64 * u < K4)
                {
                    acc = __builtin_fmaf(a[u].x, v[u].x, acc);
                    acc = __builtin_fmaf(a[u].y, v[u].y, acc);
                    acc = __builtin_fmaf(a[u].z, v[u].z, acc);
                    acc = __builtin_fmaf(a[u].w, v[u].w, acc);
                }
        }
        k = 4 * K4;
    }
    for (int kk = k + static_cast<int>(lane); kk < K; kk += 64) acc = __builtin_fmaf(r[kk], xv[kk], acc);
    return wave_sum(acc);
}

template <bool VEC, int U>
__global__ __launch_bounds__(256) void k_gemv_rows(const float* __restrict__ R, long ldr, long sR,
                                                   const float* __restrict__ x, long sx, float* y, long sy, int rows,
                                                   int K, float alpha, const float* bias, int bias_each, int accum)
{
    const unsigned lane = threadIdx.x % 64, wave = threadIdx.x / 64;
    const int i = blockIdx.x * 4 + static_cast<int>(wave);
    if (i >= rows) return;
    const long b = blockIdx.y;
    const float acc = gemv_row<VEC, U>(R + b * sR + (long)i * ldr, x + b * sx, K, lane);
    if (lane == 0)
    {
        float* out = y + b * sy + i;
        *out = gemv_epilogue(acc, alpha, bias, bias_each ? i : 0, out, accum);
    }
}

// Up to four such products of one vector x (the attention's q, k and v
// projections of one token): member blockIdx.y, R_i (rows, K) row-major.
// Member m writes v = R_m x (+ bias) to y[m] (when set) and to out[m] (when
// set; plus add[m], when set: the residual add x_new + v that follows a
// projection, or a copy of v into a KV-cache row).
struct GemvGroup
{
    const float* R[4];
    const float* bias[4];
    float* y[4];
    const float* add[4];
    float* out[4];
};
// RMS: x is first normalised as RMSNorm::forward's six calls on a (K, 1)
// column do it (the narrow kernel of nnhip_rmsnorm_forward: the same sums in
// the same order, so the same bits): y = x / sqrt(sum(x^2) inv_f + eps) *
// gamma, into LDS for the products; workgroup (0, 0) also stores the
// RMSNorm outputs that are asked for.
//
// A launch is a few memory latencies long, so every load that does not depend
// on another is issued before the first wait: the epilogue's bias and
// residual, and with RMS (VEC, K <= 1024: one float4 trip per lane, U = 4)
// x and gamma first, then the rows. Waits on the vector-memory counter are in
// issue order, so the prologue waits for x and gamma only while the rows'
// loads stay in flight.
struct RmsLoads
{
    float v[4], gm[4];
};
__device__ __forceinline__ void rms_load(const float* __restrict__ x, const float* __restrict__ gamma, int K,
                                         RmsLoads& r)
{
    const unsigned t = threadIdx.x;
#pragma unroll
    for (unsigned k = 0; k < 4; ++k)
    {
        const unsigned i = t + k * 256;
        r.v[k] = i < static_cast<unsigned>(K) ? x[i] : 0.0f;
        r.gm[k] = i < static_cast<unsigned>(K) ? gamma[i] : 0.0f;
    }
}
// The normalised vector into xs (LDS, K <= 1024 floats); ends with a barrier.
__device__ __forceinline__ void rms_finish(const RmsLoads& r, int K, const nnhip_gemv_rmsnorm& rn, float* xs,
                                           float* part, bool first)
{
    const unsigned t = threadIdx.x, lane = t % 64, wave = t / 64;
    float ss = 0.0f;
#pragma unroll
    for (unsigned k = 0; k < 4; ++k)
        if (t + k * 256 < static_cast<unsigned>(K)) ss = __builtin_fmaf(r.v[k], r.v[k], ss);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
    if (lane == 0) part[wave] = ss;
    __syncthreads();
    float sum = part[0];
#pragma unroll
    for (unsigned w = 1; w < 4; ++w) sum += part[w];
    float ri;
    {
#pragma clang fp contract(off)
        const float sc = sum * rn.inv_f, ve = sc + rn.eps;
        ri = 1.0f / sqrtf(ve);
        if (first && t == 0)
        {
            if (rn.s_raw) rn.s_raw[0] = sum;
            if (rn.scaled) rn.scaled[0] = sc;
            if (rn.var_eps) rn.var_eps[0] = ve;
            if (rn.rinv) rn.rinv[0] = ri;
        }
    }
#pragma unroll
    for (unsigned k = 0; k < 4; ++k)
    {
        const unsigned i = t + k * 256;
        if (i < static_cast<unsigned>(K))
        {
#pragma clang fp contract(off)
            const float n = r.v[k] * ri, y = n * r.gm[k];
            xs[i] = y;
            if (first)
            {
                if (rn.normed) rn.normed[i] = n;
                if (rn.out) rn.out[i] = y;
            }
        }
    }
    __syncthreads();
}
// One row's float4s for the RMS path's single trip (lane + 64 u, u < 4).
__device__ __forceinline__ void row_load4(const float* __restrict__ row, int K4, unsigned lane, bool live, float4* a)
{
    const float4* r4 = reinterpret_cast<const float4*>(row);
#pragma unroll
    for (int u = 0; u < 4; ++u)
        if (live && static_cast<int>(lane) + 64 * u < K4) a[u] = r4[lane + 64 * u];
}
// gemv_row's sums for that trip: float4 lane + 64 u in the order of u, then the wave's sum.
__device__ __forceinline__ float row_dot4(const float4* a, const float* xs, int K4, unsigned lane)
{
    const float4* x4 = reinterpret_cast<const float4*>(xs);
    float d = 0.0f;
#pragma unroll
    for (int u = 0; u < 4; ++u)
        if (static_cast<int>(lane) + 64 * u < K4)
        {
            const float4 xv4 = x4[lane + 64 * u];
            d = __builtin_fmaf(a[u].x, xv4.x, d);
            d = __builtin_fmaf(a[u].y, xv4.y, d);
            d = __builtin_fmaf(a[u].z, xv4.z, d);
            d = __builtin_fmaf(a[u].w, xv4.w, d);
        }
    return wave_sum(d);
}

template <bool VEC, int U, bool RMS>
__global__ __launch_bounds__(256) void k_gemv_group(GemvGroup g, const float* __restrict__ x, int rows, int K,
                                                    nnhip_gemv_rmsnorm rn)
{
    const unsigned lane = threadIdx.x % 64, wave = threadIdx.x / 64;
    const int i = blockIdx.x * 4 + static_cast<int>(wave);
    const int m = blockIdx.y;
    const bool live = i < rows;
    const float* bias = g.bias[m];
    const float* add = g.add[m];
    float bv = 0.0f, av = 0.0f;
    if (live && lane == 0)
    {
        if (bias) bv = bias[i];
        if (add) av = add[i];
    }
    float acc;
    if constexpr (RMS)
    {
        static_assert(!VEC || U == 4, "the RMS prologue's row covers K <= 1024 in one trip");
        __shared__ __align__(16) float xs[1024];
        __shared__ float part[4];
        RmsLoads rl;
        rms_load(x, rn.gamma, K, rl);
        const int K4 = K / 4;
        float4 a[4];
        if constexpr (VEC) row_load4(g.R[m] + (long)i * K, K4, lane, live, a);
        rms_finish(rl, K, rn, xs, part, blockIdx.x == 0 && blockIdx.y == 0);
        if (!live) return;
        if constexpr (VEC)
            acc = row_dot4(a, xs, K4, lane);
        else
            acc = gemv_row<VEC, U>(g.R[m] + (long)i * K, xs, K, lane);
    }
    else
    {
        if (!live) return;
        acc = gemv_row<VEC, U>(g.R[m] + (long)i * K, x, K, lane);
    }
    if (lane == 0)
    {
#pragma clang fp contract(off)
        float v = 1.0f * acc;
        if (bias) v = v + bv;
        if (g.y[m]) g.y[m][i] = v;
        if (g.out[m]) g.out[m][i] = add ? av + v : v;
    }
}

// A Linear of 2h rows whose output feeds SwiGLU (a token's fc1, then
// SwiGLU::forward's chain on its gate rows [0, h) and up rows [h, 2h)): wave
// i forms rows i and h + i as k_gemv_group does (the same sums, bias added
// the same way; y = both rows when set) and then the chain's values from
// them as k_swiglu_fwd forms them, s = c_div / (exp(-gate) + c_add) (when
// s_out is set) and out = (gate * s) * up. K % 4 == 0, K <= 1024 with RMS.
struct GemvSwiglu
{
    const float* R;
    const float* bias;
    float* y;
    float* s_out;
    float* out;
    int half, K;
    float c_add, c_div;
};
template <bool VEC, int U, bool RMS>
__global__ __launch_bounds__(256) void k_gemv_swiglu(GemvSwiglu g, const float* __restrict__ x, nnhip_gemv_rmsnorm rn)
{
    const unsigned lane = threadIdx.x % 64, wave = threadIdx.x / 64;
    const int i = blockIdx.x * 4 + static_cast<int>(wave);
    const bool live = i < g.half;
    const int K = g.K;
    const float* rg = g.R + (long)i * K;
    const float* ru = g.R + (long)(g.half + i) * K;
    float bg = 0.0f, bu = 0.0f;
    if (live && lane == 0 && g.bias)
    {
        bg = g.bias[i];
        bu = g.bias[g.half + i];
    }
    float accg, accu;
    if constexpr (RMS)
    {
        static_assert(VEC && U == 4, "the RMS prologue's rows cover K <= 1024 in one trip");
        __shared__ __align__(16) float xs[1024];
        __shared__ float part[4];
        RmsLoads rl;
        rms_load(x, rn.gamma, K, rl);
        const int K4 = K / 4;
        float4 a[4], b[4];
        row_load4(rg, K4, lane, live, a);
        row_load4(ru, K4, lane, live, b);
        rms_finish(rl, K, rn, xs, part, blockIdx.x == 0);
        if (!live) return;
        accg = row_dot4(a, xs, K4, lane);
        accu = row_dot4(b, xs, K4, lane);
    }
    else
    {
        if (!live) return;
        accg = gemv_row<VEC, U>(rg, x, K, lane);
        accu = gemv_row<VEC, U>(ru, x, K, lane);
    }
    if (lane == 0)
    {
#pragma clang fp contract(off)
        float vg = 1.0f * accg, vu = 1.0f * accu;
        if (g.bias)
        {
            vg = vg + bg;
            vu = vu + bu;
        }
        if (g.y)
        {
            g.y[i] = vg;
            g.y[g.half + i] = vu;
        }
        const float sv = g.c_div / (expf(-vg) + g.c_add);
        if (g.s_out) g.s_out[i] = sv;
        g.out[i] = (vg * sv) * vu;
    }
}

// y[j] = alpha * sum_k x[k] Q[k][j] over rows of Q (row stride ldq), read along j: one thread per output,
// k in order.
__global__ __launch_bounds__(256) void k_gemv_cols(const float* __restrict__ Q, long ldq, long sQ,
                                                   const float* __restrict__ x, long sx, float* y, long sy, int cols,
                                                   int K, float alpha, const float* bias, int bias_each, int accum)
{
    const int j = blockIdx.x * 256 + threadIdx.x;
    if (j >= cols) return;
    const long b = blockIdx.y;
    const float* q = Q + b * sQ + j;
    const float* xv = x + b * sx;
    float acc = 0.0f;
    int k = 0;
    for (; k + 4 <= K; k += 4)
    {
        const float a0 = q[(long)k * ldq], a1 = q[(long)(k + 1) * ldq], a2 = q[(long)(k + 2) * ldq],
                    a3 = q[(long)(k + 3) * ldq];
        acc = __builtin_fmaf(a0, xv[k], acc);
        acc = __builtin_fmaf(a1, xv[k + 1], acc);
        acc = __builtin_fmaf(a2, xv[k + 2], acc);
        acc = __builtin_fmaf(a3, xv[k + 3], acc);
    }
    for (; k < K; ++k) acc = __builtin_fmaf(q[(long)k * ldq], xv[k], acc);
    float* out = y + b * sy + j;
    *out = gemv_epilogue(acc, alpha, bias, bias_each ? j : 0, out, accum);
}

// Runs C = alpha op(A) op(B) (+ epilogue) as matrix-vector products when N == 1 or M == 1 and the
// layout allows it; returns 1 when launched (0 / error from launch_status via rc), 0 when not handled.
int try_gemv(const float* A, const float* B, float* C, size_t M, size_t N, size_t K, size_t lda, size_t ldb,
             size_t sA, size_t sB, size_t sC, bool tA, bool tB, float alpha, size_t batch, hipStream_t s, Epi e,
             int& rc)
{
    if (K == 0 || K > 0x7fffffff) return 0;
    const float* R = nullptr;   // matrix whose rows the outputs dot with, or whose rows the outputs run along
    const float* x = nullptr;
    long ld = 0, sR = 0, sx = 0;
    size_t outs = 0;
    bool rows = false;
    int bias_each = 0;
    if (N == 1 && M > 1)
    {
        // the vector is B's only column (tB = 0: stride ldb = 1) or row (tB = 1)
        if (!tB && ldb != 1) return 0;
        x = B;
        sx = static_cast<long>(sB);
        R = A;
        ld = static_cast<long>(lda);
        sR = static_cast<long>(sA);
        outs = M;
        rows = !tA;
        bias_each = 1;
    }
    else if (M == 1)
    {
        if (tA && lda != 1) return 0;
        x = A;
        sx = static_cast<long>(sA);
        R = B;
        ld = static_cast<long>(ldb);
        sR = static_cast<long>(sB);
        outs = N;
        rows = tB;
        bias_each = 0;
    }
    else
        return 0;
    if (!rows && K > 4096) return 0;   // the column form runs k serially per output
    if (outs > 0x7fffffff) return 0;
    if (rows)
    {
        const bool vec = ld % 4 == 0 && sR % 4 == 0 && sx % 4 == 0 && aligned16(R) && aligned16(x);
        const dim3 grid(static_cast<unsigned>((outs + 3) / 4), static_cast<unsigned>(batch));
        if (vec && K <= 1024)
            hipLaunchKernelGGL((k_gemv_rows<true, 4>), grid, dim3(256), 0, s, R, ld, sR, x, sx, C, (long)sC,
                               (int)outs, (int)K, alpha, e.bias, bias_each, e.accum);
        else if (vec && K <= 2048)
            hipLaunchKernelGGL((k_gemv_rows<true, 8>), grid, dim3(256), 0, s, R, ld, sR, x, sx, C, (long)sC,
                               (int)outs, (int)K, alpha, e.bias, bias_each, e.accum);
        else if (vec)
            hipLaunchKernelGGL((k_gemv_rows<true, 16>), grid, dim3(256), 0, s, R, ld, sR, x, sx, C, (long)sC,
                               (int)outs, (int)K, alpha, e.bias, bias_each, e.accum);
        else
            hipLaunchKernelGGL((k_gemv_rows<false, 1>), grid, dim3(256), 0, s, R, ld, sR, x, sx, C, (long)sC,
                               (int)outs, (int)K, alpha, e.bias, bias_each, e.accum);
    }
    else
    {
        const dim3 grid(static_cast<unsigned>((outs + 255) / 256), static_cast<unsigned>(batch));
        hipLaunchKernelGGL(k_gemv_cols, grid, dim3(256), 0, s, R, ld, sR, x, sx, C, (long)sC, (int)outs, (int)K,
                           alpha, e.bias, bias_each, e.accum);
    }
    rc = launch_status();
    return 1;
}

int gemm_dispatch(const float* A, const float* B, float* C, size_t M, size_t N, size_t K, size_t lda, size_t ldb,
                  size_t sA, size_t sB, size_t sC, bool tA, bool tB, float alpha, size_t batch, void* workspace,
                  size_t ws_bytes, void* stream, Epi e = {nullptr, 0})
{
    if (M == 0 || N == 0 || batch == 0) return 0;
    if (M > 0x7fffffff || N > 0x7fffffff || K > 0x7fffffff || batch > 65535) return -1;
    if (e.grp && tA) return -1;
    if (e.seg && !(tA && !tB)) return -1;
    if (e.by_seq && !(tA && !tB ? e.seg != nullptr : !tA && tB ? e.grp != nullptr : !tA && !tB && e.sq != nullptr))
        return -1;
    auto s = static_cast<hipStream_t>(stream);
    if (int rc = 0; !e.grp && !e.seg && !e.by_seq &&
                    try_gemv(A, B, C, M, N, K, lda, ldb, sA, sB, sC, tA, tB, alpha, batch, s, e, rc))
        return rc;
    Plan p = plan_gemm(M, N, K, batch, workspace != nullptr);
    if (p.splits > 1 && static_cast<size_t>(p.splits) * batch * (M * N + (e.rs ? M : 0)) * sizeof(float) > ws_bytes)
        p = plan_gemm(M, N, K, batch, false);
    if (e.by_seq)
    {
        // whole tiles, 16-byte loads, and no tile or stage across two sequences
        const GemmGroup& g = e.grp ? *e.grp : e.seg ? *e.seg : *e.sq;
        const bool whole = M % p.bm == 0 && N % p.bn == 0 && K % 16 == 0 && p.k_split % 16 == 0 && lda % 4 == 0 &&
                           ldb % 4 == 0 && sA % 4 == 0 && sB % 4 == 0 && aligned16(A) && aligned16(B);
        if (!whole) return -7;
        const int members = e.grp ? static_cast<int>(batch / g.nb) : 1;
        for (int i = 0; i < members && i < kGroupMax; ++i)
        {
            if (g.aT[i] < 0 || g.bT[i] < 0 || g.aS[i] % 4 != 0 || g.bS[i] % 4 != 0) return -7;
            if (g.aT[i] && (tA || g.aT[i] % 16 != 0 || g.aS[i] < g.aT[i])) return -7;
            if (g.bT[i] && (g.bT[i] % (tB ? 16 : p.bn) != 0 || g.bS[i] < g.bT[i])) return -7;
        }
    }
    float* part = p.splits > 1 ? static_cast<float*>(workspace) : nullptr;
    RowSums rsl{};
    if (e.rs)
    {
        // the row sums' slice partials follow the tiles' in the workspace
        rsl = *e.rs;
        rsl.part = part ? part + static_cast<size_t>(p.splits) * batch * M * N : nullptr;
        e.rs = &rsl;
    }
    const int m = (int)M, n = (int)N, k = (int)K, b = (int)batch;
    if (!tA && !tB) launch_trans<false, false>(p, A, B, C, m, n, k, lda, ldb, sA, sB, sC, alpha, b, part, s, e);
    else if (!tA && tB) launch_trans<false, true>(p, A, B, C, m, n, k, lda, ldb, sA, sB, sC, alpha, b, part, s, e);
    else if (tA && !tB) launch_trans<true, false>(p, A, B, C, m, n, k, lda, ldb, sA, sB, sC, alpha, b, part, s, e);
    else launch_trans<true, true>(p, A, B, C, m, n, k, lda, ldb, sA, sB, sC, alpha, b, part, s, e);
    if (p.splits > 1 && e.grp)
    {
        // grouped members (nb == 1): each member's partials into its own C
        const long mn = (long)M * (long)N;
        hipLaunchKernelGGL(k_splitk_reduce_grp, dim3(grid_for(static_cast<size_t>(batch * mn / 4 + 1), 256, 256 * 16)),
                           dim3(256), 0, s, part, *e.grp, mn, (int)batch, p.splits, alpha, e.accum,
                           e.rs ? *e.rs : RowSums{}, (int)M);
    }
    else if (p.splits > 1)
    {
        const long total = (long)batch * (long)M * (long)N;
        const int vec = aligned16(C) && (e.bias || e.accum ? N % 4 == 0 : total % 4 == 0) ? 1 : 0;
        if (e.bias || e.accum)
            hipLaunchKernelGGL(k_splitk_reduce_ep, dim3(grid_for(static_cast<size_t>(total / 4 + 1), 256, 256 * 16)),
                               dim3(256), 0, s, part, C, total, p.splits, alpha, e.bias, (long)N, e.accum, vec);
        else
            hipLaunchKernelGGL(k_splitk_reduce, dim3(grid_for(static_cast<size_t>(total / 4 + 1), 256, 256 * 16)),
                               dim3(256), 0, s, part, C, total, p.splits, alpha, vec);
    }
    return launch_status();
}

// The product of nnhip_gemm_colstats: 256 x 128 tiles of 8 waves, no split.
constexpr int kStatsBM = 256, kStatsBN = 128;
bool colstats_ok(size_t M, size_t N, size_t K, int tA, int tB)
{
    return !tA && !tB && M > 0 && N > 0 && K > 0 && M <= 0x7fffffff && N <= 0x7fffffff && K <= 0x7fffffff &&
           plan_gemm(M, N, K, 1, false).cfg == kTall;
}

} // namespace
} // namespace nnhip

using namespace nnhip;

extern "C" size_t nnhip_gemm_colstats_tiles(size_t M, size_t N, size_t K, int transA, int transB)
{
    return colstats_ok(M, N, K, transA, transB) ? (M + kStatsBM - 1) / kStatsBM : 0;
}

extern "C" int nnhip_gemm_colstats(const float* A, const float* B, float* C, size_t A_rows, size_t A_cols,
                                   size_t B_rows, size_t B_cols, int transA, int transB, const float* row_bias,
                                   float* stats, void* stream)
{
    const size_t M = transA ? A_cols : A_rows, K = transA ? A_rows : A_cols;
    const size_t K2 = transB ? B_cols : B_rows, N = transB ? B_rows : B_cols;
    if (K != K2) return -2;
    if (!colstats_ok(M, N, K, transA, transB)) return -3;
    if (!A || !B || !C || !stats) return -1;
    const int m = (int)M, n = (int)N, k = (int)K;
    const int tm = (m + kStatsBM - 1) / kStatsBM, tn = (n + kStatsBN - 1) / kStatsBN;
    const bool vec = (A_cols % 4 == 0) && (B_cols % 4 == 0) && aligned16(A) && aligned16(B);
    const bool guard = !vec || (m % kStatsBM) || (n % kStatsBN) || (k % 16);
    const dim3 grid(static_cast<unsigned>(tm * tn), 1, 1), block(512);
    auto s = static_cast<hipStream_t>(stream);
    if (guard)
        hipLaunchKernelGGL((k_gemm<4, 2, 2, 2, 16, false, false, true, true>), grid, block, 0, s, A, B, C, m, n, k,
                           (long)A_cols, (long)B_cols, 0L, 0L, 0L, 1.0f, tm, tn, k, stats, row_bias, 0, GemmGroup{});
    else
        hipLaunchKernelGGL((k_gemm<4, 2, 2, 2, 16, false, false, false, true>), grid, block, 0, s, A, B, C, m, n, k,
                           (long)A_cols, (long)B_cols, 0L, 0L, 0L, 1.0f, tm, tn, k, stats, row_bias, 0, GemmGroup{});
    return launch_status();
}

extern "C" size_t nnhip_gemm_workspace_bytes(size_t M, size_t N, size_t K, size_t batch)
{
    // (split-K partial tiles, and the slices' row sums of nnhip_gemm_group_acc)
    const Plan p = plan_gemm(M, N, K, batch, true);
    return p.splits > 1 ? static_cast<size_t>(p.splits) * batch * (M * N + M) * sizeof(float) : 0;
}

extern "C" int nnhip_gemm(const float* A, const float* B, float* C, size_t A_rows, size_t A_cols, size_t B_rows,
                          size_t B_cols, size_t batch, int transA, int transB, float alpha, void* workspace,
                          size_t workspace_bytes, void* stream)
{
    if (batch == 0 || A_rows % batch || B_rows % batch) return -2;
    const size_t ar = A_rows / batch, br = B_rows / batch;
    const size_t M = transA ? A_cols : ar, K = transA ? ar : A_cols;
    const size_t K2 = transB ? B_cols : br, N = transB ? br : B_cols;
    if (K != K2) return -2;
    return gemm_dispatch(A, B, C, M, N, K, A_cols, B_cols, ar * A_cols, br * B_cols, M * N, transA != 0, transB != 0,
                         alpha, batch, workspace, workspace_bytes, stream);
}

extern "C" int nnhip_gemm_epilogue(const float* A, const float* B, float* C, size_t A_rows, size_t A_cols,
                                   size_t B_rows, size_t B_cols, int transA, int transB, float alpha,
                                   const float* row_bias, int accumulate, void* workspace, size_t workspace_bytes,
                                   void* stream)
{
    const size_t M = transA ? A_cols : A_rows, K = transA ? A_rows : A_cols;
    const size_t K2 = transB ? B_cols : B_rows, N = transB ? B_rows : B_cols;
    if (K != K2) return -2;
    return gemm_dispatch(A, B, C, M, N, K, A_cols, B_cols, A_rows * A_cols, B_rows * B_cols, M * N, transA != 0,
                         transB != 0, alpha, 1, workspace, workspace_bytes, stream, Epi{row_bias, accumulate ? 1 : 0});
}

namespace
{
bool seq_ok(const nnhip_by_seq* q, size_t n)
{
    if (!q) return true;
    for (size_t i = 0; i < n; ++i)
        if (q[i].len > 0x7fffffff || q[i].step > 0x7fffffffffffull) return false;
    return true;
}

// The grouped accumulations: one B for every member (B_each null) or one each,
// members' operands optionally stored by sequence.
int group_acc(const float* const* A, const float* B, const float* const* B_each, float* const* C, size_t count,
              size_t M, size_t N, size_t K, int transB, int accumulate, float* const* row_sums,
              int row_sums_accumulate, void* workspace, size_t workspace_bytes, void* stream,
              const nnhip_by_seq* a_seq = nullptr, const nnhip_by_seq* b_seq = nullptr)
{
    if (!A || !(B || B_each) || !C || count == 0 || count > kGroupMax || M == 0 || N == 0 || K == 0 ||
        (M * N) % 4 != 0 || !seq_ok(a_seq, count) || !seq_ok(b_seq, count))
        return -1;
    GemmGroup g{};
    g.nb = 1;
    RowSums rs{};
    bool by_seq = false;
    for (size_t i = 0; i < count; ++i)
    {
        if (!A[i] || !C[i] || !aligned16(C[i]) || (row_sums && !row_sums[i]) || (B_each && !B_each[i])) return -1;
        g.A[i] = A[i];
        g.C[i] = C[i];
        g.B[i] = B_each ? B_each[i] : nullptr;
        rs.dst[i] = row_sums ? row_sums[i] : nullptr;
        if (a_seq && a_seq[i].len)
        {
            g.aT[i] = static_cast<int>(a_seq[i].len);
            g.aS[i] = static_cast<long>(a_seq[i].step);
            by_seq = true;
        }
        if (b_seq && b_seq[i].len)
        {
            g.bT[i] = static_cast<int>(b_seq[i].len);
            g.bS[i] = static_cast<long>(b_seq[i].step);
            by_seq = true;
        }
        // members' loads are 16-byte loads when member 0's are
        if (!aligned16(A[i]) || (B_each && !aligned16(B_each[i]))) return -1;
    }
    rs.acc = row_sums_accumulate ? 1 : 0;
    // A_i stored (M, K), B (K, N) or, with transB, (N, K); batch z of the launch is member z.
    Epi e{nullptr, accumulate ? 1 : 0};
    e.grp = &g;
    e.by_seq = by_seq;
    if (by_seq && !transB) return -1;
    if (row_sums) e.rs = &rs;
    return gemm_dispatch(A[0], B_each ? B_each[0] : B, C[0], M, N, K, K, transB ? K : N, M * K, 0, M * N, false,
                         transB != 0, 1.0f, count, workspace, workspace_bytes, stream, e);
}
} // namespace

extern "C" int nnhip_gemm_group_acc(const float* const* A, const float* B, float* const* C, size_t count, size_t M,
                                    size_t N, size_t K, int transB, int accumulate, float* const* row_sums,
                                    int row_sums_accumulate, void* workspace, size_t workspace_bytes, void* stream)
{
    return group_acc(A, B, nullptr, C, count, M, N, K, transB, accumulate, row_sums, row_sums_accumulate, workspace,
                     workspace_bytes, stream);
}

extern "C" int nnhip_gemm_group_acc_each(const float* const* A, const float* const* B, float* const* C,
                                         size_t count, size_t M, size_t N, size_t K, int transB, int accumulate,
                                         float* const* row_sums, int row_sums_accumulate, void* workspace,
                                         size_t workspace_bytes, void* stream)
{
    if (!B) return -1;
    return group_acc(A, nullptr, B, C, count, M, N, K, transB, accumulate, row_sums, row_sums_accumulate, workspace,
                     workspace_bytes, stream);
}

extern "C" int nnhip_gemm_group_acc_seq(const float* const* A, const float* const* B, float* const* C, size_t count,
                                        size_t M, size_t N, size_t K, int transB, int accumulate,
                                        float* const* row_sums, int row_sums_accumulate, const nnhip_by_seq* a_seq,
                                        const nnhip_by_seq* b_seq, void* workspace, size_t workspace_bytes,
                                        void* stream)
{
    if (!B) return -1;
    return group_acc(A, nullptr, B, C, count, M, N, K, transB, accumulate, row_sums, row_sums_accumulate, workspace,
                     workspace_bytes, stream, a_seq, b_seq);
}

extern "C" int nnhip_gemm_tn_sum(const float* const* A, const float* const* B, size_t count, float* C, size_t M,
                                 size_t N, size_t K_each, float alpha, void* workspace, size_t workspace_bytes,
                                 void* stream)
{
    if (!A || !B || !C || count == 0 || count > 3 || K_each == 0 || K_each % 16 != 0 || M % 4 != 0 || N % 4 != 0 ||
        count * K_each > 0x7fffffff)
        return -1;
    GemmGroup g{};
    g.klen = static_cast<int>(K_each);
    for (size_t i = 0; i < count; ++i)
    {
        if (!A[i] || !B[i] || !aligned16(A[i]) || !aligned16(B[i])) return -1;
        g.A[i] = A[i];
        g.B[i] = B[i];
    }
    // A_i stored (K_each, M), B_i (K_each, N); the segment pointers come from the group, A[0] and B[0] here
    // only give the launch its shape and alignment checks.
    Epi e{nullptr, 0};
    e.seg = &g;
    return gemm_dispatch(A[0], B[0], C, M, N, count * K_each, M, N, 0, 0, M * N, true, false, alpha, 1, workspace,
                         workspace_bytes, stream, e);
}

extern "C" int nnhip_gemm_tn_sum_seq(const float* const* A, const float* const* B, size_t count, float* C, size_t M,
                                     size_t N, size_t K_each, float alpha, nnhip_by_seq b_seq, void* workspace,
                                     size_t workspace_bytes, void* stream)
{
    if (!A || !B || !C || count == 0 || count > 3 || K_each == 0 || K_each % 16 != 0 || M % 4 != 0 || N % 4 != 0 ||
        count * K_each > 0x7fffffff || b_seq.len == 0 || !seq_ok(&b_seq, 1))
        return -1;
    GemmGroup g{};
    g.klen = static_cast<int>(K_each);
    g.bT[0] = static_cast<int>(b_seq.len);
    g.bS[0] = static_cast<long>(b_seq.step);
    for (size_t i = 0; i < count; ++i)
    {
        if (!A[i] || !B[i] || !aligned16(A[i]) || !aligned16(B[i])) return -1;
        g.A[i] = A[i];
        g.B[i] = B[i];
    }
    Epi e{nullptr, 0};
    e.seg = &g;
    e.by_seq = true;
    return gemm_dispatch(A[0], B[0], C, M, N, count * K_each, M, b_seq.len, 0, 0, M * N, true, false, alpha, 1,
                         workspace, workspace_bytes, stream, e);
}

extern "C" int nnhip_gemm_epilogue_seq(const float* A, const float* B, float* C, size_t M, size_t N, size_t K,
                                       float alpha, const float* row_bias, int accumulate, nnhip_by_seq b_seq,
                                       void* workspace, size_t workspace_bytes, void* stream)
{
    if (!A || !B || !C || b_seq.len == 0 || !seq_ok(&b_seq, 1)) return -1;
    GemmGroup g{};
    g.bT[0] = static_cast<int>(b_seq.len);
    g.bS[0] = static_cast<long>(b_seq.step);
    Epi e{row_bias, accumulate ? 1 : 0};
    e.sq = &g;
    e.by_seq = true;
    return gemm_dispatch(A, B, C, M, N, K, K, b_seq.len, M * K, 0, M * N, false, false, alpha, 1, workspace,
                         workspace_bytes, stream, e);
}

extern "C" int nnhip_gemm_heads(const float* W, const float* X, const float* row_bias, float* out, size_t M,
                                size_t K, size_t B, size_t T, void* stream)
{
    // Batch b: out_b (M, T) = W (M, K) X[:, b T : (b + 1) T] (+ bias), X read in place (ldb = B T); no
    // split-K (the per-batch products are whole tiles of work already).
    if (!W || !X || !out || B == 0 || T == 0 || M == 0 || K == 0) return -1;
    return gemm_dispatch(W, X, out, M, T, K, K, B * T, 0, T, M * T, false, false, 1.0f, B, nullptr, 0, stream,
                         Epi{row_bias, 0});
}

extern "C" int nnhip_gemm_heads_ex(const float* W, const float* X, const float* row_bias, float* out, size_t M,
                                   size_t K, size_t B, size_t T, int transW, void* stream)
{
    // nnhip_gemm_heads with W stored (K, M) when transW: out_b = W^T X_b (+ bias)
    if (!W || !X || !out || B == 0 || T == 0 || M == 0 || K == 0) return -1;
    return gemm_dispatch(W, X, out, M, T, K, transW ? M : K, B * T, 0, T, M * T, transW != 0, false, 1.0f, B, nullptr,
                         0, stream, Epi{row_bias, 0});
}

extern "C" int nnhip_gemm_heads_group(const float* const* W, const float* X, const float* const* row_bias,
                                      float* const* out, size_t count, size_t M, size_t K, size_t B, size_t T,
                                      void* stream)
{
    // grid z runs over count * B (member, sequence) pairs
    if (!W || !X || !out || count == 0 || count > 3 || B == 0 || T == 0 || M == 0 || K == 0 || count * B > 65535)
        return -1;
    GemmGroup g{};
    g.nb = static_cast<int>(B);
    for (size_t i = 0; i < count; ++i)
    {
        if (!W[i] || !out[i]) return -1;
        g.A[i] = W[i];
        g.C[i] = out[i];
        g.bias[i] = row_bias ? row_bias[i] : nullptr;
    }
    // Member pointers come from the group; A and C here only give the shape checks their operands.
    return gemm_dispatch(W[0], X, out[0], M, T, K, K, B * T, 0, T, M * T, false, false, 1.0f, count * B, nullptr, 0,
                         stream, Epi{nullptr, 0, &g});
}

// ── GEMM without allocation ─────────────────────────────────────────────────
// Split-K partial tiles of nnhip_gemm_noalloc live in this array. One copy
// per GPU, held from when the library's code object loads on that GPU until
// the process ends. Host code never passes `scratch` itself (its host-side
// name is not a device address): scratch_ptr() resolves the current GPU's
// copy once with hipGetSymbolAddress and every launch uses that address.
static __device__ __align__(256) float scratch[NNHIP_GEMM_NOALLOC_SCRATCH_BYTES / sizeof(float)];

namespace nnhip
{
namespace
{
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch[kMaxDevices] = {};

// The current GPU's address of `scratch` (resolved on the first call made with
// that GPU current). Returns 0, a hipError_t, or -1 for a device id past the table.
int scratch_ptr(float** out)
{
    int dev = 0;
    if (const hipError_t e = hipGetDevice(&dev); e != hipSuccess) return static_cast<int>(e);
    if (dev < 0 || dev >= kMaxDevices) return -1;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch[dev])
    {
        void* p = nullptr;
        if (const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)); e != hipSuccess)
            return static_cast<int>(e);
        if (!p) return -1;
        g_scratch[dev] = static_cast<float*>(p);
    }
    *out = g_scratch[dev];
    return 0;
}
} // namespace
} // namespace nnhip

// nnhip_gemm with the split-K partials in the library's own scratch: the same
// plan, kernels and summation order as nnhip_gemm given a workspace of
// nnhip_gemm_workspace_bytes(M, N, K, batch), so the results are identical.
// Every partial element is written by its slice before the reduction reads
// it, so nothing in the scratch has to start at zero.
extern "C" int nnhip_gemm_noalloc(const float* A, const float* B, float* C, size_t A_rows, size_t A_cols,
                                  size_t B_rows, size_t B_cols, size_t batch, int transA, int transB, float alpha,
                                  void* stream)
{
    if (batch == 0 || A_rows % batch || B_rows % batch) return -2;
    const size_t ar = A_rows / batch, br = B_rows / batch;
    const size_t M = transA ? A_cols : ar, K = transA ? ar : A_cols;
    const size_t K2 = transB ? B_cols : br, N = transB ? br : B_cols;
    if (K != K2) return -2;
    if (M == 0 || N == 0) return 0;
    if (nnhip_gemm_workspace_bytes(M, N, K, batch) > NNHIP_GEMM_NOALLOC_SCRATCH_BYTES) return -6;
    float* ws = nullptr;
    if (const int rc = scratch_ptr(&ws)) return rc;
    return gemm_dispatch(A, B, C, M, N, K, A_cols, B_cols, ar * A_cols, br * B_cols, M * N, transA != 0, transB != 0,
                         alpha, batch, ws, NNHIP_GEMM_NOALLOC_SCRATCH_BYTES, stream);
}

extern "C" int nnhip_matmul(const float* A, const float* B, float* C, size_t A_rows, size_t A_cols, size_t B_rows,
                            size_t B_cols, int transA, int transB, void* stream)
{
    return nnhip_gemm(A, B, C, A_rows, A_cols, B_rows, B_cols, 1, transA, transB, 1.0f, nullptr, 0, stream);
}

extern "C" int nnhip_batched_matmul(const float* A, const float* B, float* C, size_t A_rows, size_t A_cols,
                                    size_t B_rows, size_t B_cols, size_t batch, int transA, int transB, float alpha,
                                    void* stream)
{
    return nnhip_gemm(A, B, C, A_rows, A_cols, B_rows, B_cols, batch, transA, transB, alpha, nullptr, 0, stream);
}

// Up to four matrix-vector products of one x: v_i = R_i x (+ bias_i), each
// summed as the single product's gemv sums it (so bit-identical to
// nnhip_gemm_epilogue of (rows, K) x (K, 1) with the same bias), written to
// y_i and / or out_i (= add_i + v_i when add_i is set).
namespace
{
int gemv_group(const float* const* R, const float* x, const nnhip_gemv_rmsnorm* rms, const float* const* bias,
               float* const* y, const float* const* add, float* const* out, size_t count, size_t rows, size_t K,
               void* stream)
{
    if (count == 0 || rows == 0) return 0;
    if (count > 4 || !R || !x || (!y && !out) || K == 0 || K > 0x7fffffff || rows > 0x7fffffff) return -1;
    if (rms && (K > 1024 || !rms->gamma)) return -1;
    GemvGroup g{};
    bool vec = K % 4 == 0 && (rms || aligned16(x));
    for (size_t i = 0; i < count; ++i)
    {
        g.R[i] = R[i];
        g.y[i] = y ? y[i] : nullptr;
        g.bias[i] = bias ? bias[i] : nullptr;
        g.out[i] = out ? out[i] : nullptr;
        g.add[i] = add ? add[i] : nullptr;
        if (!R[i] || (!g.y[i] && !g.out[i]) || (g.add[i] && !g.out[i])) return -1;
        vec = vec && aligned16(R[i]);
    }
    auto s = static_cast<hipStream_t>(stream);
    const dim3 grid(static_cast<unsigned>((rows + 3) / 4), static_cast<unsigned>(count));
    const int r = static_cast<int>(rows), k = static_cast<int>(K);
    const nnhip_gemv_rmsnorm rn = rms ? *rms : nnhip_gemv_rmsnorm{};
    if (rms && vec)
        hipLaunchKernelGGL((k_gemv_group<true, 4, true>), grid, dim3(256), 0, s, g, x, r, k, rn);
    else if (rms)
        hipLaunchKernelGGL((k_gemv_group<false, 1, true>), grid, dim3(256), 0, s, g, x, r, k, rn);
    else if (vec && K <= 1024)
        hipLaunchKernelGGL((k_gemv_group<true, 4, false>), grid, dim3(256), 0, s, g, x, r, k, rn);
    else if (vec && K <= 2048)
        hipLaunchKernelGGL((k_gemv_group<true, 8, false>), grid, dim3(256), 0, s, g, x, r, k, rn);
    else if (vec)
        hipLaunchKernelGGL((k_gemv_group<true, 16, false>), grid, dim3(256), 0, s, g, x, r, k, rn);
    else
        hipLaunchKernelGGL((k_gemv_group<false, 1, false>), grid, dim3(256), 0, s, g, x, r, k, rn);
    return launch_status();
}
} // namespace

extern "C" int nnhip_gemv_group(const float* const* R, const float* x, const float* const* bias, float* const* y,
                                const float* const* add, float* const* out, size_t count, size_t rows, size_t K,
                                void* stream)
{
    return gemv_group(R, x, nullptr, bias, y, add, out, count, rows, K, stream);
}

// fc1 (2 half rows) of x or of RMSNorm(x), and SwiGLU::forward's chain on its
// two halves, in one launch: bit-identical to nnhip_gemv_group[_rmsnorm] of
// the 2 half rows followed by nnhip_swiglu_forward(y, y + half, s, out).
extern "C" int nnhip_gemv_swiglu(const float* R, const float* x, const nnhip_gemv_rmsnorm* rms, const float* bias,
                                 float* y, float* s_out, float* out, size_t half, size_t K, float c_add, float c_div,
                                 void* stream)
{
    if (half == 0) return 0;
    if (!R || !x || !out || K == 0 || K > 0x7fffffff || half > 0x3fffffff) return -1;
    if (rms && (K > 1024 || !rms->gamma)) return -1;
    const bool vec = K % 4 == 0 && (rms || aligned16(x)) && aligned16(R);
    if (rms && !vec) return -1;
    GemvSwiglu g{R, bias, y, s_out, out, static_cast<int>(half), static_cast<int>(K), c_add, c_div};
    const nnhip_gemv_rmsnorm rn = rms ? *rms : nnhip_gemv_rmsnorm{};
    auto s = static_cast<hipStream_t>(stream);
    const dim3 grid(static_cast<unsigned>((half + 3) / 4));
    if (rms)
        hipLaunchKernelGGL((k_gemv_swiglu<true, 4, true>), grid, dim3(256), 0, s, g, x, rn);
    else if (vec && K <= 1024)
        hipLaunchKernelGGL((k_gemv_swiglu<true, 4, false>), grid, dim3(256), 0, s, g, x, rn);
    else if (vec && K <= 2048)
        hipLaunchKernelGGL((k_gemv_swiglu<true, 8, false>), grid, dim3(256), 0, s, g, x, rn);
    else if (vec)
        hipLaunchKernelGGL((k_gemv_swiglu<true, 16, false>), grid, dim3(256), 0, s, g, x, rn);
    else
        hipLaunchKernelGGL((k_gemv_swiglu<false, 1, false>), grid, dim3(256), 0, s, g, x, rn);
    return launch_status();
}

// The same products of RMSNorm(x) (a (K, 1) column, K <= 1024).
extern "C" int nnhip_gemv_group_rmsnorm(const float* const* R, const float* x, const nnhip_gemv_rmsnorm* rms,
                                        const float* const* bias, float* const* y, const float* const* add,
                                        float* const* out, size_t count, size_t rows, size_t K, void* stream)
{
    if (!rms) return -1;
    return gemv_group(R, x, rms, bias, y, add, out, count, rows, K, stream);
}
