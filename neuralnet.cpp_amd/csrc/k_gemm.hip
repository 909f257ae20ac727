// k_gemm.hip — fp32 GEMM on the gfx950 matrix cores (v_mfma_f32_32x32x2_f32).
//
// Computes C_b = alpha * op(A_b) op(B_b) for `batch` row blocks, covering
// ComputeEngine::matmul (compute_engine.hpp:182-184) and ::batched_matmul
// (:195-199; cpu_engine.hpp:335-419 applies alpha after the product, so does
// the epilogue here). All four transpose combinations are handled at the
// global->LDS staging step: both operands are kept k-major in LDS
// (As[k][m], Bs[k][n]) so every MFMA fragment read is 32 consecutive floats.
//
// Tiling: a workgroup of 4 waves owns a (64*WM) x (64*WN) tile of C
// (WM*WN = 4); each wave owns 64x64 = 2x2 MFMA 32x32 blocks (64 accumulators
// per lane). K advances 16 at a time through two LDS buffers: the next
// stage's global loads are issued into registers before the current stage's
// MFMAs and written to the other buffer afterwards (one barrier per stage).
//
// MFMA 32x32x2 f32 operand layout (per lane l, k-step of 2):
//   A: A[i = l%32][k = l/32],  B: B[k = l/32][j = l%32],
//   D: 16 values, value r at row 8*(r/4) + 4*(l/32) + r%4, column l%32.
#include "common.hpp"
#include "nnhip_kernels.h"

namespace nnhip
{
namespace
{

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int BK = 16;
constexpr int PAD = 4;

template <int WM, int WN, bool TA, bool TB, bool GUARD>
__global__ __launch_bounds__(256) void k_gemm(const float* __restrict__ A, const float* __restrict__ B,
                                              float* __restrict__ C, int M, int N, int K, long lda, long ldb,
                                              long strideA, long strideB, long strideC, float alpha, int tiles_n)
{
    constexpr int BM = 64 * WM, BN = 64 * WN;
    constexpr int LDA_S = BM + PAD, LDB_S = BN + PAD;
    constexpr int LA = BM * BK / 4 / 256;   // float4 per thread per stage for A
    constexpr int LB = BN * BK / 4 / 256;
    __shared__ __attribute__((aligned(16))) float As[2][BK][LDA_S];
    __shared__ __attribute__((aligned(16))) float Bs[2][BK][LDB_S];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int tile = blockIdx.x;
    const int m0 = (tile / tiles_n) * BM, n0 = (tile % tiles_n) * BN;
    const long bz = blockIdx.z;
    A += bz * strideA;
    B += bz * strideB;
    C += bz * strideC;

    float4 ra[LA], rb[LB];

    // A_eff(m, k) = TA ? A[k*lda + m] : A[m*lda + k]
    auto load_a = [&](int k0) {
#pragma unroll
        for (int s = 0; s < LA; ++s)
        {
            const int idx = tid + 256 * s;
            int m, k;
            if constexpr (TA) { k = idx / (BM / 4); m = (idx % (BM / 4)) * 4; }
            else { m = idx / (BK / 4); k = (idx % (BK / 4)) * 4; }
            const int gm = m0 + m, gk = k0 + k;
            if constexpr (!GUARD)
            {
                ra[s] = TA ? *reinterpret_cast<const float4*>(A + (long)gk * lda + gm)
                           : *reinterpret_cast<const float4*>(A + (long)gm * lda + gk);
            }
            else
            {
                float v[4];
#pragma unroll
                for (int q = 0; q < 4; ++q)
                {
                    const int mm = TA ? gm + q : gm, kk = TA ? gk : gk + q;
                    v[q] = (mm < M && kk < K) ? (TA ? A[(long)kk * lda + mm] : A[(long)mm * lda + kk]) : 0.0f;
                }
                ra[s] = make_float4(v[0], v[1], v[2], v[3]);
            }
        }
    };
    // B_eff(k, n) = TB ? B[n*ldb + k] : B[k*ldb + n]
    auto load_b = [&](int k0) {
#pragma unroll
        for (int s = 0; s < LB; ++s)
        {
            const int idx = tid + 256 * s;
            int n, k;
            if constexpr (!TB) { k = idx / (BN / 4); n = (idx % (BN / 4)) * 4; }
            else { n = idx / (BK / 4); k = (idx % (BK / 4)) * 4; }
            const int gn = n0 + n, gk = k0 + k;
            if constexpr (!GUARD)
            {
                rb[s] = !TB ? *reinterpret_cast<const float4*>(B + (long)gk * ldb + gn)
                            : *reinterpret_cast<const float4*>(B + (long)gn * ldb + gk);
            }
            else
            {
                float v[4];
#pragma unroll
                for (int q = 0; q < 4; ++q)
                {
                    const int nn = !TB ? gn + q : gn, kk = !TB ? gk : gk + q;
                    v[q] = (nn < N && kk < K) ? (!TB ? B[(long)kk * ldb + nn] : B[(long)nn * ldb + kk]) : 0.0f;
                }
                rb[s] = make_float4(v[0], v[1], v[2], v[3]);
            }
        }
    };
    auto store_a = [&](int buf) {
#pragma unroll
        for (int s = 0; s < LA; ++s)
        {
            const int idx = tid + 256 * s;
            if constexpr (TA)
            {
                const int k = idx / (BM / 4), m = (idx % (BM / 4)) * 4;
                *reinterpret_cast<float4*>(&As[buf][k][m]) = ra[s];
            }
            else
            {
                const int m = idx / (BK / 4), k = (idx % (BK / 4)) * 4;
                As[buf][k + 0][m] = ra[s].x;
                As[buf][k + 1][m] = ra[s].y;
                As[buf][k + 2][m] = ra[s].z;
                As[buf][k + 3][m] = ra[s].w;
            }
        }
    };
    auto store_b = [&](int buf) {
#pragma unroll
        for (int s = 0; s < LB; ++s)
        {
            const int idx = tid + 256 * s;
            if constexpr (!TB)
            {
                const int k = idx / (BN / 4), n = (idx % (BN / 4)) * 4;
                *reinterpret_cast<float4*>(&Bs[buf][k][n]) = rb[s];
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

    floatx16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    const int kt_n = (K + BK - 1) / BK;
    if (kt_n > 0)
    {
        load_a(0);
        load_b(0);
        store_a(0);
        store_b(0);
        __syncthreads();
    }
    const int am = wm * 64 + (lane & 31), bn = wn * 64 + (lane & 31), kl = lane >> 5;
    for (int kt = 0; kt < kt_n; ++kt)
    {
        const int buf = kt & 1;
        const bool more = kt + 1 < kt_n;
        if (more)
        {
            load_a((kt + 1) * BK);
            load_b((kt + 1) * BK);
        }
#pragma unroll
        for (int kk = 0; kk < BK; kk += 2)
        {
            const float a0 = As[buf][kk + kl][am], a1 = As[buf][kk + kl][am + 32];
            const float b0 = Bs[buf][kk + kl][bn], b1 = Bs[buf][kk + kl][bn + 32];
            acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b0, acc[0][0], 0, 0, 0);
            acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b1, acc[0][1], 0, 0, 0);
            acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b0, acc[1][0], 0, 0, 0);
            acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b1, acc[1][1], 0, 0, 0);
        }
        if (more)
        {
            store_a(buf ^ 1);
            store_b(buf ^ 1);
        }
        __syncthreads();
    }

    // Epilogue: C = alpha * acc.
    const int col_l = lane & 31, row_l = 4 * (lane >> 5);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
        {
            const int gn = n0 + wn * 64 + j * 32 + col_l;
#pragma unroll
            for (int r = 0; r < 16; ++r)
            {
                const int gm = m0 + wm * 64 + i * 32 + 8 * (r / 4) + row_l + (r % 4);
                if (!GUARD || (gm < M && gn < N)) C[(long)gm * N + gn] = alpha * acc[i][j][r];
            }
        }
}

template <int WM, int WN, bool TA, bool TB>
void launch_cfg(const float* A, const float* B, float* C, int M, int N, int K, long lda, long ldb, long sA, long sB,
                long sC, float alpha, int batch, bool guard, hipStream_t s)
{
    constexpr int BM = 64 * WM, BN = 64 * WN;
    const int tm = (M + BM - 1) / BM, tn = (N + BN - 1) / BN;
    const dim3 grid(static_cast<unsigned>(tm * tn), 1, static_cast<unsigned>(batch));
    if (guard)
        hipLaunchKernelGGL((k_gemm<WM, WN, TA, TB, true>), grid, dim3(256), 0, s, A, B, C, M, N, K, lda, ldb, sA, sB,
                           sC, alpha, tn);
    else
        hipLaunchKernelGGL((k_gemm<WM, WN, TA, TB, false>), grid, dim3(256), 0, s, A, B, C, M, N, K, lda, ldb, sA,
                           sB, sC, alpha, tn);
}

template <bool TA, bool TB>
void launch_trans(const float* A, const float* B, float* C, int M, int N, int K, long lda, long ldb, long sA, long sB,
                  long sC, float alpha, int batch, hipStream_t s)
{
    const bool vec_ok = (lda % 4 == 0) && (ldb % 4 == 0) && (sA % 4 == 0) && (sB % 4 == 0) && aligned16(A) &&
                        aligned16(B);
    if (M <= 64)
    {
        const bool guard = !vec_ok || (M % 64) || (N % 256) || (K % BK);
        launch_cfg<1, 4, TA, TB>(A, B, C, M, N, K, lda, ldb, sA, sB, sC, alpha, batch, guard, s);
    }
    else if (N <= 64)
    {
        const bool guard = !vec_ok || (M % 256) || (N % 64) || (K % BK);
        launch_cfg<4, 1, TA, TB>(A, B, C, M, N, K, lda, ldb, sA, sB, sC, alpha, batch, guard, s);
    }
    else
    {
        const bool guard = !vec_ok || (M % 128) || (N % 128) || (K % BK);
        launch_cfg<2, 2, TA, TB>(A, B, C, M, N, K, lda, ldb, sA, sB, sC, alpha, batch, guard, s);
    }
}

int gemm_dispatch(const float* A, const float* B, float* C, size_t M, size_t N, size_t K, size_t lda, size_t ldb,
                  size_t sA, size_t sB, size_t sC, bool tA, bool tB, float alpha, size_t batch, void* stream)
{
    if (M == 0 || N == 0 || batch == 0) return 0;
    if (M > 0x7fffffff || N > 0x7fffffff || K > 0x7fffffff || batch > 65535) return -1;
    auto s = static_cast<hipStream_t>(stream);
    const int m = (int)M, n = (int)N, k = (int)K, b = (int)batch;
    if (!tA && !tB) launch_trans<false, false>(A, B, C, m, n, k, lda, ldb, sA, sB, sC, alpha, b, s);
    else if (!tA && tB) launch_trans<false, true>(A, B, C, m, n, k, lda, ldb, sA, sB, sC, alpha, b, s);
    else if (tA && !tB) launch_trans<true, false>(A, B, C, m, n, k, lda, ldb, sA, sB, sC, alpha, b, s);
    else launch_trans<true, true>(A, B, C, m, n, k, lda, ldb, sA, sB, sC, alpha, b, s);
    return launch_status();
}

} // namespace
} // namespace nnhip

using namespace nnhip;

extern "C" int nnhip_matmul(const float* A, const float* B, float* C, size_t A_rows, size_t A_cols, size_t B_rows,
                            size_t B_cols, int transA, int transB, void* stream)
{
    const size_t M = transA ? A_cols : A_rows, K = transA ? A_rows : A_cols;
    const size_t K2 = transB ? B_cols : B_rows, N = transB ? B_rows : B_cols;
    if (K != K2) return -2;
    return gemm_dispatch(A, B, C, M, N, K, A_cols, B_cols, 0, 0, 0, transA != 0, transB != 0, 1.0f, 1, stream);
}

extern "C" int nnhip_batched_matmul(const float* A, const float* B, float* C, size_t A_rows, size_t A_cols,
                                    size_t B_rows, size_t B_cols, size_t batch, int transA, int transB, float alpha,
                                    void* stream)
{
    if (batch == 0 || A_rows % batch || B_rows % batch) return -2;
    const size_t ar = A_rows / batch, br = B_rows / batch;
    const size_t M = transA ? A_cols : ar, K = transA ? ar : A_cols;
    const size_t K2 = transB ? B_cols : br, N = transB ? br : B_cols;
    if (K != K2) return -2;
    return gemm_dispatch(A, B, C, M, N, K, A_cols, B_cols, ar * A_cols, br * B_cols, M * N, transA != 0, transB != 0,
                         alpha, batch, stream);
}
