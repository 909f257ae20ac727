// attn_mfma.hpp — host interface of the matrix-core attention kernels
// (k_attn_mfma.hip), used by the fused attention entry points in k_attention.hip.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>

namespace nnhip
{

struct AttnArgs
{
    const float* A;
    const float* B;
    const float* mask;   // (M, N) shared by all batches, or nullptr
    int M, N, K;
    int tA, tB;
    float alpha;
};

enum { kFwdMax = 0, kFwdDenom = 1, kFwdApply = 2 };

// Workspace of one fused-attention call on (batch, M, N, K) with value width D:
// the mask-cell table, the combine counters and the partial results.
size_t attn_workspace_bytes(size_t batch, size_t M, size_t N, size_t K, size_t D);
// Shapes the matrix-core path takes (K <= 128, M and N <= 32768); the caller
// must also pass a workspace, else the general kernels run.
bool attn_mfma_supported(size_t batch, size_t M, size_t N, size_t K);
// mode kFwdMax: out[b*M+i] = max_j s_ij; kFwdDenom: out = sum_j exp(s_ij - m_i);
// kFwdApply: out[(b*M+i)*D + k] = sum_j W_ij V[(b*N+j)*D + k]   (D <= 128).
int attn_mfma_forward(const AttnArgs& d, size_t batch, int mode, const float* row_max, const float* denom,
                      const float* V, size_t D, float* out, void* workspace, hipStream_t s);
// kv = false: o1 = dQ, o2 = R;  kv = true: o1 = dK, o2 = dV (G has D >= K columns, R_in given).
int attn_mfma_backward(const AttnArgs& d, size_t batch, bool kv, const float* P, const float* G, size_t D,
                       const float* R_in, const float* row_max, const float* denom, float* o1, float* o2,
                       void* workspace, hipStream_t s);

} // namespace nnhip
