// flash.hpp — host interface of the one-pass attention chains (k_flash.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>

#include "nnhip_kernels.h"

namespace nnhip
{

// Geometry of one launch (filled by the host planner in k_flash.hip).
struct FlashGeo
{
    int M, N;        // queries, keys per batch entry
    int RT, CT;      // 32-wide query tiles, key tiles
    int R, NR;       // cells per range, ranges per line
    int G;           // line groups (4 lines each) per batch entry
    int pw;          // floats per (line, range) partial
    const unsigned char* cls;   // RT x CT mask cell classes, or nullptr without a mask
    long cls_bs;     // bytes between batch entries' cell tables (0: one table shared)
    float* part;     // partials of lines cut into several ranges
    const int* order;   // workgroup -> work item (a permutation of the grid), or nullptr
};

// Forward: m, l (batch*M) and, when O is not null, O (batch*M, D).
struct FlashFwdArgs
{
    const float* Q;      // per batch (K, M)
    const float* Kt;     // per batch (K, N)
    const float* V;      // per batch (N, D); unused without O
    const float* mask;   // (M, N) per batch entry (mask_bs apart), or nullptr
    float* m;
    float* l;
    float* O;
    int M, N, K, D;
    float alpha;
    long mask_bs;        // floats between batch entries' masks (0: one mask shared)
    int v_dm;            // V per batch is (D, N) [dim][key] instead of (N, D)
    int o_dm;            // O per batch is written (D, M) [dim][query] instead of (M, D)
    float* S;            // when set: each visited cell's scores (alpha q.k + mask) as a score block
};

// Backward: R (batch*M), dQ (batch*K, M), dK and dV (batch*K, N) from
// P_ij = alpha2 * sum_k dO(k, i) V'(k, j) (recomputed), G (per batch (M, ldg)).
struct FlashBwdArgs
{
    const float* Q;      // per batch (K, M)
    const float* Kt;     // per batch (K, N)
    const float* dO;     // per batch (Kd, M)
    const float* Vp;     // per batch (Kd, N)
    const float* G;      // per batch (M, ldg), ldg >= K; unused when g_do
    const float* mask;   // (M, N) per batch entry (mask_bs apart), or nullptr
    const float* m;
    const float* l;
    float* R;
    float* dQ;
    float* dK;
    float* dV;
    int M, N, K, Kd, ldg;
    float alpha, alpha2;
    long mask_bs;        // floats between batch entries' masks (0: one mask shared)
    int g_do;            // G_i is dO's column i (dV_j = sum_i W dO_i; needs Kd == K)
    float* dS;           // the key-line pass also stores dS_ij = W (P - R_i) here, (batch*M, N)
    const float* S;      // when set: the forward's score blocks; the key-line pass reads them instead of
                         // recomputing alpha q.k + mask
};
// One launch over several independent calls ("rows": e.g. the packed rows of a
// document-masked batch, each with its own (M, N) mask) of the same shape.
// Batch entry b of the launch belongs to row b / hpr. Each row's arguments
// hold pointers pre-offset by -(row * hpr) batch entries, so that the kernels
// index every array with the launch-wide b exactly as in a one-row launch;
// cls[row] likewise for the row's mask cell tables.
constexpr int kFlashMaxRows = NNHIP_FLASH_MAX_ROWS;
template <class Args>
struct FlashSet
{
    Args a[kFlashMaxRows];
    const unsigned char* cls[kFlashMaxRows];
    int hpr;   // batch entries per row (>= 1)
    int rows;
};
using FlashFwdSet = FlashSet<FlashFwdArgs>;
using FlashBwdSet = FlashSet<FlashBwdArgs>;

// Score blocks: one per 32 x 32 cell, block (b, query tile, key tile) at
// ((b RT + qt) CT + kt) 1024 floats; inside, score (query q, key k) at
// r 64 + h 32 + q with drow(r, h) = k (the forward's lane order).
inline size_t score_blocks_floats(size_t batch, size_t M, size_t N)
{
    return batch * ((M + 31) / 32) * ((N + 31) / 32) * 1024;
}

// Shapes the one-pass kernels take: head dims K (and Kd) <= 64, value width
// D <= 64 with D % 4 == 0. The backward also needs K % 4 == 0 and ldg % 4 == 0.
bool flash_supported(size_t batch, size_t M, size_t N, size_t K, size_t D);
// Mask cell table: one byte per 32x32 cell of each (M, N) mask (0 all -inf, 1 all zero, 2 general);
// masks batches, mask_bs floats apart, give batches tables of flash_cells_bytes(M, N) each.
size_t flash_cells_bytes(size_t M, size_t N);
int flash_classify(const float* mask, size_t masks, long mask_bs, size_t M, size_t N, void* cells, hipStream_t s);
size_t flash_workspace_bytes(size_t batch, size_t M, size_t N, size_t K, size_t D, bool backward);
// Work order tables (workgroup -> item) for kind 0 forward, 1 backward, 2 the dS backward.
size_t flash_order_bytes(size_t batch, size_t M, size_t N, int kind);
int flash_build_order(const unsigned char* cells, size_t batch, size_t M, size_t N, bool per_batch_cls, int kind,
                      void* order, hipStream_t s);
// order: a table from flash_build_order for the same cells and shape, or nullptr (grid order).
int flash_forward(const FlashFwdArgs& a, const unsigned char* cells, size_t batch, void* workspace, const int* order,
                  hipStream_t s);
int flash_backward(const FlashBwdArgs& a, const unsigned char* cells, size_t batch, void* workspace, const int* order,
                   hipStream_t s);
// Backward when the forward output O (from the same V as V') is at hand: R_i = alpha2 dO_i . O_i
// directly (O per batch (Kd, M) dim-major, or (M, Kd) query-major when o_qm; R kept when a.R is set),
// one key-line pass for dK, dV and dS, then dQ = alpha dS K.
size_t flash_ds_workspace_bytes(size_t batch, size_t M, size_t N, size_t K);
int flash_backward_ds(const FlashBwdArgs& a, const float* O, int o_qm, const unsigned char* cells, size_t batch,
                      void* workspace, const int* order, hipStream_t s);

// Multi-row forms: `rows` calls of `hpr` batch entries each, row r with its own
// arguments (unshifted pointers, as for the one-row call) and cells[r]; the
// workspace and order table cover batch rows * hpr (flash_rows_order_bytes /
// flash_build_rows_order; flash_workspace_bytes and flash_ds_workspace_bytes
// at that batch).
int flash_forward_rows(const FlashFwdArgs* a, const unsigned char* const* cells, int rows, size_t hpr,
                       void* workspace, const int* order, hipStream_t s);
int flash_backward_ds_rows(const FlashBwdArgs* a, const float* const* O, int o_qm, const unsigned char* const* cells,
                           int rows, size_t hpr, void* workspace, const int* order, hipStream_t s);
int flash_build_rows_order(const unsigned char* const* cells, int rows, size_t hpr, size_t M, size_t N,
                           bool per_batch_cls, int kind, void* order, hipStream_t s);

} // namespace nnhip
