// k_expr.hip — ExprSpec evaluation on the GPU (eval_expr / eval_expr_reduce).
//
// Semantics are those of the CPU interpreter (cpu_engine.hpp:1298-1659):
//   1. every reduce VIEW becomes a per-row / per-column vector of its input
//      (max starts from lowest(), sum from 0);
//   2. reduce INSTRUCTIONS are evaluated in program order, each reducing the
//      elementwise prefix before it over the full grid (row reductions: one
//      wave per row; column reductions: row-chunk partials merged in order);
//   3. the elementwise pass evaluates the whole program per element, or per
//      representative element (r,0) / (0,c) for the reduced-vector output.
// The program travels by value in the kernel arguments, so every branch on
// an opcode or operand kind is uniform across the wave; the register file
// lives in VGPRs.
#include <cstring>
#include <vector>

#include "common.hpp"
#include "nn/expr_spec.hpp"
#include "nnhip_kernels.h"

namespace nnhip
{
namespace
{

constexpr unsigned kThreads = 256;

// Device-side copy of the program. Every field indexed at run time is a
// 32-bit word or wider and every record is 8-byte aligned: a byte array
// indexed by a run-time value lets the compiler form a scalar-load base of
// kernarg + index (not dword-aligned) and reuse it for the word arrays beside
// it, and scalar loads drop the low two address bits of such a base.
struct ViewArg
{
    const float* in;
    const float* vred;      // reduce-view vector
    unsigned param;         // RotateHalf block / RowMod modulus
    unsigned kind;
    unsigned negate;
    unsigned pad;
};
struct ExprArgs
{
    unsigned instrs[64][2];   // the 8 instruction bytes as two little-endian words
    float consts[16];
    ViewArg view[8];
    const float* rvec[16];    // reduce-instruction vectors, by destination register
    unsigned raxis[16];       // 1 = per column, 0 = per row
    unsigned n_instrs;
    size_t rows, cols;
};

// Byte b (0..7) of instruction j.
__device__ __forceinline__ unsigned ibyte(const ExprArgs& A, unsigned j, unsigned b)
{
    return (A.instrs[j][b >> 2] >> (8 * (b & 3))) & 0xffu;
}

enum : unsigned char { K_REG = 0, K_INPUT = 1, K_CONST = 2, K_FANOUT = 3, K_REDUCE = 4 };
enum : unsigned char
{
    V_LINEAR = 0, V_ROTATE = 1, V_ROWMOD = 2, V_COLSUM = 3, V_COLMAX = 4, V_ROWSUM = 5, V_ROWMAX = 6,
    V_ROWBC = 7, V_COLBC = 8
};
enum : unsigned char
{
    E_NEG = 0, E_EXP, E_LOG, E_SQRT, E_RSQRT, E_ABS, E_TANH, E_ADD, E_SUB, E_MUL, E_DIV, E_MAX, E_MIN, E_LT, E_LE,
    E_GT, E_GE, E_EQ, E_NE, E_SELECT, E_COLSUM, E_COLMAX, E_ROWSUM, E_ROWMAX
};

__device__ __forceinline__ bool is_reduce(unsigned op) { return op >= E_COLSUM; }

__device__ __forceinline__ float read_input(const ExprArgs& A, unsigned k, size_t r, size_t c)
{
    const ViewArg& v = A.view[k];
    const float* s = v.in;
    const size_t cols = A.cols;
    switch (v.kind)
    {
    case V_ROTATE:
    {
        const size_t blk = v.param, rl = r % blk, h = blk / 2;
        const size_t rr = (r / blk) * blk + (rl < h ? rl + h : rl - h);
        const float x = s[rr * cols + c];
        return (v.negate && rl < h) ? -x : x;
    }
    case V_ROWMOD: return s[(r % v.param) * cols + c];
    case V_ROWSUM:
    case V_ROWMAX: return v.vred[r];
    case V_COLSUM:
    case V_COLMAX: return v.vred[c];
    case V_ROWBC: return s[r];
    case V_COLBC: return s[c];
    default: return s[r * cols + c];
    }
}

__device__ __forceinline__ float operand(const ExprArgs& A, unsigned kind, unsigned idx, size_t r, size_t c,
                                         const float* regs)
{
    switch (kind)
    {
    case K_CONST: return A.consts[idx];
    case K_INPUT: return read_input(A, idx, r, c);
    case K_REDUCE: return A.rvec[idx][A.raxis[idx] ? c : r];
    default: return regs[idx];
    }
}

__device__ __forceinline__ float apply(unsigned op, float a, float b, float c)
{
    switch (op)
    {
    case E_NEG: return -a;
    case E_EXP: return expf(a);
    case E_LOG: return logf(a);
    case E_SQRT: return sqrtf(a);
    case E_RSQRT: return 1.0f / sqrtf(a);
    case E_ABS: return fabsf(a);
    case E_TANH: return tanhf(a);
    case E_ADD: return a + b;
    case E_SUB: return a - b;
    case E_MUL: return a * b;
    case E_DIV: return a / b;
    case E_MAX: return fmax_std(a, b);
    case E_MIN: return fmin_std(a, b);
    case E_LT: return a < b ? 1.0f : 0.0f;
    case E_LE: return a <= b ? 1.0f : 0.0f;
    case E_GT: return a > b ? 1.0f : 0.0f;
    case E_GE: return a >= b ? 1.0f : 0.0f;
    case E_EQ: return a == b ? 1.0f : 0.0f;
    case E_NE: return a != b ? 1.0f : 0.0f;
    case E_SELECT: return a != 0.0f ? b : c;
    default: return 0.0f;
    }
}

// Evaluates the elementwise instructions [0, upto) at (r, c).
__device__ __forceinline__ void run_prefix(const ExprArgs& A, unsigned upto, size_t r, size_t c, float* regs)
{
    for (unsigned j = 0; j < upto; ++j)
    {
        const unsigned op = ibyte(A, j, 0);
        if (is_reduce(op)) continue;
        const float a = operand(A, ibyte(A, j, 2), ibyte(A, j, 3), r, c, regs);
        const float b = (op >= E_ADD) ? operand(A, ibyte(A, j, 4), ibyte(A, j, 5), r, c, regs) : 0.0f;
        const float cc = (op == E_SELECT) ? operand(A, ibyte(A, j, 6), ibyte(A, j, 7), r, c, regs) : 0.0f;
        regs[ibyte(A, j, 1)] = apply(op, a, b, cc);
    }
}

__device__ __forceinline__ float eval_reduce_source(const ExprArgs& A, unsigned ri, size_t r, size_t c)
{
    float regs[16];
    run_prefix(A, ri, r, c, regs);
    return operand(A, ibyte(A, ri, 2), ibyte(A, ri, 3), r, c, regs);
}

// Row-axis reduce instruction ri: one wave per row.
__global__ __launch_bounds__(kThreads) void k_expr_reduce_rows(ExprArgs A, unsigned ri, float* out, int is_max)
{
    const size_t r = static_cast<size_t>(blockIdx.x) * 4 + threadIdx.x / 64;
    if (r >= A.rows) return;
    const unsigned lane = threadIdx.x % 64;
    float acc = is_max ? kLowest : 0.0f;
    for (size_t c = lane; c < A.cols; c += 64)
    {
        const float v = eval_reduce_source(A, ri, r, c);
        acc = is_max ? fmax_std(acc, v) : acc + v;
    }
    acc = is_max ? wave_max(acc) : wave_sum(acc);
    if (lane == 0) out[r] = acc;
}

// Column-axis reduce instruction ri: per row chunk, one lane per column.
__global__ __launch_bounds__(kThreads) void k_expr_reduce_cols(ExprArgs A, unsigned ri, float* part,
                                                               size_t rows_per_chunk, int is_max)
{
    const size_t c = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (c >= A.cols) return;
    const size_t r0 = static_cast<size_t>(blockIdx.y) * rows_per_chunk;
    size_t r1 = r0 + rows_per_chunk;
    if (r1 > A.rows) r1 = A.rows;
    float acc = is_max ? kLowest : 0.0f;
    for (size_t r = r0; r < r1; ++r)
    {
        const float v = eval_reduce_source(A, ri, r, c);
        acc = is_max ? fmax_std(acc, v) : acc + v;
    }
    part[static_cast<size_t>(blockIdx.y) * A.cols + c] = acc;
}

__global__ __launch_bounds__(kThreads) void k_expr_merge_cols(const float* part, float* out, size_t chunks,
                                                              size_t cols, int is_max)
{
    const size_t c = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (c >= cols) return;
    float acc = part[c];
    for (size_t k = 1; k < chunks; ++k) acc = is_max ? fmax_std(acc, part[k * cols + c]) : acc + part[k * cols + c];
    out[c] = acc;
}

// Elementwise output over the full grid.
__global__ __launch_bounds__(kThreads) void k_expr_elementwise(ExprArgs A, float* out)
{
    const size_t n = A.rows * A.cols;
    const unsigned last = A.n_instrs - 1;
    const unsigned lop = ibyte(A, last, 0), ldst = ibyte(A, last, 1);
    const size_t stride = static_cast<size_t>(gridDim.x) * kThreads;
    for (size_t i = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x; i < n; i += stride)
    {
        const size_t r = i / A.cols, c = i % A.cols;
        if (is_reduce(lop))
        {
            out[i] = A.rvec[ldst][A.raxis[ldst] ? c : r];
            continue;
        }
        float regs[16];
        run_prefix(A, A.n_instrs, r, c, regs);
        out[i] = regs[ldst];
    }
}

// Reduced-vector output at the representative elements (k,0) or (0,k).
__global__ __launch_bounds__(kThreads) void k_expr_vector(ExprArgs A, float* out, size_t len, int row_axis)
{
    const size_t k = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (k >= len) return;
    const unsigned last = A.n_instrs - 1;
    const unsigned lop = ibyte(A, last, 0), ldst = ibyte(A, last, 1);
    if (is_reduce(lop))
    {
        out[k] = A.rvec[ldst][k];
        return;
    }
    float regs[16];
    const size_t r = row_axis ? k : 0, c = row_axis ? 0 : k;
    run_prefix(A, A.n_instrs, r, c, regs);
    out[k] = regs[ldst];
}

struct Chunks
{
    size_t chunks, rows_per_chunk;
};
Chunks col_chunks(size_t rows, size_t cols)
{
    const size_t col_blocks = (cols + kThreads - 1) / kThreads;
    size_t chunks = 2048 / (col_blocks ? col_blocks : 1);
    const size_t max_chunks = (rows + 15) / 16;
    if (chunks > max_chunks) chunks = max_chunks;
    if (chunks < 1) chunks = 1;
    Chunks c;
    c.rows_per_chunk = (rows + chunks - 1) / chunks;
    if (c.rows_per_chunk == 0) c.rows_per_chunk = 1;
    c.chunks = (rows + c.rows_per_chunk - 1) / c.rows_per_chunk;
    if (c.chunks < 1) c.chunks = 1;
    return c;
}

nn::ExprSpec to_spec(const nnhip_expr_program& p)
{
    nn::ExprSpec s;
    for (unsigned i = 0; i < p.n_instrs && i < 64; ++i)
    {
        const unsigned char* b = p.instrs[i];
        s.instrs.push_back(nn::ExprInstr{b[0], b[1], {b[2], b[3]}, {b[4], b[5]}, {b[6], b[7]}});
    }
    for (unsigned i = 0; i < p.n_views && i < 8; ++i)
        s.views.push_back(nn::ExprView{p.view_kind[i], p.view_negate[i], p.view_param[i]});
    for (unsigned i = 0; i < p.n_consts && i < 16; ++i) s.consts.push_back(p.consts[i]);
    s.num_regs = p.num_regs;
    return s;
}

// Workspace layout: [view vectors | reduce-instruction vectors | column partials].
struct Layout
{
    size_t view_off[8], rvec_off[16], part_off, total;   // in floats
};
Layout layout(const nnhip_expr_program& p, size_t rows, size_t cols)
{
    Layout L{};
    size_t off = 0;
    for (unsigned k = 0; k < p.n_views; ++k)
    {
        const unsigned char v = p.view_kind[k];
        L.view_off[k] = off;
        if (v >= V_COLSUM && v <= V_ROWMAX) off += (v >= V_ROWSUM) ? rows : cols;
    }
    for (unsigned j = 0; j < p.n_instrs; ++j)
    {
        const unsigned char op = p.instrs[j][0], dst = p.instrs[j][1];
        if (op >= E_COLSUM && dst < 16)
        {
            L.rvec_off[dst] = off;
            off += (op == E_COLSUM || op == E_COLMAX) ? cols : rows;
        }
    }
    L.part_off = off;
    const Chunks ch = col_chunks(rows, cols);
    off += ch.chunks * cols;
    L.total = off;
    return L;
}

} // namespace
} // namespace nnhip

using namespace nnhip;

extern "C" size_t nnhip_eval_expr_workspace_bytes(const nnhip_expr_program* prog, size_t rows, size_t cols)
{
    return layout(*prog, rows, cols).total * sizeof(float) + 256;
}

extern "C" int nnhip_eval_expr(const nnhip_expr_program* prog, const float* const* inputs, float* out, size_t rows,
                               size_t cols, int vector_out, void* workspace, void* stream)
{
    const nnhip_expr_program& p = *prog;
    if (p.n_instrs == 0 || p.n_instrs > 64 || p.n_views > 8 || p.n_consts > 16) return -2;
    if (auto v = nn::validate_expr_spec(to_spec(p), p.n_views); !v) return -2;
    const nn::ExprSpec spec = to_spec(p);
    const int raxis = nn::expr_spec_reduce_axis(spec);
    if (vector_out && raxis != 0 && raxis != 1) return -2;
    if (rows == 0 || cols == 0) return 0;
    if (rows * cols > (size_t{1} << 40)) return -1;

    auto s = static_cast<hipStream_t>(stream);
    const Layout L = layout(p, rows, cols);
    float* ws = static_cast<float*>(workspace);
    ExprArgs A;
    std::memset(&A, 0, sizeof(A));
    for (unsigned j = 0; j < p.n_instrs; ++j)
        for (unsigned b = 0; b < 8; ++b) A.instrs[j][b >> 2] |= static_cast<unsigned>(p.instrs[j][b]) << (8 * (b & 3));
    for (unsigned q = 0; q < p.n_consts; ++q) A.consts[q] = p.consts[q];
    A.n_instrs = p.n_instrs;
    A.rows = rows;
    A.cols = cols;
    for (unsigned k = 0; k < p.n_views; ++k)
    {
        A.view[k].in = inputs[k];
        A.view[k].param = p.view_param[k];
        A.view[k].kind = p.view_kind[k];
        A.view[k].negate = p.view_negate[k];
    }

    // 1. reduce views (an input that appears twice with the same view is reduced once).
    for (unsigned k = 0; k < p.n_views; ++k)
    {
        const unsigned char v = p.view_kind[k];
        if (v < V_COLSUM || v > V_ROWMAX) continue;
        float* dst = ws + L.view_off[k];
        A.view[k].vred = dst;
        bool reused = false;
        for (unsigned q = 0; q < k; ++q)
            if (p.view_kind[q] == v && inputs[q] == inputs[k])
            {
                A.view[k].vred = A.view[q].vred;
                reused = true;
                break;
            }
        if (reused) continue;
        const unsigned mode = (v == V_COLMAX || v == V_ROWMAX) ? 1u : 0u;
        int rc = (v >= V_ROWSUM) ? nnhip_reduce_row(inputs[k], dst, rows, cols, mode, stream)
                                 : nnhip_reduce_col(inputs[k], dst, rows, cols, mode, ws + L.part_off, stream);
        if (rc) return rc;
    }
    // 2. reduce instructions, in program order.
    for (unsigned j = 0; j < p.n_instrs; ++j)
    {
        const unsigned char op = p.instrs[j][0], dst = p.instrs[j][1];
        if (op < E_COLSUM) continue;
        const bool col = op == E_COLSUM || op == E_COLMAX;
        const int is_max = (op == E_COLMAX || op == E_ROWMAX) ? 1 : 0;
        float* vec = ws + L.rvec_off[dst];
        if (col)
        {
            const Chunks ch = col_chunks(rows, cols);
            const unsigned cb = static_cast<unsigned>((cols + kThreads - 1) / kThreads);
            hipLaunchKernelGGL(k_expr_reduce_cols, dim3(cb, static_cast<unsigned>(ch.chunks)), dim3(kThreads), 0, s, A,
                               j, ws + L.part_off, ch.rows_per_chunk, is_max);
            hipLaunchKernelGGL(k_expr_merge_cols, dim3(cb), dim3(kThreads), 0, s, ws + L.part_off, vec, ch.chunks, cols,
                               is_max);
        }
        else
        {
            hipLaunchKernelGGL(k_expr_reduce_rows, dim3(grid_for(rows, 4, 1u << 30)), dim3(kThreads), 0, s, A, j, vec,
                               is_max);
        }
        if (int rc = launch_status()) return rc;
        // Later instructions read this vector through Reduce operands.
        A.rvec[dst] = vec;
        A.raxis[dst] = col ? 1 : 0;
    }
    // 3. output.
    if (vector_out)
    {
        const bool row_axis = raxis == 0;
        const unsigned char lop = p.instrs[p.n_instrs - 1][0];
        if (!(lop >= E_COLSUM))
        {
            // The output chain must reach inputs only through reduce / broadcast views
            // (cpu_engine.hpp:1583-1642).
            bool needed[16] = {};
            needed[p.instrs[p.n_instrs - 1][1]] = true;
            for (int ii = static_cast<int>(p.n_instrs) - 1; ii >= 0; --ii)
            {
                const unsigned char* in = p.instrs[ii];
                if (!needed[in[1]] || in[0] >= E_COLSUM) continue;
                const size_t nops = nn::expr_instr_num_operands(static_cast<nn::ExprOp>(in[0]));
                for (size_t q = 0; q < nops; ++q)
                {
                    const unsigned char kind = in[2 + 2 * q], idx = in[3 + 2 * q];
                    if (kind == K_INPUT)
                    {
                        const unsigned char v = p.view_kind[idx];
                        if (!((v >= V_COLSUM && v <= V_ROWMAX) || v == V_ROWBC || v == V_COLBC)) return -4;
                    }
                    else if (kind == K_REG || kind == K_FANOUT || kind == K_REDUCE)
                        needed[idx] = true;
                }
            }
        }
        const size_t len = row_axis ? rows : cols;
        hipLaunchKernelGGL(k_expr_vector, dim3(grid_for(len, kThreads, 1u << 30)), dim3(kThreads), 0, s, A, out, len,
                           row_axis ? 1 : 0);
    }
    else
    {
        hipLaunchKernelGGL(k_expr_elementwise, dim3(grid_for(rows * cols, kThreads, 256 * 64)), dim3(kThreads), 0, s, A,
                           out);
    }
    return launch_status();
}
