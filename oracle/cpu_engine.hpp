// ORACLE — test infrastructure only. Nothing in the product links this.
// Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it,
// and only as the checker / CPU baseline.
//
// cpu_engine.hpp — a CPU restatement of the reference CpuEngine
// (/root/reference/include/neuralnet.cpp/cpu_engine.hpp) implementing the same
// nn::ComputeEngine interface as the HIP engine, so the GPT layers run
// unchanged over either engine. Semantics, loop orders and error checks follow
// the reference function by function (line numbers below). The fused
// attention / cross-entropy / eval_expr primitives are serial loops, exactly
// as in the reference.
#pragma once

#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>
#include <string>
#include <vector>

#include "cpu_algebra.hpp"
#include "nn/compute_engine.hpp"

namespace nn::oracle
{

// Float-encoded row index: valid iff static_cast<size_t>(f) < rows for the
// values where that cast is defined (f > -1, finite, < 2^64). Values in
// (-1, 0) truncate to row 0 as in the reference cast.
inline bool row_index(float f, std::size_t rows, std::size_t& out)
{
    if (!(f > -1.0f) || !(f < 1.8446744e19f)) return false;
    const auto r = static_cast<std::size_t>(f);
    if (r >= rows) return false;
    out = r;
    return true;
}

inline float op_max(float a, float b) { return (a < b) ? b : a; }   // std::max
inline float op_min(float a, float b) { return (b < a) ? b : a; }   // std::min

inline float apply_binary(BinaryOp op, float a, float b)
{
    switch (op)
    {
    case BinaryOp::Add: return a + b;
    case BinaryOp::Sub: return a - b;
    case BinaryOp::Mul: return a * b;
    case BinaryOp::Div: return a / b;
    case BinaryOp::Max: return op_max(a, b);
    case BinaryOp::Min: return op_min(a, b);
    }
    return 0.0f;
}

inline float apply_unary(UnaryOp op, float x)
{
    switch (op)
    {
    case UnaryOp::Neg: return -x;
    case UnaryOp::Exp: return std::exp(x);
    case UnaryOp::Log: return std::log(x);
    case UnaryOp::Sqrt: return std::sqrt(x);
    case UnaryOp::Rsqrt: return 1.0f / std::sqrt(x);
    case UnaryOp::Abs: return std::fabs(x);
    case UnaryOp::Tanh: return std::tanh(x);
    }
    return 0.0f;
}

class CpuEngine final : public ComputeEngine
{
    static constexpr float kNegInf = -std::numeric_limits<float>::infinity();

    static const float* P(const Tensor& t) { return t.cpu_matrix().data(); }
    static float* W(Tensor& t) { return t.cpu_matrix().data(); }
    static Result<void> need_cpu(std::initializer_list<const Tensor*> ts)
    {
        for (const Tensor* t : ts)
            if (t && !t->is_cpu()) return fail("CpuEngine: GPU tensor on CPU engine");
        return {};
    }

    // Logical batched dims (reference cpu_engine.hpp:357-366 and repeats).
    struct BDims
    {
        std::size_t M, K, N;
    };
    static Result<BDims> bdims(const Tensor& A, const Tensor& B, std::size_t batch, bool tA, bool tB,
                               const char* who)
    {
        if (batch == 0) return fail(std::string(who) + ": batch must be > 0");
        if (A.rows() % batch != 0 || B.rows() % batch != 0)
            return fail(std::string(who) + ": rows not divisible by batch");
        const std::size_t ar = A.rows() / batch, br = B.rows() / batch;
        BDims d{tA ? A.cols() : ar, tA ? ar : A.cols(), tB ? br : B.cols()};
        const std::size_t K2 = tB ? B.cols() : br;
        if (d.K != K2) return fail(std::string(who) + ": K dimension mismatch");
        return d;
    }

public:
    Device device() const noexcept override { return Device::CPU; }
    Result<void> begin_batch() override { return {}; }
    Result<void> end_batch() override { return {}; }
    Result<void> flush_batch() override { return {}; }
    Result<void> begin_expr() override { return {}; }
    Result<void> end_expr() override { return {}; }

    // reference :40-72
    Tensor create_tensor(std::size_t rows, std::size_t cols) override { return Tensor::cpu(rows, cols); }
    Result<Tensor> from_matrix(const Matrix& m) override { return Tensor::from_matrix(Matrix(m)); }
    Result<Matrix> to_matrix(const Tensor& t) override
    {
        if (!t.is_cpu()) return fail("to_matrix: tensor is not CPU");
        return Matrix(t.cpu_matrix());
    }
    Result<void> copy_from(Tensor& dst, const Matrix& src) override
    {
        if (!dst.is_cpu()) return fail("copy_from: dst tensor is not CPU");
        if (dst.rows() != src.rows() || dst.cols() != src.cols()) return fail("copy_from: shape mismatch");
        dst.cpu_matrix() = src;
        return {};
    }
    Result<Tensor> clone(const Tensor& src) override
    {
        if (!src.is_cpu()) return fail("clone: src tensor is not CPU");
        return Tensor::from_matrix(Matrix(src.cpu_matrix()));
    }

    // reference :75-114
    Result<Tensor> slice_rows(const Tensor& src, std::size_t start, std::size_t count) override
    {
        if (!src.is_cpu()) return fail("slice_rows: src tensor is not CPU");
        if (start + count > src.rows()) return fail("slice_rows: range out of bounds");
        Matrix r(count, src.cols());
        std::memcpy(r.data(), P(src) + start * src.cols(), count * src.cols() * sizeof(float));
        return Tensor::from_matrix(std::move(r));
    }
    Result<void> insert_rows(Tensor& dst, std::size_t start, const Tensor& src) override
    {
        if (!dst.is_cpu() || !src.is_cpu()) return fail("insert_rows: tensors are not CPU");
        if (dst.cols() != src.cols()) return fail("insert_rows: column count mismatch");
        if (start + src.rows() > dst.rows()) return fail("insert_rows: range out of bounds");
        std::memcpy(W(dst) + start * dst.cols(), P(src), src.size() * sizeof(float));
        return {};
    }

    // reference :125-179 (out-of-range index -> zero row)
    Result<Tensor> gather_rows(const Tensor& table, const Tensor& indices) override
    {
        if (!table.is_cpu() || !indices.is_cpu()) return fail("gather_rows: tensors are not CPU");
        const std::size_t V = table.rows(), D = table.cols(), n = indices.size();
        Matrix out(n, D);
        const float* t = P(table);
        const float* idx = P(indices);
        for (std::size_t i = 0; i < n; ++i)
        {
            std::size_t r;
            if (row_index(idx[i], V, r)) std::memcpy(out.data() + i * D, t + r * D, D * sizeof(float));
            else std::fill_n(out.data() + i * D, D, 0.0f);
        }
        return Tensor::from_matrix(std::move(out));
    }
    // reference :184-216: dst[idx[i]] += grad[i], serially in i order.
    Result<void> scatter_add_rows(Tensor& dst, const Tensor& indices, const Tensor& grad) override
    {
        if (!dst.is_cpu() || !indices.is_cpu() || !grad.is_cpu()) return fail("scatter_add_rows: tensors are not CPU");
        if (dst.cols() != grad.cols()) return fail("scatter_add_rows: column count mismatch");
        const std::size_t V = dst.rows(), D = dst.cols(), n = indices.size();
        if (grad.rows() < n) return fail("scatter_add_rows: grad has fewer rows than indices");
        float* d = W(dst);
        const float* idx = P(indices);
        const float* g = P(grad);
        for (std::size_t i = 0; i < n; ++i)
        {
            std::size_t r;
            if (!row_index(idx[i], V, r)) continue;
            for (std::size_t c = 0; c < D; ++c) d[r * D + c] += g[i * D + c];
        }
        return {};
    }

    // reference :226-279
    Result<Tensor> rearrange_3d(const Tensor& x, std::size_t M, std::size_t B, std::size_t N, bool inverse) override
    {
        NN_CHECK(need_cpu({&x}));
        if (x.size() != M * B * N) return fail("rearrange_3d: element count mismatch");
        Matrix out(inverse ? M : B * M, inverse ? B * N : N);
        const float* s = P(x);
        float* d = out.data();
        for (std::size_t b = 0; b < B; ++b)
            for (std::size_t m = 0; m < M; ++m)
            {
                const std::size_t a = (b * M + m) * N, c = m * (B * N) + b * N;
                std::memcpy(d + (inverse ? c : a), s + (inverse ? a : c), N * sizeof(float));
            }
        return Tensor::from_matrix(std::move(out));
    }
    // reference :282-287
    Result<Tensor> transpose(const Tensor& A) override
    {
        NN_CHECK(need_cpu({&A}));
        Matrix out(A.cols(), A.rows());
        oracle::transpose(P(A), out.data(), A.rows(), A.cols());
        return Tensor::from_matrix(std::move(out));
    }

    // reference :293-331
    Result<Tensor> matmul(const Tensor& A, const Tensor& B, bool tA, bool tB) override
    {
        NN_CHECK(need_cpu({&A, &B}));
        const std::size_t M = tA ? A.cols() : A.rows(), K = tA ? A.rows() : A.cols();
        const std::size_t K2 = tB ? B.cols() : B.rows(), N = tB ? B.rows() : B.cols();
        if (K != K2)
            return fail("matmul: dimension mismatch A=" + std::to_string(A.rows()) + "x" + std::to_string(A.cols()) +
                        " B=" + std::to_string(B.rows()) + "x" + std::to_string(B.cols()));
        Matrix C(M, N);
        gemm(C.data(), M, N, K, P(A), A.cols(), tA, P(B), B.cols(), tB);
        return Tensor::from_matrix(std::move(C));
    }

    // reference :335-419 (alpha applied after the product when != 1)
    Result<Tensor> batched_matmul(const Tensor& A, const Tensor& B, std::size_t batch, bool tA, bool tB,
                                  Scalar alpha) override
    {
        NN_CHECK(need_cpu({&A, &B}));
        NN_TRY(d, bdims(A, B, batch, tA, tB, "batched_matmul"));
        Matrix C(batch * d.M, d.N);
        const std::size_t as = A.rows() / batch * A.cols(), bs = B.rows() / batch * B.cols();
        for (std::size_t b = 0; b < batch; ++b)
            gemm(C.data() + b * d.M * d.N, d.M, d.N, d.K, P(A) + b * as, A.cols(), tA, P(B) + b * bs, B.cols(), tB);
        if (alpha != 1.0f)
            for (auto& v : C.span()) v *= alpha;
        return Tensor::from_matrix(std::move(C));
    }

private:
    // Scalar dot of the fused primitives (reference :393-408): k ascending.
    static float fdot(const float* a, const float* b, std::size_t M, std::size_t K, std::size_t N, bool tA, bool tB,
                      std::size_t bi, std::size_t i, std::size_t j)
    {
        float s = 0.0f;
        const std::size_t ab = bi * M * K, bb = bi * K * N;
        for (std::size_t k = 0; k < K; ++k)
        {
            const float av = !tA ? a[ab + i * K + k] : a[ab + k * M + i];
            const float bv = !tB ? b[bb + k * N + j] : b[bb + j * K + k];
            s += av * bv;
        }
        return s;
    }
    static Result<void> mask_ok(const Tensor* mask, std::size_t M, std::size_t N, const char* who)
    {
        if (mask && (mask->rows() != M || mask->cols() != N)) return fail(std::string(who) + ": mask shape mismatch");
        if (mask && !mask->is_cpu()) return fail("CpuEngine: GPU tensor on CPU engine");
        return {};
    }
    static Result<void> vec_ok(const Tensor& t, std::size_t rows, const char* who, const char* what)
    {
        if (t.rows() != rows || t.cols() != 1) return fail(std::string(who) + ": " + what + " shape mismatch");
        return {};
    }

public:
    // reference :426-532
    Result<Tensor> batched_matmul_reduce(const Tensor& A, const Tensor& B, std::size_t batch, ReduceOp op, bool tA,
                                         bool tB, Scalar alpha, bool reduce_cols, const Tensor* mask) override
    {
        NN_CHECK(need_cpu({&A, &B}));
        NN_TRY(d, bdims(A, B, batch, tA, tB, "batched_matmul_reduce"));
        NN_CHECK(mask_ok(mask, d.M, d.N, "batched_matmul_reduce"));
        const float* a = P(A);
        const float* b = P(B);
        const float* mk = mask ? P(*mask) : nullptr;
        const float init = op == ReduceOp::Max ? std::numeric_limits<float>::lowest()
                           : op == ReduceOp::Min ? std::numeric_limits<float>::max()
                                                 : 0.0f;
        auto combine = [op](float acc, float v) {
            return op == ReduceOp::Max ? op_max(acc, v) : op == ReduceOp::Min ? op_min(acc, v) : acc + v;
        };
        const bool skip = op == ReduceOp::Sum || op == ReduceOp::Min;
        const std::size_t outer = reduce_cols ? d.M : d.N, inner = reduce_cols ? d.N : d.M;
        Matrix out(reduce_cols ? batch * d.M : batch, reduce_cols ? 1 : d.N);
        for (std::size_t bi = 0; bi < batch; ++bi)
            for (std::size_t o = 0; o < outer; ++o)
            {
                float acc = init;
                for (std::size_t q = 0; q < inner; ++q)
                {
                    const std::size_t i = reduce_cols ? o : q, j = reduce_cols ? q : o;
                    const float mv = mk ? mk[i * d.N + j] : 0.0f;
                    if (skip && mv == kNegInf) continue;
                    acc = combine(acc, alpha * fdot(a, b, d.M, d.K, d.N, tA, tB, bi, i, j) + mv);
                }
                out.data()[bi * outer + o] = acc;
            }
        return Tensor::from_matrix(std::move(out));
    }

    // reference :535-604
    Result<Tensor> batched_matmul_softmax_denom(const Tensor& A, const Tensor& B, const Tensor& row_max,
                                                std::size_t batch, bool tA, bool tB, Scalar alpha,
                                                const Tensor* mask) override
    {
        NN_CHECK(need_cpu({&A, &B, &row_max}));
        NN_TRY(d, bdims(A, B, batch, tA, tB, "batched_matmul_softmax_denom"));
        NN_CHECK(vec_ok(row_max, batch * d.M, "batched_matmul_softmax_denom", "row_max"));
        NN_CHECK(mask_ok(mask, d.M, d.N, "batched_matmul_softmax_denom"));
        const float *a = P(A), *b = P(B), *m = P(row_max);
        const float* mk = mask ? P(*mask) : nullptr;
        Matrix out(batch * d.M, 1);
        for (std::size_t bi = 0; bi < batch; ++bi)
            for (std::size_t i = 0; i < d.M; ++i)
            {
                const float mval = m[bi * d.M + i];
                float acc = 0.0f;
                for (std::size_t j = 0; j < d.N; ++j)
                {
                    const float mv = mk ? mk[i * d.N + j] : 0.0f;
                    if (mv == kNegInf) continue;
                    acc += std::exp(alpha * fdot(a, b, d.M, d.K, d.N, tA, tB, bi, i, j) + mv - mval);
                }
                out.data()[bi * d.M + i] = acc;
            }
        return Tensor::from_matrix(std::move(out));
    }

    // reference :607-699
    Result<Tensor> batched_matmul_softmax_apply(const Tensor& A, const Tensor& B, const Tensor& V,
                                                const Tensor& row_max, const Tensor& denom, std::size_t batch,
                                                bool tA, bool tB, Scalar alpha, const Tensor* mask) override
    {
        NN_CHECK(need_cpu({&A, &B, &V, &row_max, &denom}));
        if (batch != 0 && V.rows() % batch != 0)
            return fail("batched_matmul_softmax_apply: rows not divisible by batch");
        NN_TRY(d, bdims(A, B, batch, tA, tB, "batched_matmul_softmax_apply"));
        if (V.rows() / batch != d.N) return fail("batched_matmul_softmax_apply: V rows per batch != N");
        NN_CHECK(vec_ok(row_max, batch * d.M, "batched_matmul_softmax_apply", "row_max"));
        NN_CHECK(vec_ok(denom, batch * d.M, "batched_matmul_softmax_apply", "denom"));
        NN_CHECK(mask_ok(mask, d.M, d.N, "batched_matmul_softmax_apply"));
        const std::size_t D = V.cols();
        const float *a = P(A), *b = P(B), *v = P(V), *m = P(row_max), *l = P(denom);
        const float* mk = mask ? P(*mask) : nullptr;
        Matrix out(batch * d.M, D);
        std::vector<float> w(d.N);
        for (std::size_t bi = 0; bi < batch; ++bi)
            for (std::size_t i = 0; i < d.M; ++i)
            {
                const float mval = m[bi * d.M + i], inv_l = 1.0f / l[bi * d.M + i];
                for (std::size_t j = 0; j < d.N; ++j)
                {
                    const float mv = mk ? mk[i * d.N + j] : 0.0f;
                    w[j] = mv == kNegInf
                               ? 0.0f
                               : std::exp(alpha * fdot(a, b, d.M, d.K, d.N, tA, tB, bi, i, j) + mv - mval) * inv_l;
                }
                for (std::size_t k = 0; k < D; ++k)
                {
                    float acc = 0.0f;
                    for (std::size_t j = 0; j < d.N; ++j) acc += w[j] * v[(bi * d.N + j) * D + k];
                    out.data()[(bi * d.M + i) * D + k] = acc;
                }
            }
        return Tensor::from_matrix(std::move(out));
    }

    // reference :702-801
    Result<Tensor> batched_matmul_softmax_backward_q(const Tensor& A, const Tensor& B, const Tensor& Pm,
                                                     const Tensor& row_max, const Tensor& denom, std::size_t batch,
                                                     bool tA, bool tB, Scalar alpha, Tensor& r_out,
                                                     const Tensor* mask) override
    {
        NN_CHECK(need_cpu({&A, &B, &Pm, &row_max, &denom}));
        NN_TRY(d, bdims(A, B, batch, tA, tB, "batched_matmul_softmax_backward_q"));
        if (Pm.rows() != batch * d.M || Pm.cols() != d.N)
            return fail("batched_matmul_softmax_backward_q: P shape mismatch");
        NN_CHECK(vec_ok(row_max, batch * d.M, "batched_matmul_softmax_backward_q", "row_max"));
        NN_CHECK(vec_ok(denom, batch * d.M, "batched_matmul_softmax_backward_q", "denom"));
        NN_CHECK(mask_ok(mask, d.M, d.N, "batched_matmul_softmax_backward_q"));
        const float *a = P(A), *b = P(B), *p = P(Pm), *m = P(row_max), *l = P(denom);
        const float* mk = mask ? P(*mask) : nullptr;
        Matrix out(batch * d.K, d.M), r(batch * d.M, 1);
        std::vector<float> w(d.N);
        for (std::size_t bi = 0; bi < batch; ++bi)
            for (std::size_t i = 0; i < d.M; ++i)
            {
                const std::size_t ri = bi * d.M + i;
                const float mval = m[ri], inv_l = 1.0f / l[ri];
                float rv = 0.0f;
                for (std::size_t j = 0; j < d.N; ++j)
                {
                    const float mv = mk ? mk[i * d.N + j] : 0.0f;
                    if (mv == kNegInf)
                    {
                        w[j] = 0.0f;
                        continue;
                    }
                    w[j] = std::exp(alpha * fdot(a, b, d.M, d.K, d.N, tA, tB, bi, i, j) + mv - mval) * inv_l;
                    rv += w[j] * p[ri * d.N + j];
                }
                r.data()[ri] = rv;
                for (std::size_t k = 0; k < d.K; ++k)
                {
                    float acc = 0.0f;
                    for (std::size_t j = 0; j < d.N; ++j)
                    {
                        const float bv = !tB ? b[(bi * d.K + k) * d.N + j] : b[(bi * d.N + j) * d.K + k];
                        acc += w[j] * (p[ri * d.N + j] - rv) * bv;
                    }
                    out.data()[(bi * d.K + k) * d.M + i] = alpha * acc;
                }
            }
        r_out = Tensor::from_matrix(std::move(r));
        return Tensor::from_matrix(std::move(out));
    }

    // reference :804-915
    Result<Tensor> batched_matmul_softmax_backward_kv(const Tensor& A, const Tensor& B, const Tensor& Pm,
                                                      const Tensor& G, const Tensor& R, const Tensor& row_max,
                                                      const Tensor& denom, std::size_t batch, bool tA, bool tB,
                                                      Scalar alpha, Tensor& grad_v_out, const Tensor* mask) override
    {
        NN_CHECK(need_cpu({&A, &B, &Pm, &G, &R, &row_max, &denom}));
        NN_TRY(d, bdims(A, B, batch, tA, tB, "batched_matmul_softmax_backward_kv"));
        if (Pm.rows() != batch * d.M || Pm.cols() != d.N)
            return fail("batched_matmul_softmax_backward_kv: P shape mismatch");
        if (G.rows() != batch * d.M) return fail("batched_matmul_softmax_backward_kv: G rows != batch*M");
        NN_CHECK(vec_ok(R, batch * d.M, "batched_matmul_softmax_backward_kv", "R"));
        NN_CHECK(vec_ok(row_max, batch * d.M, "batched_matmul_softmax_backward_kv", "row_max"));
        NN_CHECK(vec_ok(denom, batch * d.M, "batched_matmul_softmax_backward_kv", "denom"));
        NN_CHECK(mask_ok(mask, d.M, d.N, "batched_matmul_softmax_backward_kv"));
        const std::size_t D = G.cols();
        if (D < d.K) return fail("batched_matmul_softmax_backward_kv: G cols < K");
        const float *a = P(A), *b = P(B), *p = P(Pm), *g = P(G), *rr = P(R), *m = P(row_max), *l = P(denom);
        const float* mk = mask ? P(*mask) : nullptr;
        Matrix out(batch * d.K, d.N), gv(batch * d.K, d.N);
        std::vector<float> w(d.M);
        for (std::size_t bi = 0; bi < batch; ++bi)
            for (std::size_t j = 0; j < d.N; ++j)
            {
                for (std::size_t i = 0; i < d.M; ++i)
                {
                    const float mv = mk ? mk[i * d.N + j] : 0.0f;
                    const std::size_t ri = bi * d.M + i;
                    w[i] = mv == kNegInf
                               ? 0.0f
                               : std::exp(alpha * fdot(a, b, d.M, d.K, d.N, tA, tB, bi, i, j) + mv - m[ri]) / l[ri];
                }
                for (std::size_t k = 0; k < d.K; ++k)
                {
                    float accK = 0.0f, accV = 0.0f;
                    for (std::size_t i = 0; i < d.M; ++i)
                    {
                        const std::size_t ri = bi * d.M + i;
                        const float av = !tA ? a[(bi * d.M + i) * d.K + k] : a[(bi * d.K + k) * d.M + i];
                        accK += w[i] * (p[ri * d.N + j] - rr[ri]) * av;
                        accV += w[i] * g[ri * D + k];
                    }
                    out.data()[(bi * d.K + k) * d.N + j] = alpha * accK;
                    gv.data()[(bi * d.K + k) * d.N + j] = accV;
                }
            }
        grad_v_out = Tensor::from_matrix(std::move(gv));
        return Tensor::from_matrix(std::move(out));
    }

    // reference :922-945
    Result<Tensor> col_softmax_denom(const Tensor& logits, const Tensor& col_max) override
    {
        NN_CHECK(need_cpu({&logits, &col_max}));
        const std::size_t C = logits.rows(), N = logits.cols();
        if (col_max.rows() != 1 || col_max.cols() != N) return fail("col_softmax_denom: col_max shape mismatch");
        const float *L = P(logits), *m = P(col_max);
        Matrix out(1, N);
        for (std::size_t i = 0; i < N; ++i)
        {
            float acc = 0.0f;
            for (std::size_t r = 0; r < C; ++r) acc += std::exp(L[r * N + i] - m[i]);
            out.data()[i] = acc;
        }
        return Tensor::from_matrix(std::move(out));
    }

    // reference :948-1006
    Result<Tensor> col_softmax_sparse_forward(const Tensor& logits, const Tensor& labels, const Tensor* mask,
                                              std::size_t vocab, Scalar inv, Tensor& loss_vec_out) override
    {
        NN_CHECK(need_cpu({&logits, &labels, mask}));
        if (vocab > (std::size_t{1} << 24))
            return fail("col_softmax_sparse_forward: vocab_size exceeds 2^24 (float labels not exactly representable)");
        const std::size_t C = logits.rows(), N = logits.cols();
        if (labels.rows() != 1 || labels.cols() != N) return fail("col_softmax_sparse_forward: labels shape mismatch");
        if (vocab > C) return fail("col_softmax_sparse_forward: vocab_size > classes");
        if (mask && (mask->rows() != 1 || mask->cols() != N))
            return fail("col_softmax_sparse_forward: mask shape mismatch");
        const float *L = P(logits), *lb = P(labels);
        const float* mk = mask ? P(*mask) : nullptr;
        Matrix grad(C, N), lv(1, N);
        float* g = grad.data();
        for (std::size_t i = 0; i < N; ++i)
        {
            const float f = lb[i];
            const std::size_t lbl = f >= 0.0f ? static_cast<std::size_t>(f) : 0;
            const bool valid = (!mk || mk[i] >= 0.5f) && lbl < vocab;
            if (!valid)
            {
                for (std::size_t r = 0; r < C; ++r) g[r * N + i] = 0.0f;
                lv.data()[i] = 0.0f;
                continue;
            }
            float mx = -std::numeric_limits<float>::infinity();
            for (std::size_t r = 0; r < C; ++r) mx = op_max(mx, L[r * N + i]);
            float den = 0.0f;
            for (std::size_t r = 0; r < C; ++r) den += std::exp(L[r * N + i] - mx);
            for (std::size_t r = 0; r < C; ++r) g[r * N + i] = inv * std::exp(L[r * N + i] - mx) / den;
            g[lbl * N + i] -= inv;
            lv.data()[i] = L[lbl * N + i] - mx - std::log(den);
        }
        loss_vec_out = Tensor::from_matrix(std::move(lv));
        return Tensor::from_matrix(std::move(grad));
    }

    // reference :1008-1044
    Result<void> add_inplace(Tensor& A, const Tensor& B) override
    {
        if (A.rows() != B.rows() || A.cols() != B.cols()) return fail("add_inplace: shape mismatch");
        float* a = W(A);
        const float* b = P(B);
        for_range(A.size(), [&](std::size_t i) { a[i] = a[i] + b[i]; });
        return {};
    }
    Result<void> scale_inplace(Tensor& A, Scalar s) override
    {
        float* a = W(A);
        for_range(A.size(), [&](std::size_t i) { a[i] = a[i] * s; });
        return {};
    }
    Result<void> axpy_inplace(Tensor& A, Scalar s, const Tensor& B) override
    {
        if (A.rows() != B.rows() || A.cols() != B.cols()) return fail("axpy_inplace: shape mismatch");
        float* a = W(A);
        const float* b = P(B);
        for_range(A.size(), [&](std::size_t i) { a[i] = a[i] + s * b[i]; });
        return {};
    }
    Result<void> zero(Tensor& A) override
    {
        A.cpu_matrix().zero();
        return {};
    }

    // reference :1050-1086
    Result<Tensor> row_reduce_sum(const Tensor& A) override
    {
        Matrix o(A.rows(), 1);
        row_reduce(P(A), o.data(), A.rows(), A.cols(), 0.0f, [](float x, float y) { return x + y; });
        return Tensor::from_matrix(std::move(o));
    }
    Result<Tensor> col_reduce_sum(const Tensor& A) override
    {
        Matrix o(1, A.cols());
        col_reduce(P(A), o.data(), A.rows(), A.cols(), 0.0f, [](float x, float y) { return x + y; });
        return Tensor::from_matrix(std::move(o));
    }
    Result<Tensor> row_reduce_max(const Tensor& A) override
    {
        Matrix o(A.rows(), 1);
        row_reduce(P(A), o.data(), A.rows(), A.cols(), std::numeric_limits<float>::lowest(), op_max);
        return Tensor::from_matrix(std::move(o));
    }
    Result<Tensor> col_reduce_max(const Tensor& A) override
    {
        Matrix o(1, A.cols());
        col_reduce(P(A), o.data(), A.rows(), A.cols(), std::numeric_limits<float>::lowest(), op_max);
        return Tensor::from_matrix(std::move(o));
    }

    // reference :1092-1125 (shape checked as the reference Matrix asserts do)
    Result<void> broadcast_row_inplace(Tensor& A, const Tensor& v, BinaryOp op) override
    {
        if (v.rows() != A.rows() || v.cols() != 1) return fail("broadcast_row_inplace: row_vec shape mismatch");
        float* a = W(A);
        const float* b = P(v);
        const std::size_t C = A.cols();
        for_range(A.size(), [&](std::size_t i) { a[i] = apply_binary(op, a[i], b[i / C]); });
        return {};
    }
    Result<void> broadcast_col_inplace(Tensor& A, const Tensor& v, BinaryOp op) override
    {
        if (v.rows() != 1 || v.cols() != A.cols()) return fail("broadcast_col_inplace: col_vec shape mismatch");
        float* a = W(A);
        const float* b = P(v);
        const std::size_t C = A.cols();
        for_range(A.size(), [&](std::size_t i) { a[i] = apply_binary(op, a[i], b[i % C]); });
        return {};
    }

    // reference :1131-1215
    Result<Tensor> elementwise_unary(UnaryOp op, const Tensor& A) override
    {
        Matrix o(A.rows(), A.cols());
        const float* a = P(A);
        float* out = o.data();
        for_range(A.size(), [&](std::size_t i) { out[i] = apply_unary(op, a[i]); });
        return Tensor::from_matrix(std::move(o));
    }
    Result<Tensor> elementwise_binary(BinaryOp op, const Tensor& A, const Tensor& B) override
    {
        if (A.rows() != B.rows() || A.cols() != B.cols()) return fail("elementwise_binary: shape mismatch");
        Matrix o(A.rows(), A.cols());
        const float *a = P(A), *b = P(B);
        float* out = o.data();
        for_range(A.size(), [&](std::size_t i) { out[i] = apply_binary(op, a[i], b[i]); });
        return Tensor::from_matrix(std::move(o));
    }
    Result<Tensor> elementwise_binary_scalar(BinaryOp op, const Tensor& A, Scalar s, bool scalar_first) override
    {
        Matrix o(A.rows(), A.cols());
        const float* a = P(A);
        float* out = o.data();
        for_range(A.size(), [&](std::size_t i) { out[i] = scalar_first ? apply_binary(op, s, a[i]) : apply_binary(op, a[i], s); });
        return Tensor::from_matrix(std::move(o));
    }
    // reference :1221-1266
    Result<Tensor> elementwise_select_scalar_cond(CompareOp cmp, const Tensor& A, Scalar sb, const Tensor& T,
                                                  Scalar se) override
    {
        if (A.rows() != T.rows() || A.cols() != T.cols()) return fail("elementwise_select: A and then shape mismatch");
        Matrix o(A.rows(), A.cols());
        const float *a = P(A), *t = P(T);
        float* out = o.data();
        for (std::size_t i = 0; i < A.size(); ++i)
        {
            bool c = false;
            switch (cmp)
            {
            case CompareOp::Lt: c = a[i] < sb; break;
            case CompareOp::Le: c = a[i] <= sb; break;
            case CompareOp::Gt: c = a[i] > sb; break;
            case CompareOp::Ge: c = a[i] >= sb; break;
            case CompareOp::Eq: c = a[i] == sb; break;
            case CompareOp::Ne: c = a[i] != sb; break;
            }
            out[i] = c ? t[i] : se;
        }
        return Tensor::from_matrix(std::move(o));
    }

    Result<Tensor> eval_expr(const ExprSpec& spec, std::span<const Tensor> inputs, std::size_t rows,
                             std::size_t cols) override
    {
        return eval_expr_impl(spec, inputs, rows, cols, false);
    }
    Result<Tensor> eval_expr_reduce(const ExprSpec& spec, std::span<const Tensor> inputs, std::size_t rows,
                                    std::size_t cols) override
    {
        return eval_expr_impl(spec, inputs, rows, cols, true);
    }

private:
    static float eval_instr(ExprOp op, float va, float vb, float vc)
    {
        switch (op)
        {
        case ExprOp::Neg: return -va;
        case ExprOp::Exp: return std::exp(va);
        case ExprOp::Log: return std::log(va);
        case ExprOp::Sqrt: return std::sqrt(va);
        case ExprOp::Rsqrt: return 1.0f / std::sqrt(va);
        case ExprOp::Abs: return std::fabs(va);
        case ExprOp::Tanh: return std::tanh(va);
        case ExprOp::Add: return va + vb;
        case ExprOp::Sub: return va - vb;
        case ExprOp::Mul: return va * vb;
        case ExprOp::Div: return va / vb;
        case ExprOp::Max: return op_max(va, vb);
        case ExprOp::Min: return op_min(va, vb);
        case ExprOp::Lt: return va < vb ? 1.0f : 0.0f;
        case ExprOp::Le: return va <= vb ? 1.0f : 0.0f;
        case ExprOp::Gt: return va > vb ? 1.0f : 0.0f;
        case ExprOp::Ge: return va >= vb ? 1.0f : 0.0f;
        case ExprOp::Eq: return va == vb ? 1.0f : 0.0f;
        case ExprOp::Ne: return va != vb ? 1.0f : 0.0f;
        case ExprOp::Select: return va != 0.0f ? vb : vc;
        default: return 0.0f;
        }
    }

    // reference :1298-1659
    Result<Tensor> eval_expr_impl(const ExprSpec& spec, std::span<const Tensor> inputs, std::size_t rows,
                                  std::size_t cols, bool vector_out)
    {
        NN_CHECK(validate_expr_spec(spec, inputs.size()));
        const int raxis = vector_out ? expr_spec_reduce_axis(spec) : -1;
        if (vector_out && raxis != 0 && raxis != 1)
            return fail("eval_expr_reduce: expression must reduce along rows or along columns");
        const bool vec_is_row = raxis == 0;

        std::vector<const float*> data(inputs.size());
        for (std::size_t k = 0; k < inputs.size(); ++k)
        {
            const Tensor& t = inputs[k];
            if (!t.is_cpu()) return fail("eval_expr: input not CPU");
            const ExprView& v = spec.views[k];
            switch (static_cast<ExprViewKind>(v.kind))
            {
            case ExprViewKind::RotateHalf:
                if (t.rows() != rows || t.cols() != cols || v.param == 0 || rows % v.param != 0 || v.param % 2 != 0)
                    return fail("eval_expr: RotateHalf shape/param invalid");
                break;
            case ExprViewKind::RowMod:
                if (t.rows() != v.param || t.cols() != cols || v.param == 0 || rows % v.param != 0)
                    return fail("eval_expr: RowMod shape/param invalid");
                break;
            case ExprViewKind::RowBroadcast:
                if (t.rows() != rows || t.cols() != 1) return fail("eval_expr: RowBroadcast input must be (rows,1)");
                break;
            case ExprViewKind::ColBroadcast:
                if (t.rows() != 1 || t.cols() != cols) return fail("eval_expr: ColBroadcast input must be (1,cols)");
                break;
            default:
                if (t.rows() != rows || t.cols() != cols)
                    return fail("eval_expr: Linear/reduce input shape mismatch");
                break;
            }
            data[k] = P(t);
        }

        const std::size_t n = rows * cols;
        if (n == 0)   // the reference returns the (rows, cols) shape here even for vector output
            return Tensor::from_matrix(Matrix(rows, cols));

        // Reduce views: one scalar per row / column, computed first.
        std::vector<std::vector<float>> vred(inputs.size());
        for (std::size_t k = 0; k < inputs.size(); ++k)
        {
            const auto kind = static_cast<ExprViewKind>(spec.views[k].kind);
            if (!expr_view_is_reduce(kind)) continue;
            const bool is_row = expr_view_reduces_rows(kind);
            const bool is_max = kind == ExprViewKind::RowReduceMax || kind == ExprViewKind::ColReduceMax;
            auto& acc = vred[k];
            acc.assign(is_row ? rows : cols, is_max ? std::numeric_limits<float>::lowest() : 0.0f);
            const float* s = data[k];
            if (is_row)
            {
                for (std::size_t r = 0; r < rows; ++r)
                    for (std::size_t c = 0; c < cols; ++c)
                        acc[r] = is_max ? op_max(acc[r], s[r * cols + c]) : acc[r] + s[r * cols + c];
            }
            else
            {
                for (std::size_t c = 0; c < cols; ++c)
                    for (std::size_t r = 0; r < rows; ++r)
                        acc[c] = is_max ? op_max(acc[c], s[r * cols + c]) : acc[c] + s[r * cols + c];
            }
        }

        auto read_input = [&](std::size_t k, std::size_t r, std::size_t c) -> float {
            const ExprView& v = spec.views[k];
            const float* s = data[k];
            switch (static_cast<ExprViewKind>(v.kind))
            {
            case ExprViewKind::RotateHalf:
            {
                const std::size_t blk = v.param, rl = r % blk;
                const std::size_t rr = (r / blk) * blk + (rl < blk / 2 ? rl + blk / 2 : rl - blk / 2);
                const float val = s[rr * cols + c];
                return (v.negate_first_half && rl < blk / 2) ? -val : val;
            }
            case ExprViewKind::RowMod: return s[(r % v.param) * cols + c];
            case ExprViewKind::RowReduceSum:
            case ExprViewKind::RowReduceMax: return vred[k][r];
            case ExprViewKind::ColReduceSum:
            case ExprViewKind::ColReduceMax: return vred[k][c];
            case ExprViewKind::RowBroadcast: return s[r];
            case ExprViewKind::ColBroadcast: return s[c];
            default: return s[r * cols + c];
            }
        };

        std::vector<std::vector<float>> rvec(EXPR_MAX_REGS);
        std::vector<std::uint8_t> raxis_of(EXPR_MAX_REGS, 0);   // 1 = per column, 0 = per row

        // Evaluates the elementwise instructions [0, upto) at (r, c) into regs.
        auto run_prefix = [&](std::size_t upto, std::size_t r, std::size_t c, float* regs) {
            auto opnd = [&](const ExprOperand& o) -> float {
                switch (static_cast<ExprOperandKind>(o.kind))
                {
                case ExprOperandKind::Const: return spec.consts[o.idx];
                case ExprOperandKind::Input: return read_input(o.idx, r, c);
                case ExprOperandKind::Reduce: return rvec[o.idx][raxis_of[o.idx] ? c : r];
                default: return regs[o.idx];
                }
            };
            for (std::size_t j = 0; j < upto; ++j)
            {
                const ExprInstr& J = spec.instrs[j];
                const auto op = static_cast<ExprOp>(J.op);
                if (expr_op_is_reduce(op)) continue;
                const std::size_t no = expr_instr_num_operands(op);
                const float va = opnd(J.a);
                const float vb = no >= 2 ? opnd(J.b) : 0.0f;
                const float vc = no >= 3 ? opnd(J.c) : 0.0f;
                regs[J.dst] = eval_instr(op, va, vb, vc);
            }
        };

        // Reduce instructions in instruction order, each replaying the prefix
        // over the full grid in row-major order (reference :1442-1522).
        for (std::size_t ri = 0; ri < spec.instrs.size(); ++ri)
        {
            const ExprInstr& R = spec.instrs[ri];
            const auto rop = static_cast<ExprOp>(R.op);
            if (!expr_op_is_reduce(rop)) continue;
            const bool is_col = expr_op_reduces_cols(rop);
            const bool is_max = rop == ExprOp::ColMax || rop == ExprOp::RowMax;
            raxis_of[R.dst] = is_col ? 1 : 0;
            auto& acc = rvec[R.dst];
            acc.assign(is_col ? cols : rows, is_max ? std::numeric_limits<float>::lowest() : 0.0f);
            for (std::size_t i = 0; i < n; ++i)
            {
                const std::size_t r = i / cols, c = i % cols;
                float regs[EXPR_MAX_REGS] = {};
                run_prefix(ri, r, c, regs);
                float v;
                switch (static_cast<ExprOperandKind>(R.a.kind))
                {
                case ExprOperandKind::Const: v = spec.consts[R.a.idx]; break;
                case ExprOperandKind::Input: v = read_input(R.a.idx, r, c); break;
                case ExprOperandKind::Reduce: v = rvec[R.a.idx][raxis_of[R.a.idx] ? c : r]; break;
                default: v = regs[R.a.idx]; break;
                }
                float& slot = acc[is_col ? c : r];
                slot = is_max ? op_max(slot, v) : slot + v;
            }
        }

        const ExprInstr& last = spec.instrs.back();
        const bool last_is_reduce = expr_op_is_reduce(static_cast<ExprOp>(last.op));
        auto element = [&](std::size_t r, std::size_t c) {
            float regs[EXPR_MAX_REGS] = {};
            run_prefix(spec.instrs.size(), r, c, regs);
            return regs[last.dst];
        };

        if (vector_out)
        {
            const std::size_t len = vec_is_row ? rows : cols;
            Matrix o(vec_is_row ? rows : 1, vec_is_row ? 1 : cols);
            if (last_is_reduce)
            {
                std::copy_n(rvec[last.dst].begin(), len, o.data());
                return Tensor::from_matrix(std::move(o));
            }
            // The output chain must read inputs only through reduce / broadcast
            // views so that it is constant along the reduced axis (reference :1583-1642).
            std::vector<std::uint8_t> needed(EXPR_MAX_REGS, 0);
            needed[last.dst] = 1;
            for (std::size_t ii = spec.instrs.size(); ii-- > 0;)
            {
                const ExprInstr& in = spec.instrs[ii];
                if (!needed[in.dst] || expr_op_is_reduce(static_cast<ExprOp>(in.op))) continue;
                const ExprOperand* ops[3] = {&in.a, &in.b, &in.c};
                const std::size_t no = expr_instr_num_operands(static_cast<ExprOp>(in.op));
                for (std::size_t q = 0; q < no; ++q)
                {
                    const ExprOperand& o2 = *ops[q];
                    const auto k = static_cast<ExprOperandKind>(o2.kind);
                    if (k == ExprOperandKind::Input)
                    {
                        const auto vk = static_cast<ExprViewKind>(spec.views[o2.idx].kind);
                        if (!expr_view_is_reduce(vk) && !expr_view_is_broadcast(vk))
                            return fail("eval_expr_reduce: output chain reads an input directly; "
                                        "the output is not constant along the reduced axis");
                    }
                    else if (k == ExprOperandKind::Reg || k == ExprOperandKind::Fanout ||
                             k == ExprOperandKind::Reduce)
                        needed[o2.idx] = 1;
                }
            }
            for (std::size_t k = 0; k < len; ++k)
                o.data()[k] = element(vec_is_row ? k : 0, vec_is_row ? 0 : k);
            return Tensor::from_matrix(std::move(o));
        }

        Matrix out(rows, cols);
        for (std::size_t i = 0; i < n; ++i)
        {
            const std::size_t r = i / cols, c = i % cols;
            out.data()[i] = last_is_reduce ? rvec[last.dst][raxis_of[last.dst] ? c : r] : element(r, c);
        }
        return Tensor::from_matrix(std::move(out));
    }
};

} // namespace nn::oracle
