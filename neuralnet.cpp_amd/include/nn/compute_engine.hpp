// compute_engine.hpp — the op-level engine interface (the drop-in boundary).
//
// Same virtual surface, argument meaning, defaults and op codes as the
// reference's nn::ComputeEngine (include/neuralnet.cpp/compute_engine.hpp:87-410).
// Default arguments live only on this base declaration, so callers go
// through ComputeEngine& exactly as the reference's layers do. Layers hold
// the algorithms; engines implement only these primitives.
//
// Shape conventions shared by every engine (reference :130-200):
//   * all tensors are row-major fp32; index tensors hold integers as floats;
//   * batched ops split A/B into `batch` consecutive row blocks;
//     A_b is (M,K), or (K,M) stored when transA; B_b is (K,N), or (N,K) when transB;
//   * masks are dense (M,N) float tensors shared by all batches:
//     -inf excludes a position, a finite value is added to the score.
#pragma once

#include <cstddef>
#include <cstdint>
#include <span>

#include "core_errors.hpp"
#include "expr_spec.hpp"
#include "tensor.hpp"

namespace nn
{

// Op codes keep the reference's numeric values (compute_engine.hpp:43-82);
// they are also the op ids of the kernel C-ABI.
enum class UnaryOp : std::uint32_t { Neg = 0, Exp = 1, Log = 2, Sqrt = 3, Rsqrt = 4, Abs = 5, Tanh = 6 };
enum class BinaryOp : std::uint32_t { Add = 0, Sub = 1, Mul = 2, Div = 3, Max = 4, Min = 5 };
enum class CompareOp : std::uint32_t { Lt = 0, Le = 1, Gt = 2, Ge = 3, Eq = 4, Ne = 5 };
enum class ReduceOp : std::uint32_t { Sum = 0, Max = 1, Min = 2 };

class ComputeEngine
{
public:
    virtual ~ComputeEngine() = default;

    [[nodiscard]] virtual Device device() const noexcept = 0;

    // Batch / expression regions (reference :93-118).
    [[nodiscard]] virtual Result<void> begin_batch() = 0;
    [[nodiscard]] virtual Result<void> end_batch() = 0;
    [[nodiscard]] virtual Result<void> begin_expr() = 0;
    [[nodiscard]] virtual Result<void> end_expr() = 0;
    [[nodiscard]] virtual Result<void> flush_batch() { return {}; }

    // Factories and transfers (reference :121-131).
    [[nodiscard]] virtual Tensor create_tensor(std::size_t rows, std::size_t cols) = 0;
    [[nodiscard]] virtual Result<Tensor> from_matrix(const Matrix& m) = 0;
    [[nodiscard]] virtual Result<Matrix> to_matrix(const Tensor& t) = 0;
    [[nodiscard]] virtual Result<void> copy_from(Tensor& dst, const Matrix& src) = 0;
    [[nodiscard]] virtual Result<Tensor> clone(const Tensor& src) = 0;

    // Row slices (reference :136-143).
    [[nodiscard]] virtual Result<Tensor> slice_rows(const Tensor& src, std::size_t start_row, std::size_t count) = 0;
    [[nodiscard]] virtual Result<void> insert_rows(Tensor& dst, std::size_t dst_start_row, const Tensor& src) = 0;

    // Row gather / scatter-add by float-encoded indices (reference :151-161).
    [[nodiscard]] virtual Result<Tensor> gather_rows(const Tensor& table, const Tensor& indices) = 0;
    [[nodiscard]] virtual Result<void> scatter_add_rows(Tensor& dst, const Tensor& indices, const Tensor& grad) = 0;

    // (M, B*N) <-> (B*M, N) (reference :170-172) and 2-D transpose (:175).
    [[nodiscard]] virtual Result<Tensor> rearrange_3d(const Tensor& x, std::size_t M, std::size_t B, std::size_t N,
                                                      bool inverse = false) = 0;
    [[nodiscard]] virtual Result<Tensor> transpose(const Tensor& A) = 0;

    // GEMMs (reference :182-199).
    [[nodiscard]] virtual Result<Tensor> matmul(const Tensor& A, const Tensor& B, bool transA = false,
                                                bool transB = false) = 0;
    [[nodiscard]] virtual Result<Tensor> batched_matmul(const Tensor& A, const Tensor& B, std::size_t batch,
                                                        bool transA = false, bool transB = false,
                                                        Scalar alpha = Scalar{1}) = 0;

    // Fused attention primitives (reference :217-276).
    [[nodiscard]] virtual Result<Tensor> batched_matmul_reduce(const Tensor& A, const Tensor& B, std::size_t batch,
                                                               ReduceOp op, bool transA, bool transB, Scalar alpha,
                                                               bool reduce_cols = true,
                                                               const Tensor* mask = nullptr) = 0;
    [[nodiscard]] virtual Result<Tensor> batched_matmul_softmax_denom(const Tensor& A, const Tensor& B,
                                                                      const Tensor& row_max, std::size_t batch,
                                                                      bool transA, bool transB, Scalar alpha,
                                                                      const Tensor* mask = nullptr) = 0;
    [[nodiscard]] virtual Result<Tensor> batched_matmul_softmax_apply(const Tensor& A, const Tensor& B,
                                                                      const Tensor& V, const Tensor& row_max,
                                                                      const Tensor& denom, std::size_t batch,
                                                                      bool transA, bool transB, Scalar alpha,
                                                                      const Tensor* mask = nullptr) = 0;
    [[nodiscard]] virtual Result<Tensor> batched_matmul_softmax_backward_q(
        const Tensor& A, const Tensor& B, const Tensor& P, const Tensor& row_max, const Tensor& denom,
        std::size_t batch, bool transA, bool transB, Scalar alpha, Tensor& r_out,
        const Tensor* mask = nullptr) = 0;
    [[nodiscard]] virtual Result<Tensor> batched_matmul_softmax_backward_kv(
        const Tensor& A, const Tensor& B, const Tensor& P, const Tensor& G, const Tensor& R,
        const Tensor& row_max, const Tensor& denom, std::size_t batch, bool transA, bool transB, Scalar alpha,
        Tensor& grad_v_out, const Tensor* mask = nullptr) = 0;

    // Column softmax primitives for cross-entropy (reference :289-303).
    [[nodiscard]] virtual Result<Tensor> col_softmax_denom(const Tensor& logits, const Tensor& col_max) = 0;
    [[nodiscard]] virtual Result<Tensor> col_softmax_sparse_forward(const Tensor& logits, const Tensor& labels,
                                                                    const Tensor* mask, std::size_t vocab_size,
                                                                    Scalar inv_num_valid,
                                                                    Tensor& loss_vec_out) = 0;

    // In-place updates (reference :306-316).
    [[nodiscard]] virtual Result<void> add_inplace(Tensor& A, const Tensor& B) = 0;
    [[nodiscard]] virtual Result<void> scale_inplace(Tensor& A, Scalar s) = 0;
    [[nodiscard]] virtual Result<void> axpy_inplace(Tensor& A, Scalar scalar, const Tensor& B) = 0;
    [[nodiscard]] virtual Result<void> zero(Tensor& A) = 0;

    // Reductions (reference :324-336).
    [[nodiscard]] virtual Result<Tensor> row_reduce_sum(const Tensor& A) = 0;
    [[nodiscard]] virtual Result<Tensor> col_reduce_sum(const Tensor& A) = 0;
    [[nodiscard]] virtual Result<Tensor> row_reduce_max(const Tensor& A) = 0;
    [[nodiscard]] virtual Result<Tensor> col_reduce_max(const Tensor& A) = 0;

    // Broadcasts (reference :344-350).
    [[nodiscard]] virtual Result<void> broadcast_row_inplace(Tensor& A, const Tensor& row_vec, BinaryOp op) = 0;
    [[nodiscard]] virtual Result<void> broadcast_col_inplace(Tensor& A, const Tensor& col_vec, BinaryOp op) = 0;

    // Elementwise (reference :357-378).
    [[nodiscard]] virtual Result<Tensor> elementwise_unary(UnaryOp op, const Tensor& A) = 0;
    [[nodiscard]] virtual Result<Tensor> elementwise_binary(BinaryOp op, const Tensor& A, const Tensor& B) = 0;
    [[nodiscard]] virtual Result<Tensor> elementwise_binary_scalar(BinaryOp op, const Tensor& A, Scalar s,
                                                                   bool scalar_first = false) = 0;
    [[nodiscard]] virtual Result<Tensor> elementwise_select_scalar_cond(CompareOp cmp, const Tensor& A,
                                                                        Scalar scalar_b, const Tensor& then_t,
                                                                        Scalar scalar_else) = 0;

    // Expression evaluation (reference :392-409).
    [[nodiscard]] virtual Result<Tensor> eval_expr(const ExprSpec& spec, std::span<const Tensor> inputs,
                                                   std::size_t rows, std::size_t cols) = 0;
    [[nodiscard]] virtual Result<Tensor> eval_expr_reduce(const ExprSpec& spec, std::span<const Tensor> inputs,
                                                          std::size_t rows, std::size_t cols)
    {
        (void)spec;
        (void)inputs;
        (void)rows;
        (void)cols;
        return fail("eval_expr_reduce: not supported by this engine");
    }

    // Queues everything t's values depend on, as a read through the engine
    // would, without waiting (engines that defer work; others have nothing
    // to do). No reference counterpart: the reference reads through to_matrix.
    [[nodiscard]] virtual Result<void> settle_for_read(const Tensor& t)
    {
        (void)t;
        return {};
    }
};

} // namespace nn
