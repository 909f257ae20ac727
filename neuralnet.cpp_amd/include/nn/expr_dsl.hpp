// expr_dsl.hpp — inline-math front end that folds into an ExprSpec.
//
// Layers write ordinary expressions (leaf(x) * col_broadcast(r), exp(...),
// row_reduce_sum(...)) and call dsl::compute / dsl::compute_reduce. The
// expression tree is folded into a flat ExprSpec (left operand before right,
// so the structural key is stable, as in reference expr_dsl.hpp:258-265) and
// handed to engine.eval_expr. On a CPU engine, expressions with no
// reduction/broadcast node are evaluated directly from the tree instead
// (reference expr_dsl.hpp:464-475); the arithmetic order is the same either way.
//
// Fold rules (reference expr_dsl.hpp:46-117, 188-220):
//   * every leaf or view is a new input slot, even for the same tensor;
//   * row_/col_reduce_*(Tensor) is a reduce VIEW; row_/col_reduce_*(expr) is a
//     reduce INSTRUCTION read back through a Reduce operand;
//   * a scalar operand becomes a new constant-pool entry.
#pragma once

#include <cmath>
#include <cstdint>
#include <utility>
#include <vector>

#include "compute_engine.hpp"
#include "expr_spec.hpp"
#include "tensor.hpp"

namespace nn::dsl
{

struct SpecBuilder
{
    ExprSpec spec;
    std::vector<Tensor> inputs;

    ExprOperand constant(Scalar v)
    {
        spec.consts.push_back(v);
        return expr::cst(static_cast<std::uint8_t>(spec.consts.size() - 1));
    }
    ExprOperand input(const Tensor& t, ExprView view)
    {
        spec.views.push_back(view);
        inputs.push_back(t);
        return expr::input(static_cast<std::uint8_t>(inputs.size() - 1));
    }
    ExprOperand instr(ExprOp op, ExprOperand a, ExprOperand b = {}, ExprOperand c = {})
    {
        ExprInstr in;
        in.op = static_cast<std::uint8_t>(op);
        in.dst = static_cast<std::uint8_t>(spec.num_regs++);
        in.a = a;
        in.b = b;
        in.c = c;
        spec.instrs.push_back(in);
        return expr_op_is_reduce(op) ? expr::reduce(in.dst) : expr::reg(in.dst);
    }
};

// ── op tags: host arithmetic (used by the CPU tree evaluation) + op id ─────
namespace op
{
#define NN_DSL_UNARY_TAG(Name, expr_)                                            \
    struct Name                                                                  \
    {                                                                            \
        static Scalar apply(Scalar a) noexcept { return expr_; }                 \
        static constexpr ExprOp id = ExprOp::Name;                               \
    };
NN_DSL_UNARY_TAG(Neg, -a)
NN_DSL_UNARY_TAG(Exp, std::exp(a))
NN_DSL_UNARY_TAG(Log, std::log(a))
NN_DSL_UNARY_TAG(Sqrt, std::sqrt(a))
NN_DSL_UNARY_TAG(Rsqrt, Scalar{1} / std::sqrt(a))
NN_DSL_UNARY_TAG(Abs, std::fabs(a))
NN_DSL_UNARY_TAG(Tanh, std::tanh(a))
#undef NN_DSL_UNARY_TAG

#define NN_DSL_BINARY_TAG(Name, expr_)                                           \
    struct Name                                                                  \
    {                                                                            \
        static Scalar apply(Scalar a, Scalar b) noexcept { return expr_; }       \
        static constexpr ExprOp id = ExprOp::Name;                               \
    };
NN_DSL_BINARY_TAG(Add, a + b)
NN_DSL_BINARY_TAG(Sub, a - b)
NN_DSL_BINARY_TAG(Mul, a * b)
NN_DSL_BINARY_TAG(Div, a / b)
NN_DSL_BINARY_TAG(Max, (a < b) ? b : a)
NN_DSL_BINARY_TAG(Min, (b < a) ? b : a)
NN_DSL_BINARY_TAG(Lt, (a < b) ? Scalar{1} : Scalar{0})
NN_DSL_BINARY_TAG(Le, (a <= b) ? Scalar{1} : Scalar{0})
NN_DSL_BINARY_TAG(Gt, (a > b) ? Scalar{1} : Scalar{0})
NN_DSL_BINARY_TAG(Ge, (a >= b) ? Scalar{1} : Scalar{0})
NN_DSL_BINARY_TAG(Eq, (a == b) ? Scalar{1} : Scalar{0})
NN_DSL_BINARY_TAG(Ne, (a != b) ? Scalar{1} : Scalar{0})
#undef NN_DSL_BINARY_TAG
} // namespace op

// ── nodes ──────────────────────────────────────────────────────────────────
// Every node has: eval(i) for the CPU tree path, fold(SpecBuilder&), and
// `engine_only` (true when the node needs eval_expr semantics: reductions or
// broadcast views, which a flat per-element walk cannot express).

struct ConstNode
{
    Scalar v;
    static constexpr bool engine_only = false;
    Scalar eval(std::size_t) const noexcept { return v; }
    ExprOperand fold(SpecBuilder& b) const { return b.constant(v); }
};

struct LeafNode
{
    Tensor t;
    static constexpr bool engine_only = false;
    Scalar eval(std::size_t i) const { return t.cpu_matrix().span()[i]; }
    ExprOperand fold(SpecBuilder& b) const { return b.input(t, expr::linear()); }
};

struct RotateHalfNode
{
    Tensor t;
    std::uint32_t block;
    static constexpr bool engine_only = false;
    Scalar eval(std::size_t i) const
    {
        const std::size_t cols = t.cols(), r = i / cols, c = i % cols;
        const std::size_t half = block / 2, rl = r % block;
        const std::size_t src = (r / block) * block + (rl < half ? rl + half : rl - half);
        const Scalar v = t.cpu_matrix().span()[src * cols + c];
        return rl < half ? -v : v;
    }
    ExprOperand fold(SpecBuilder& b) const { return b.input(t, expr::rotate_half(block, true)); }
};

struct RowModNode
{
    Tensor t;
    std::uint32_t mod;
    static constexpr bool engine_only = false;
    Scalar eval(std::size_t i) const
    {
        const std::size_t cols = t.cols(), r = i / cols, c = i % cols;
        return t.cpu_matrix().span()[(r % mod) * cols + c];
    }
    ExprOperand fold(SpecBuilder& b) const { return b.input(t, expr::row_mod(mod)); }
};

// Reduce views and broadcast views of a tensor.
template <ExprViewKind K>
struct ViewNode
{
    Tensor t;
    static constexpr bool engine_only = true;
    Scalar eval(std::size_t) const noexcept { return Scalar{0}; }
    ExprOperand fold(SpecBuilder& b) const
    {
        ExprView v;
        v.kind = static_cast<std::uint8_t>(K);
        return b.input(t, v);
    }
};

template <class Op, class C>
struct UnaryNode
{
    C c;
    static constexpr bool engine_only = C::engine_only;
    Scalar eval(std::size_t i) const { return Op::apply(c.eval(i)); }
    ExprOperand fold(SpecBuilder& b) const { return b.instr(Op::id, c.fold(b)); }
};

template <class Op, class L, class R>
struct BinaryNode
{
    L l;
    R r;
    static constexpr bool engine_only = L::engine_only || R::engine_only;
    Scalar eval(std::size_t i) const { return Op::apply(l.eval(i), r.eval(i)); }
    ExprOperand fold(SpecBuilder& b) const
    {
        const ExprOperand lo = l.fold(b);   // left first: fixes the key
        const ExprOperand ro = r.fold(b);
        return b.instr(Op::id, lo, ro);
    }
};

template <class C, class T, class E>
struct SelectNode
{
    C c;
    T t;
    E e;
    static constexpr bool engine_only = C::engine_only || T::engine_only || E::engine_only;
    Scalar eval(std::size_t i) const { return c.eval(i) != Scalar{0} ? t.eval(i) : e.eval(i); }
    ExprOperand fold(SpecBuilder& b) const
    {
        const ExprOperand co = c.fold(b);
        const ExprOperand to = t.fold(b);
        const ExprOperand eo = e.fold(b);
        return b.instr(ExprOp::Select, co, to, eo);
    }
};

template <class C, ExprOp R>
struct ReduceNode
{
    C c;
    static constexpr bool engine_only = true;
    Scalar eval(std::size_t) const noexcept { return Scalar{0}; }
    ExprOperand fold(SpecBuilder& b) const { return b.instr(R, c.fold(b)); }
};

template <class T>
concept Node = requires(const T& t, SpecBuilder& b) {
    { t.fold(b) } -> std::same_as<ExprOperand>;
    { T::engine_only } -> std::convertible_to<bool>;
};

// ── constructors ──────────────────────────────────────────────────────────
inline LeafNode leaf(Tensor t) { return {std::move(t)}; }
inline RotateHalfNode rotate_half(Tensor t, std::uint32_t block) { return {std::move(t), block}; }
inline RowModNode row_mod(Tensor t, std::uint32_t mod) { return {std::move(t), mod}; }

inline ViewNode<ExprViewKind::RowReduceSum> row_reduce_sum(Tensor t) { return {std::move(t)}; }
inline ViewNode<ExprViewKind::RowReduceMax> row_reduce_max(Tensor t) { return {std::move(t)}; }
inline ViewNode<ExprViewKind::ColReduceSum> col_reduce_sum(Tensor t) { return {std::move(t)}; }
inline ViewNode<ExprViewKind::ColReduceMax> col_reduce_max(Tensor t) { return {std::move(t)}; }
inline ViewNode<ExprViewKind::RowBroadcast> row_broadcast(Tensor t) { return {std::move(t)}; }
inline ViewNode<ExprViewKind::ColBroadcast> col_broadcast(Tensor t) { return {std::move(t)}; }

template <Node E> ReduceNode<E, ExprOp::RowSum> row_reduce_sum(const E& e) { return {e}; }
template <Node E> ReduceNode<E, ExprOp::RowMax> row_reduce_max(const E& e) { return {e}; }
template <Node E> ReduceNode<E, ExprOp::ColSum> col_reduce_sum(const E& e) { return {e}; }
template <Node E> ReduceNode<E, ExprOp::ColMax> col_reduce_max(const E& e) { return {e}; }

template <Node E> UnaryNode<op::Neg, E> neg(const E& e) { return {e}; }
template <Node E> UnaryNode<op::Exp, E> exp(const E& e) { return {e}; }
template <Node E> UnaryNode<op::Log, E> log(const E& e) { return {e}; }
template <Node E> UnaryNode<op::Sqrt, E> sqrt(const E& e) { return {e}; }
template <Node E> UnaryNode<op::Rsqrt, E> rsqrt(const E& e) { return {e}; }
template <Node E> UnaryNode<op::Abs, E> abs(const E& e) { return {e}; }
template <Node E> UnaryNode<op::Tanh, E> tanh(const E& e) { return {e}; }
template <Node E> UnaryNode<op::Neg, E> operator-(const E& e) { return {e}; }

template <Node L, Node R> BinaryNode<op::Max, L, R> max(const L& l, const R& r) { return {l, r}; }
template <Node L, Node R> BinaryNode<op::Min, L, R> min(const L& l, const R& r) { return {l, r}; }
template <Node E> BinaryNode<op::Max, E, ConstNode> max(const E& e, Scalar s) { return {e, ConstNode{s}}; }
template <Node E> BinaryNode<op::Min, E, ConstNode> min(const E& e, Scalar s) { return {e, ConstNode{s}}; }

template <Node C, Node T, Node E> SelectNode<C, T, E> select(const C& c, const T& t, const E& e) { return {c, t, e}; }
template <Node C, Node T> SelectNode<C, T, ConstNode> select(const C& c, const T& t, Scalar e)
{
    return {c, t, ConstNode{e}};
}

#define NN_DSL_OPERATOR(SYM, Tag)                                                                  \
    template <Node L, Node R> BinaryNode<op::Tag, L, R> operator SYM(const L& l, const R& r)       \
    {                                                                                              \
        return {l, r};                                                                             \
    }                                                                                              \
    template <Node L> BinaryNode<op::Tag, L, ConstNode> operator SYM(const L& l, Scalar s)         \
    {                                                                                              \
        return {l, ConstNode{s}};                                                                  \
    }                                                                                              \
    template <Node R> BinaryNode<op::Tag, ConstNode, R> operator SYM(Scalar s, const R& r)         \
    {                                                                                              \
        return {ConstNode{s}, r};                                                                  \
    }
NN_DSL_OPERATOR(+, Add)
NN_DSL_OPERATOR(-, Sub)
NN_DSL_OPERATOR(*, Mul)
NN_DSL_OPERATOR(/, Div)
NN_DSL_OPERATOR(<, Lt)
NN_DSL_OPERATOR(<=, Le)
NN_DSL_OPERATOR(>, Gt)
NN_DSL_OPERATOR(>=, Ge)
NN_DSL_OPERATOR(==, Eq)
NN_DSL_OPERATOR(!=, Ne)
#undef NN_DSL_OPERATOR

// ── fold + evaluate ───────────────────────────────────────────────────────
template <Node E>
std::pair<ExprSpec, std::vector<Tensor>> to_expr_spec(const E& e)
{
    SpecBuilder b;
    (void)e.fold(b);
    return {std::move(b.spec), std::move(b.inputs)};
}

template <Node E>
Tensor eval_cpu(const E& e, std::size_t rows, std::size_t cols)
{
    Matrix out(rows, cols);
    auto sp = out.span();
    for (std::size_t i = 0; i < sp.size(); ++i)
        sp[i] = e.eval(i);
    return Tensor::from_matrix(std::move(out));
}

// Evaluate to a (rows, cols) tensor.
template <Node E>
Result<Tensor> compute(ComputeEngine& eng, const E& e, std::size_t rows, std::size_t cols)
{
    if constexpr (!E::engine_only)
    {
        if (eng.device() == Device::CPU)
            return eval_cpu(e, rows, cols);
    }
    auto [spec, inputs] = to_expr_spec(e);
    if (auto v = validate_expr_spec(spec, inputs.size()); !v)
        return unexpected(v.error());
    return eng.eval_expr(spec, inputs, rows, cols);
}

// Evaluate to the reduced vector itself: (rows,1) for a row reduction,
// (1,cols) for a column reduction (reference expr_dsl.hpp:521-544).
template <Node E>
Result<Tensor> compute_reduce(ComputeEngine& eng, const E& e, std::size_t rows, std::size_t cols)
{
    auto [spec, inputs] = to_expr_spec(e);
    if (auto v = validate_expr_spec(spec, inputs.size()); !v)
        return unexpected(v.error());
    return eng.eval_expr_reduce(spec, inputs, rows, cols);
}

} // namespace nn::dsl
