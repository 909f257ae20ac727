// expr_spec.hpp — the flat elementwise/reduction program evaluated by eval_expr.
//
// This is an interchange format shared with the reference, so the op codes,
// operand kinds, view kinds, field layout, limits, validation rules and the
// structural key are kept identical to include/neuralnet.cpp/expr_spec.hpp:
//   ExprOp            :30-62     operand kinds :94-101   views :116-159
//   ExprInstr/ExprSpec:161-186   key (FNV-1a)  :262-306  limits :309-312
//   validate_expr_spec:316-390
// Semantics (reference cpu_engine.hpp:1298-1659):
//   * every input has a view (Linear, RotateHalf, RowMod, Row/ColReduce{Sum,Max},
//     Row/ColBroadcast); reduce views stand for a per-row/per-column vector;
//   * instructions run in order, each writing regs[dst];
//   * reduce instructions (ColSum/ColMax/RowSum/RowMax) produce a per-column or
//     per-row vector, read back only through Reduce operands;
//   * the output is regs[last.dst] (or, for eval_expr_reduce, the reduced vector).
#pragma once

#include <cstdint>
#include <cstdio>
#include <string>
#include <vector>

#include "core_errors.hpp"
#include "matrix.hpp"

namespace nn
{

enum class ExprOp : std::uint8_t
{
    Neg = 0, Exp = 1, Log = 2, Sqrt = 3, Rsqrt = 4, Abs = 5, Tanh = 6,
    Add = 7, Sub = 8, Mul = 9, Div = 10, Max = 11, Min = 12,
    Lt = 13, Le = 14, Gt = 15, Ge = 16, Eq = 17, Ne = 18,
    Select = 19,                // dst = (a != 0) ? b : c
    ColSum = 20, ColMax = 21,   // per-column vector (1, cols)
    RowSum = 22, RowMax = 23,   // per-row vector (rows, 1)
};

[[nodiscard]] constexpr bool expr_op_is_reduce(ExprOp op) noexcept
{
    return op == ExprOp::ColSum || op == ExprOp::ColMax || op == ExprOp::RowSum || op == ExprOp::RowMax;
}
[[nodiscard]] constexpr bool expr_op_reduces_cols(ExprOp op) noexcept
{
    return op == ExprOp::ColSum || op == ExprOp::ColMax;
}
[[nodiscard]] constexpr std::size_t expr_instr_num_operands(ExprOp op) noexcept
{
    if (op == ExprOp::Select) return 3;
    if (static_cast<std::uint8_t>(op) <= static_cast<std::uint8_t>(ExprOp::Tanh) || expr_op_is_reduce(op))
        return 1;
    return 2;
}

enum class ExprOperandKind : std::uint8_t
{
    Reg = 0,
    Input = 1,
    Const = 2,
    Fanout = 3,   // same meaning as Reg
    Reduce = 4,   // broadcast read of a reduce instruction's vector
};

struct ExprOperand
{
    std::uint8_t kind = 0;
    std::uint8_t idx = 0;
    friend bool operator==(const ExprOperand&, const ExprOperand&) = default;
};

enum class ExprViewKind : std::uint8_t
{
    Linear = 0,
    RotateHalf = 1,     // block-local half swap, first half negated (param = block rows)
    RowMod = 2,         // reads row r % param
    ColReduceSum = 3,
    ColReduceMax = 4,
    RowReduceSum = 5,
    RowReduceMax = 6,
    RowBroadcast = 7,   // input (rows,1)
    ColBroadcast = 8,   // input (1,cols)
};

[[nodiscard]] constexpr bool expr_view_is_reduce(ExprViewKind k) noexcept
{
    return k == ExprViewKind::ColReduceSum || k == ExprViewKind::ColReduceMax ||
           k == ExprViewKind::RowReduceSum || k == ExprViewKind::RowReduceMax;
}
[[nodiscard]] constexpr bool expr_view_reduces_rows(ExprViewKind k) noexcept
{
    return k == ExprViewKind::RowReduceSum || k == ExprViewKind::RowReduceMax;
}
[[nodiscard]] constexpr bool expr_view_is_broadcast(ExprViewKind k) noexcept
{
    return k == ExprViewKind::RowBroadcast || k == ExprViewKind::ColBroadcast;
}
[[nodiscard]] constexpr bool expr_view_has_runtime_param(ExprViewKind k) noexcept
{
    return k == ExprViewKind::RowMod || k == ExprViewKind::RotateHalf;
}

struct ExprView
{
    std::uint8_t kind = 0;
    std::uint8_t negate_first_half = 0;
    std::uint32_t param = 0;
    friend bool operator==(const ExprView&, const ExprView&) = default;
};

struct ExprInstr
{
    std::uint8_t op = 0;
    std::uint8_t dst = 0;
    ExprOperand a;
    ExprOperand b;
    ExprOperand c;
    friend bool operator==(const ExprInstr&, const ExprInstr&) = default;
};

struct ExprSpec
{
    std::vector<ExprInstr> instrs;
    std::vector<ExprView> views;
    std::vector<Scalar> consts;
    std::uint32_t num_regs = 0;
};

inline constexpr std::size_t EXPR_MAX_INPUTS = 8;
inline constexpr std::size_t EXPR_MAX_CONSTS = 16;
inline constexpr std::size_t EXPR_MAX_REGS = 16;
inline constexpr std::size_t EXPR_MAX_INSTRS = 64;

// -1 = no reduction, 0 = every reduction is along rows (row vectors),
// 1 = every reduction is along columns, -2 = mixed.
[[nodiscard]] inline int expr_spec_reduce_axis(const ExprSpec& s)
{
    int axis = -1;
    auto merge = [&axis](int a) {
        if (axis == -1) axis = a;
        else if (axis != a) axis = -2;
    };
    for (const auto& v : s.views)
    {
        const auto k = static_cast<ExprViewKind>(v.kind);
        if (expr_view_is_reduce(k)) merge(expr_view_reduces_rows(k) ? 0 : 1);
    }
    for (const auto& in : s.instrs)
    {
        const auto op = static_cast<ExprOp>(in.op);
        if (expr_op_is_reduce(op)) merge(expr_op_reduces_cols(op) ? 1 : 0);
    }
    return axis;
}

[[nodiscard]] inline bool expr_spec_equal(const ExprSpec& a, const ExprSpec& b)
{
    return a.instrs == b.instrs && a.views == b.views && a.consts == b.consts && a.num_regs == b.num_regs;
}

// Structural key: 64-bit FNV-1a over the byte fields in the reference's
// order (num_regs, instruction count, per-instruction op/dst/a/b/c, view
// count, per-view kind/negate/param (param skipped for RowMod/RotateHalf),
// constant count, constants), printed as 16 hex digits.
[[nodiscard]] inline std::string expr_spec_key(const ExprSpec& s)
{
    std::uint64_t h = 0xcbf29ce484222325ull;
    auto bytes = [&h](const void* p, std::size_t n) {
        const auto* b = static_cast<const unsigned char*>(p);
        for (std::size_t i = 0; i < n; ++i)
        {
            h ^= b[i];
            h *= 0x100000001b3ull;
        }
    };
    auto u32 = [&bytes](std::uint32_t v) { bytes(&v, 4); };
    u32(s.num_regs);
    u32(static_cast<std::uint32_t>(s.instrs.size()));
    for (const auto& in : s.instrs)
    {
        const std::uint8_t f[8] = {in.op, in.dst, in.a.kind, in.a.idx, in.b.kind, in.b.idx, in.c.kind, in.c.idx};
        bytes(f, 8);
    }
    u32(static_cast<std::uint32_t>(s.views.size()));
    for (const auto& v : s.views)
    {
        bytes(&v.kind, 1);
        bytes(&v.negate_first_half, 1);
        if (!expr_view_has_runtime_param(static_cast<ExprViewKind>(v.kind)))
            u32(v.param);
    }
    u32(static_cast<std::uint32_t>(s.consts.size()));
    for (Scalar c : s.consts)
        bytes(&c, sizeof(c));
    char buf[17];
    std::snprintf(buf, sizeof buf, "%016llx", static_cast<unsigned long long>(h));
    return buf;
}

[[nodiscard]] inline Result<void> validate_expr_spec(const ExprSpec& spec, std::size_t num_inputs)
{
    if (spec.instrs.empty()) return fail("validate_expr_spec: empty instruction list");
    if (spec.instrs.size() > EXPR_MAX_INSTRS) return fail("validate_expr_spec: too many instructions");
    if (spec.num_regs == 0 || spec.num_regs > EXPR_MAX_REGS) return fail("validate_expr_spec: invalid num_regs");
    if (num_inputs > EXPR_MAX_INPUTS) return fail("validate_expr_spec: too many inputs");
    if (spec.consts.size() > EXPR_MAX_CONSTS) return fail("validate_expr_spec: too many constants");
    if (spec.views.size() != num_inputs) return fail("validate_expr_spec: views count != inputs count");

    // Pass 1: ranges (reference expr_spec.hpp:331-348). Unknown op / operand /
    // view codes are rejected too; the reference would silently treat them as
    // register reads.
    for (const auto& ins : spec.instrs)
    {
        if (ins.op > static_cast<std::uint8_t>(ExprOp::RowMax)) return fail("validate_expr_spec: unknown op");
        if (ins.dst >= spec.num_regs) return fail("validate_expr_spec: dst reg out of range");
        const ExprOperand* ops[3] = {&ins.a, &ins.b, &ins.c};
        const std::size_t n = expr_instr_num_operands(static_cast<ExprOp>(ins.op));
        for (std::size_t i = 0; i < n; ++i)
        {
            const ExprOperand& o = *ops[i];
            if (o.kind > static_cast<std::uint8_t>(ExprOperandKind::Reduce))
                return fail("validate_expr_spec: unknown operand kind");
            const auto k = static_cast<ExprOperandKind>(o.kind);
            if ((k == ExprOperandKind::Reg || k == ExprOperandKind::Fanout) && o.idx >= spec.num_regs)
                return fail("validate_expr_spec: src reg out of range");
            if (k == ExprOperandKind::Input && o.idx >= num_inputs)
                return fail("validate_expr_spec: input index out of range");
            if (k == ExprOperandKind::Const && o.idx >= spec.consts.size())
                return fail("validate_expr_spec: const index out of range");
        }
    }
    // Pass 2: reduce semantics (reference :356-388). The destination of the
    // current instruction is classified before its operands are checked.
    std::vector<std::uint8_t> is_reduce_dst(spec.num_regs, 0), is_elem_dst(spec.num_regs, 0);
    for (const auto& ins : spec.instrs)
    {
        const auto op = static_cast<ExprOp>(ins.op);
        (expr_op_is_reduce(op) ? is_reduce_dst : is_elem_dst)[ins.dst] = 1;
        const ExprOperand* ops[3] = {&ins.a, &ins.b, &ins.c};
        const std::size_t n = expr_instr_num_operands(op);
        for (std::size_t i = 0; i < n; ++i)
        {
            const ExprOperand& o = *ops[i];
            const auto k = static_cast<ExprOperandKind>(o.kind);
            if (k == ExprOperandKind::Reduce)
            {
                if (o.idx >= spec.num_regs) return fail("validate_expr_spec: reduce ref out of range");
                if (o.idx == ins.dst) return fail("validate_expr_spec: reduce self-reference");
                if (!is_reduce_dst[o.idx] || is_elem_dst[o.idx])
                    return fail("validate_expr_spec: Reduce operand must reference a prior reduce instruction");
            }
            else if ((k == ExprOperandKind::Reg || k == ExprOperandKind::Fanout) && is_reduce_dst[o.idx])
            {
                return fail("validate_expr_spec: register ref to reduce dst (use Reduce operand)");
            }
        }
    }
    for (const auto& v : spec.views)
        if (v.kind > static_cast<std::uint8_t>(ExprViewKind::ColBroadcast))
            return fail("validate_expr_spec: unknown view kind");
    return {};
}

// Operand / view constructors (reference expr_spec.hpp:394-410).
namespace expr
{
constexpr ExprOperand reg(std::uint8_t r) { return {0, r}; }
constexpr ExprOperand input(std::uint8_t i) { return {1, i}; }
constexpr ExprOperand cst(std::uint8_t c) { return {2, c}; }
constexpr ExprOperand fanout(std::uint8_t r) { return {3, r}; }
constexpr ExprOperand reduce(std::uint8_t r) { return {4, r}; }
constexpr ExprView linear() { return {0, 0, 0}; }
constexpr ExprView rotate_half(std::uint32_t block_rows, bool negate_first_half = true)
{
    return {1, static_cast<std::uint8_t>(negate_first_half ? 1 : 0), block_rows};
}
constexpr ExprView row_mod(std::uint32_t modulo) { return {2, 0, modulo}; }
constexpr ExprView col_reduce_sum() { return {3, 0, 0}; }
constexpr ExprView col_reduce_max() { return {4, 0, 0}; }
constexpr ExprView row_reduce_sum() { return {5, 0, 0}; }
constexpr ExprView row_reduce_max() { return {6, 0, 0}; }
constexpr ExprView row_broadcast() { return {7, 0, 0}; }
constexpr ExprView col_broadcast() { return {8, 0, 0}; }
} // namespace expr

} // namespace nn
