// layer_exprs.hpp — the elementwise / reduction expressions of the GPT layers.
//
// One definition per expression, used both by the layers (compute_layer.hpp)
// to issue eval_expr / eval_expr_reduce and by the HIP engine to recognise
// those programs structurally and run a fused kernel for each (the role the
// reference's ahead-of-time fused shaders play, one per ExprSpec key:
// tools/scan_exprs.cpp, tools/gen_fused.cpp). Any other program still goes
// to the generic evaluator.
//
// Expression text follows the reference layers:
//   RMSNorm forward  compute_layer.hpp:733-754,  backward :772-795
//   Softmax forward  :840-844,                   backward :855-860
//   SwiGLU backward  :436-444
//   LayerNorm        forward :541-592, backward :601-660
//   RoPE             :884-984
#pragma once

#include "expr_dsl.hpp"

namespace nn::layer_exprs
{

// RMSNorm forward: column sum of squares, (F,N) -> (1,N).
inline auto rms_sum_sq(const Tensor& x) { return dsl::col_reduce_sum(dsl::leaf(x) * dsl::leaf(x)); }
// normed = x * colbcast(rms_inv).
inline auto rms_normalize(const Tensor& x, const Tensor& rms_inv) { return dsl::leaf(x) * dsl::col_broadcast(rms_inv); }
// out = normed * rowbcast(gamma).
inline auto rms_scale(const Tensor& normed, const Tensor& gamma) { return dsl::leaf(normed) * dsl::row_broadcast(gamma); }

// RMSNorm backward: m_raw = ColSum(g * gamma * normed) -> (1,N).
inline auto rms_bwd_colsum(const Tensor& g, const Tensor& gamma, const Tensor& normed)
{
    return dsl::col_reduce_sum(dsl::leaf(g) * dsl::row_broadcast(gamma) * dsl::leaf(normed));
}
// dx = (g * gamma - colbcast(m) * normed) * colbcast(rms_inv).
inline auto rms_bwd_dx(const Tensor& g, const Tensor& gamma, const Tensor& m, const Tensor& normed,
                       const Tensor& rms_inv)
{
    return (dsl::leaf(g) * dsl::row_broadcast(gamma) - dsl::col_broadcast(m) * dsl::leaf(normed)) *
           dsl::col_broadcast(rms_inv);
}
// grad_gamma increment = RowSum(g * gamma * normed) -> (F,1).
inline auto rms_bwd_rowsum(const Tensor& g, const Tensor& gamma, const Tensor& normed)
{
    return dsl::row_reduce_sum(dsl::leaf(g) * dsl::row_broadcast(gamma) * dsl::leaf(normed));
}

// Softmax over rows and its backward.
inline auto softmax_rows(const Tensor& x)
{
    return dsl::exp(dsl::leaf(x) - dsl::row_reduce_max(x)) /
           dsl::row_reduce_sum(dsl::exp(dsl::leaf(x) - dsl::row_reduce_max(x)));
}
inline auto softmax_rows_backward(const Tensor& y, const Tensor& g)
{
    return dsl::leaf(y) * (dsl::leaf(g) - dsl::row_reduce_sum(dsl::leaf(y) * dsl::leaf(g)));
}

// SwiGLU backward: grad_gate = g * up * (s * (1 + gate * (1 - s))), grad_up = g * gate * s.
inline auto swiglu_grad_gate(const Tensor& g, const Tensor& up, const Tensor& s, const Tensor& gate)
{
    const Scalar one{1};
    return dsl::leaf(g) * dsl::leaf(up) * (dsl::leaf(s) * (one + dsl::leaf(gate) * (one - dsl::leaf(s))));
}
inline auto swiglu_grad_up(const Tensor& g, const Tensor& gate, const Tensor& s)
{
    return dsl::leaf(g) * dsl::leaf(gate) * dsl::leaf(s);
}

// LayerNorm forward (reference compute_layer.hpp:541-592): mean_raw = ColSum(x);
// diff = x - colbcast(mean); var_raw = ColSum(diff*diff); normed = diff * colbcast(std_inv);
// out = normed * rowbcast(gamma) + rowbcast(beta).
inline auto ln_col_sum(const Tensor& x) { return dsl::col_reduce_sum(dsl::leaf(x)); }
inline auto ln_center(const Tensor& x, const Tensor& mean) { return dsl::leaf(x) - dsl::col_broadcast(mean); }
inline auto ln_sum_sq(const Tensor& diff) { return dsl::col_reduce_sum(dsl::leaf(diff) * dsl::leaf(diff)); }
inline auto ln_normalize(const Tensor& diff, const Tensor& std_inv)
{
    return dsl::leaf(diff) * dsl::col_broadcast(std_inv);
}
inline auto ln_affine(const Tensor& normed, const Tensor& gamma, const Tensor& beta)
{
    return dsl::leaf(normed) * dsl::row_broadcast(gamma) + dsl::row_broadcast(beta);
}
// LayerNorm backward (reference :601-660).
inline auto ln_bwd_colsum_g(const Tensor& g, const Tensor& gamma)
{
    return dsl::col_reduce_sum(dsl::leaf(g) * dsl::row_broadcast(gamma));
}
inline auto ln_bwd_colsum_gn(const Tensor& g, const Tensor& gamma, const Tensor& normed)
{
    return dsl::col_reduce_sum(dsl::leaf(g) * dsl::row_broadcast(gamma) * dsl::leaf(normed));
}
inline auto ln_bwd_dx(const Tensor& g, const Tensor& gamma, const Tensor& mean_g, const Tensor& normed,
                      const Tensor& mean_gn, const Tensor& std_inv)
{
    return (dsl::leaf(g) * dsl::row_broadcast(gamma) - dsl::col_broadcast(mean_g) -
            dsl::leaf(normed) * dsl::col_broadcast(mean_gn)) *
           dsl::col_broadcast(std_inv);
}
inline auto ln_bwd_rowsum_gn(const Tensor& g, const Tensor& gamma, const Tensor& normed)
{
    return dsl::row_reduce_sum(dsl::leaf(g) * dsl::row_broadcast(gamma) * dsl::leaf(normed));
}
inline auto ln_bwd_rowsum(const Tensor& g) { return dsl::row_reduce_sum(dsl::leaf(g)); }

// RoPE (reference :884-984): q*RowMod(cos) + RotateHalf(q)*RowMod(sin), its
// inverse rotation with Sub; RotateHalf negates the first half of each block.
inline auto rope_forward(const Tensor& q, const Tensor& cos, const Tensor& sin, std::uint32_t dk)
{
    return dsl::leaf(q) * dsl::row_mod(cos, dk) + dsl::rotate_half(q, dk) * dsl::row_mod(sin, dk);
}
inline auto rope_backward(const Tensor& q, const Tensor& cos, const Tensor& sin, std::uint32_t dk)
{
    return dsl::leaf(q) * dsl::row_mod(cos, dk) - dsl::rotate_half(q, dk) * dsl::row_mod(sin, dk);
}

} // namespace nn::layer_exprs
