"""The ExprSpec programs the GPT layers issue (compute_layer.hpp:733-795 RMSNorm,
:436-444 SwiGLU backward, :840-860 Softmax, :884-984 RoPE), built the way the expression DSL
folds them (left operand before right; every leaf or view is a new input
slot; reduce instructions are referenced through Reduce operands). The HIP
engine recognises exactly these programs and runs a fused kernel for each,
so tests and the bench built from them exercise those kernels; the generic
interpreter handles any other program and the shapes the fused kernels do
not take.

Each builder returns (spec, slots): `slots` names, per input slot, which
argument the caller passes there. ARGS lists each builder's arguments in the
parameter order of its C++ counterpart in include/nn/layer_exprs.hpp, whose
serialised programs the library exports (nnhip_layer_program): the tests
check that every program here equals the engine's, instruction for
instruction, so the fused-kernel tests cannot drift onto the interpreter.
"""
from nnengine import ExprSpec, cst, inp, red, reg


def rms_sum_sq():                        # ColSum(x*x) -> (1,N)
    s = ExprSpec()
    s.view("Linear"), s.view("Linear")
    r0 = s.ins("Mul", inp(0), inp(1))
    s.ins("ColSum", reg(r0))
    return s, ("x", "x")


def rms_normalize():                     # x * colbcast(rms_inv)
    s = ExprSpec()
    s.view("Linear"), s.view("ColBroadcast")
    s.ins("Mul", inp(0), inp(1))
    return s, ("x", "rinv")


def rms_scale():                         # normed * rowbcast(gamma)
    s = ExprSpec()
    s.view("Linear"), s.view("RowBroadcast")
    s.ins("Mul", inp(0), inp(1))
    return s, ("normed", "gamma")


def _g_gamma_n(s):
    s.view("Linear"), s.view("RowBroadcast"), s.view("Linear")
    r0 = s.ins("Mul", inp(0), inp(1))
    return s.ins("Mul", reg(r0), inp(2))


def rms_bwd_colsum():                    # ColSum(g*gamma*normed) -> (1,N)
    s = ExprSpec()
    s.ins("ColSum", reg(_g_gamma_n(s)))
    return s, ("g", "gamma", "normed")


def rms_bwd_rowsum():                    # RowSum(g*gamma*normed) -> (F,1)
    s = ExprSpec()
    s.ins("RowSum", reg(_g_gamma_n(s)))
    return s, ("g", "gamma", "normed")


def rms_bwd_dx():                        # (g*gamma - colbcast(m)*normed) * colbcast(rinv)
    s = ExprSpec()
    for v in ("Linear", "RowBroadcast", "ColBroadcast", "Linear", "ColBroadcast"):
        s.view(v)
    r0 = s.ins("Mul", inp(0), inp(1))
    r1 = s.ins("Mul", inp(2), inp(3))
    r2 = s.ins("Sub", reg(r0), reg(r1))
    s.ins("Mul", reg(r2), inp(4))
    return s, ("g", "gamma", "m", "normed", "rinv")


def swiglu_grad_gate():                  # g*up*(s*(1 + gate*(1 - s)))
    s = ExprSpec()
    for _ in range(5):
        s.view("Linear")
    c0, c1 = s.const(1.0), s.const(1.0)
    r0 = s.ins("Mul", inp(0), inp(1))
    r1 = s.ins("Sub", cst(c1), inp(4))
    r2 = s.ins("Mul", inp(3), reg(r1))
    r3 = s.ins("Add", cst(c0), reg(r2))
    r4 = s.ins("Mul", inp(2), reg(r3))
    s.ins("Mul", reg(r0), reg(r4))
    return s, ("g", "up", "s", "gate", "s")


def swiglu_grad_up():                    # g*gate*s
    s = ExprSpec()
    for _ in range(3):
        s.view("Linear")
    r0 = s.ins("Mul", inp(0), inp(1))
    s.ins("Mul", reg(r0), inp(2))
    return s, ("g", "gate", "s")


def softmax_rows():                      # exp(x - rowmax(x)) / RowSum(exp(x - rowmax(x)))
    s = ExprSpec()
    for v in ("Linear", "RowReduceMax", "Linear", "RowReduceMax"):
        s.view(v)
    r0 = s.ins("Sub", inp(0), inp(1))
    r1 = s.ins("Exp", reg(r0))
    r2 = s.ins("Sub", inp(2), inp(3))
    r3 = s.ins("Exp", reg(r2))
    r4 = s.ins("RowSum", reg(r3))
    s.ins("Div", reg(r1), red(r4))
    return s, ("x", "x", "x", "x")


def softmax_rows_backward():             # y * (g - RowSum(y*g))
    s = ExprSpec()
    for _ in range(4):
        s.view("Linear")
    r0 = s.ins("Mul", inp(2), inp(3))
    r1 = s.ins("RowSum", reg(r0))
    r2 = s.ins("Sub", inp(1), red(r1))
    s.ins("Mul", inp(0), reg(r2))
    return s, ("y", "g", "y", "g")


def rope(dk, backward=False):            # q*RowMod(cos) +/- RotateHalf(q)*RowMod(sin)  (compute_layer.hpp:884-984)
    s = ExprSpec()
    s.view("Linear"), s.view("RowMod", dk), s.view("RotateHalf", dk, 1), s.view("RowMod", dk)
    r0 = s.ins("Mul", inp(0), inp(1))
    r1 = s.ins("Mul", inp(2), inp(3))
    s.ins("Sub" if backward else "Add", reg(r0), reg(r1))
    return s, ("q", "cos", "q", "sin")


def rope_tables(dk, T):
    """(dk, T) cos / sin tables: rows j and j + dk/2 hold cos / sin(pos * 10000^(-2j/dk))."""
    import numpy as np
    half = dk // 2
    ang = np.arange(T)[None, :] / (10000.0 ** (2.0 * np.arange(half)[:, None] / dk))
    c = np.concatenate([np.cos(ang)] * 2).astype(np.float32)
    sn = np.concatenate([np.sin(ang)] * 2).astype(np.float32)
    return c, sn


# C++ name (include/nn/layer_exprs.hpp) and argument order of each builder.
ARGS = {
    "rms_sum_sq": ("rms_sum_sq", ("x",)),
    "rms_normalize": ("rms_normalize", ("x", "rinv")),
    "rms_scale": ("rms_scale", ("normed", "gamma")),
    "rms_bwd_colsum": ("rms_bwd_colsum", ("g", "gamma", "normed")),
    "rms_bwd_rowsum": ("rms_bwd_rowsum", ("g", "gamma", "normed")),
    "rms_bwd_dx": ("rms_bwd_dx", ("g", "gamma", "m", "normed", "rinv")),
    "swiglu_grad_gate": ("swiglu_grad_gate", ("g", "up", "s", "gate")),
    "swiglu_grad_up": ("swiglu_grad_up", ("g", "gate", "s")),
    "softmax_rows": ("softmax_rows", ("x",)),
    "softmax_rows_backward": ("softmax_rows_backward", ("y", "g")),
    "rope": ("rope_forward", ("q", "cos", "sin")),
    "rope_backward": ("rope_backward", ("q", "cos", "sin")),
}


# (builder, reduced-vector output, closed form over float64 numpy arrays)
PROGRAMS = {
    "rms_sum_sq": (rms_sum_sq, True, lambda a: (a["x"] ** 2).sum(0, keepdims=True)),
    "rms_normalize": (rms_normalize, False, lambda a: a["x"] * a["rinv"]),
    "rms_scale": (rms_scale, False, lambda a: a["normed"] * a["gamma"]),
    "rms_bwd_colsum": (rms_bwd_colsum, True, lambda a: (a["g"] * a["gamma"] * a["normed"]).sum(0, keepdims=True)),
    "rms_bwd_rowsum": (rms_bwd_rowsum, True, lambda a: (a["g"] * a["gamma"] * a["normed"]).sum(1, keepdims=True)),
    "rms_bwd_dx": (rms_bwd_dx, False, lambda a: (a["g"] * a["gamma"] - a["m"] * a["normed"]) * a["rinv"]),
    "swiglu_grad_gate": (swiglu_grad_gate, False,
                         lambda a: a["g"] * a["up"] * (a["s"] * (1 + a["gate"] * (1 - a["s"])))),
    "swiglu_grad_up": (swiglu_grad_up, False, lambda a: a["g"] * a["gate"] * a["s"]),
}
