"""Row sums folded into the gradient they are added to.

Linear::backward issues gb = row_reduce_sum(G) then add_inplace(grad_b, gb)
(compute_layer.hpp Linear); RMSNorm::backward issues gg = eval_expr_reduce(row
sums of g * gamma * normed) then add_inplace(grad_gamma, gg). The HIP engine
records the row sum and lets the add's kernel be the row-sum kernel adding into
the gradient; the sums themselves are computed only if read later. Bars: the
gradient bit-identical to the unfused calls (the sums read before the add),
the sums bit-identical when read after the fold, and a write to G after the
fold leaving the sums as they were before it; every result within 1e-5
(normwise) of the oracle.
"""
import numpy as np
import pytest

import layer_programs as lp
from helpers import normal, nrm_err, uniform

pytestmark = pytest.mark.gpu

BROW, _ = lp.rms_bwd_rowsum()


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def linear_bias(e, G, B0, how):
    g, b = e.tensor(G), e.tensor(B0)
    s = e.row_reduce_sum(g)
    if how == "read_first":
        s.numpy()
    e.add_inplace(b, s)
    out = {"grad_b": b.numpy()}
    if how == "write_g":
        e.scale_inplace(g, 2.0)
    out["sums"] = s.numpy()
    return out


def rms_gamma(e, Gr, Ga, Nm, B0, how):
    g, ga, nm, b = e.tensor(Gr), e.tensor(Ga), e.tensor(Nm), e.tensor(B0)
    F, N = Gr.shape
    s = e.eval_expr_reduce(BROW, [g, ga, nm], F, N)
    if how == "read_first":
        s.numpy()
    e.add_inplace(b, s)
    out = {"grad_b": b.numpy()}
    if how == "write_g":
        e.scale_inplace(g, 2.0)
    out["sums"] = s.numpy()
    return out


@pytest.mark.parametrize("R,C", [(768, 8192), (6144, 8192), (33, 4100), (7, 20), (100, 36)])
def test_linear_bias_gradient_fold(hip, cpu, R, C):
    rng = np.random.default_rng(R + C)
    G, B0 = normal(rng, (R, C)), normal(rng, (R, 1))
    ref = linear_bias(cpu, G, B0, "read_first")
    base = linear_bias(hip, G, B0, "read_first")
    for how in ("fold", "write_g"):
        print(f"[rowsum fold] {R}x{C} {how}", flush=True)
        h = linear_bias(hip, G, B0, how)
        assert np.array_equal(bits(h["grad_b"]), bits(base["grad_b"])), how
        assert np.array_equal(bits(h["sums"]), bits(base["sums"])), how
    for k in ("grad_b", "sums"):
        assert nrm_err(base[k], ref[k]) <= 1e-5, k


@pytest.mark.parametrize("F,N", [(768, 8192), (24, 36), (300, 100)])
def test_rmsnorm_gamma_gradient_fold(hip, cpu, F, N):
    rng = np.random.default_rng(F * 3 + N)
    Gr, Nm = normal(rng, (F, N)), normal(rng, (F, N))
    Ga, B0 = uniform(rng, (F, 1), 0.5, 1.5), normal(rng, (F, 1))
    ref = rms_gamma(cpu, Gr, Ga, Nm, B0, "read_first")
    base = rms_gamma(hip, Gr, Ga, Nm, B0, "read_first")
    for how in ("fold", "write_g"):
        h = rms_gamma(hip, Gr, Ga, Nm, B0, how)
        assert np.array_equal(bits(h["grad_b"]), bits(base["grad_b"])), how
        assert np.array_equal(bits(h["sums"]), bits(base["sums"])), how
    for k in ("grad_b", "sums"):
        assert nrm_err(base[k], ref[k]) <= 1e-5, k
