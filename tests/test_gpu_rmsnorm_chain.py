"""RMSNorm through the engine as the layer issues it (compute_layer.hpp RMSNorm):
forward s = sum of squares of x's columns, s * 1/F, + eps, rsqrt, normalize,
scale by gamma; backward m_raw = column sums of g * gamma * normed, m = m_raw / F,
dx = (g * gamma - m * normed) * rinv.

The HIP engine records these calls and, when the chain's last one arrives, runs
them as one pass (nnhip_rmsnorm_forward / nnhip_rmsnorm_backward, the big inputs
read once); any other use of an intermediate, or a write to an input, runs the
calls so far with their separate kernels. The GPT block's residual adds join
these passes: x + a recorded before the forward's first call is formed by the
forward pass, and grad + dx after the backward's dx call by the backward pass. Bars: every output of the one-pass run
bit-identical to the separate kernels' (the chain cut right after its first
call), every cut variant equal to it too, and all of them within 1e-5
(normwise) of the oracle running the same calls.
"""
import numpy as np
import pytest

import layer_programs as lp
from helpers import normal, nrm_err, uniform

pytestmark = pytest.mark.gpu

SQ, _ = lp.rms_sum_sq()
NORM, _ = lp.rms_normalize()
SCALE, _ = lp.rms_scale()
NAMES = ("s", "scaled", "var_eps", "rinv", "normed", "out")
BCOL, _ = lp.rms_bwd_colsum()
BDX, _ = lp.rms_bwd_dx()
BROW, _ = lp.rms_bwd_rowsum()
BNAMES = ("m_raw", "m", "dx", "gg")


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def chain(e, X, G, eps, cut=None):
    """The layer's calls; `cut` names the interruption: "s" reads s after the first call,
    "rinv" reads rinv before the normalize, "write_x" scales x in place before the scale call."""
    F, N = X.shape
    x, g = e.tensor(X), e.tensor(G)
    s = e.eval_expr_reduce(SQ, [x, x], F, N)
    if cut == "s":
        s.numpy()
    sc = e.elementwise_binary_scalar("Mul", s, 1.0 / F)
    ve = e.elementwise_binary_scalar("Add", sc, eps)
    ri = e.elementwise_unary("Rsqrt", ve)
    if cut == "rinv":
        ri.numpy()
    nm = e.eval_expr(NORM, [x, ri], F, N)
    if cut == "write_x":
        e.scale_inplace(x, 2.0)
    out = e.eval_expr(SCALE, [nm, g], F, N)
    res = dict(zip(NAMES, (t.numpy() for t in (s, sc, ve, ri, nm, out))))
    res["x"] = x.numpy()
    return res


@pytest.mark.parametrize("F,N", [(768, 8192), (128, 36), (1024, 64), (1100, 40), (24, 10), (5, 4), (300, 100),
                                 (768, 1), (1024, 1), (7, 2), (1025, 1), (200, 13)])
def test_rmsnorm_forward_chain(hip, cpu, F, N):
    """N % 4 != 0 with F <= 1024 (one token's (d_model, 1) activations in incremental inference) runs the
    narrow kernels, whose one-pass forward and separate calls share one summation order."""
    rng = np.random.default_rng(F * 131 + N)
    X, G = normal(rng, (F, N)), uniform(rng, (F, 1), 0.5, 1.5)
    eps = 1e-5
    fused = chain(hip, X, G, eps)
    ref = chain(cpu, X, G, eps)
    for cut in ("s", "rinv", "write_x"):
        other = chain(hip, X, G, eps, cut)
        print(f"[rmsnorm] F{F} N{N} cut={cut}", flush=True)
        for n in NAMES:
            assert np.array_equal(bits(fused[n]), bits(other[n])), (cut, n)
        assert np.array_equal(bits(other["x"]), bits(X * (2.0 if cut == "write_x" else 1.0))), cut
    for n in NAMES:
        assert fused[n].shape == ref[n].shape, n
        assert nrm_err(fused[n], ref[n]) <= 1e-5, n
    # closed form in float64
    x64 = X.astype(np.float64)
    r = 1.0 / np.sqrt((x64 * x64).sum(0, keepdims=True) / F + eps)
    assert nrm_err(fused["out"], x64 * r * G.astype(np.float64)) <= 1e-5


def test_rmsnorm_chain_two_layers_interleaved(hip, cpu):
    """A second chain starting before the first is complete runs the first one's calls separately."""
    rng = np.random.default_rng(11)
    F, N = 256, 512
    X1, X2 = normal(rng, (F, N)), normal(rng, (F, N))
    G = uniform(rng, (F, 1), 0.5, 1.5)

    def go(e):
        x1, x2, g = e.tensor(X1), e.tensor(X2), e.tensor(G)
        s1 = e.eval_expr_reduce(SQ, [x1, x1], F, N)
        s2 = e.eval_expr_reduce(SQ, [x2, x2], F, N)
        r1 = e.elementwise_unary("Rsqrt", e.elementwise_binary_scalar("Add", e.elementwise_binary_scalar("Mul", s1, 1.0 / F), 1e-5))
        r2 = e.elementwise_unary("Rsqrt", e.elementwise_binary_scalar("Add", e.elementwise_binary_scalar("Mul", s2, 1.0 / F), 1e-5))
        o1 = e.eval_expr(SCALE, [e.eval_expr(NORM, [x1, r1], F, N), g], F, N)
        o2 = e.eval_expr(SCALE, [e.eval_expr(NORM, [x2, r2], F, N), g], F, N)
        return [t.numpy() for t in (s1, s2, r1, r2, o1, o2)]

    for a, b in zip(go(hip), go(cpu)):
        assert nrm_err(a, b) <= 1e-5


def bwd_chain(e, Gr, Ga, Nm, Ri, cut=None):
    """The backward's calls; `cut`: "m_raw" reads m_raw after the first call, "write_g" scales g
    in place before the dx call, "write_gamma" scales gamma in place there."""
    F, N = Gr.shape
    g, ga, nm, ri = e.tensor(Gr), e.tensor(Ga), e.tensor(Nm), e.tensor(Ri)
    m_raw = e.eval_expr_reduce(BCOL, [g, ga, nm], F, N)
    if cut == "m_raw":
        m_raw.numpy()
    m = e.elementwise_binary_scalar("Mul", m_raw, 1.0 / F)
    if cut == "write_g":
        e.scale_inplace(g, 2.0)
    if cut == "write_gamma":
        e.scale_inplace(ga, 2.0)
    dx = e.eval_expr(BDX, [g, ga, m, nm, ri], F, N)
    gg = e.eval_expr_reduce(BROW, [g, ga, nm], F, N)
    return dict(zip(BNAMES, (t.numpy() for t in (m_raw, m, dx, gg))))


@pytest.mark.parametrize("F,N", [(768, 8192), (128, 36), (1024, 64), (1100, 40), (24, 10), (300, 100)])
def test_rmsnorm_backward_chain(hip, cpu, F, N):
    rng = np.random.default_rng(F * 7 + N)
    Gr, Nm = normal(rng, (F, N)), normal(rng, (F, N))
    Ga, Ri = uniform(rng, (F, 1), 0.5, 1.5), uniform(rng, (1, N), 0.5, 2.0)
    fused = bwd_chain(hip, Gr, Ga, Nm, Ri)
    ref = bwd_chain(cpu, Gr, Ga, Nm, Ri)
    cut = bwd_chain(hip, Gr, Ga, Nm, Ri, "m_raw")
    for n in BNAMES:
        assert np.array_equal(bits(fused[n]), bits(cut[n])), n
        assert nrm_err(fused[n], ref[n]) <= 1e-5, n
    # writes between the column sum and dx: the column sums see the old values, dx the new ones
    for w in ("write_g", "write_gamma"):
        print(f"[rmsnorm bwd] F{F} N{N} {w}", flush=True)
        h, c = bwd_chain(hip, Gr, Ga, Nm, Ri, w), bwd_chain(cpu, Gr, Ga, Nm, Ri, w)
        for n in BNAMES:
            assert nrm_err(h[n], c[n]) <= 1e-5, (w, n)
        assert np.array_equal(bits(h["m_raw"]), bits(fused["m_raw"])), w
    g64, n64, a64 = Gr.astype(np.float64), Nm.astype(np.float64), Ga.astype(np.float64)
    m = (g64 * a64 * n64).sum(0, keepdims=True) / F
    assert nrm_err(fused["dx"], (g64 * a64 - m * n64) * Ri.astype(np.float64)) <= 1e-5


# ── the block's residual adds taken into the RMSNorm passes (GPTBlock, compute_layer.hpp:2366-2405) ──
def residual_chain(e, X, A, G, eps, cut=None):
    """y = x + a (GPTBlock::forward's residual add), then the layer's six calls on y; `cut`: "y" reads y
    after the first call, "write_a" scales a in place before the scale call, "early" reads y right
    after the add (the add then runs alone)."""
    F, N = X.shape
    x, a, g = e.tensor(X), e.tensor(A), e.tensor(G)
    y = e.elementwise_binary("Add", x, a)
    if cut == "early":
        y.numpy()
    s = e.eval_expr_reduce(SQ, [y, y], F, N)
    if cut == "y":
        y.numpy()
    sc = e.elementwise_binary_scalar("Mul", s, 1.0 / F)
    ve = e.elementwise_binary_scalar("Add", sc, eps)
    ri = e.elementwise_unary("Rsqrt", ve)
    nm = e.eval_expr(NORM, [y, ri], F, N)
    if cut == "write_a":
        e.scale_inplace(a, 2.0)
    out = e.eval_expr(SCALE, [nm, g], F, N)
    res = dict(zip(NAMES, (t.numpy() for t in (s, sc, ve, ri, nm, out))))
    res["y"], res["a"] = y.numpy(), a.numpy()
    return res


@pytest.mark.parametrize("F,N", [(768, 8192), (128, 36), (1100, 40), (300, 100), (768, 1), (200, 13)])
def test_residual_add_then_rmsnorm(hip, cpu, F, N):
    """The recorded x + a is formed and written by the RMSNorm pass (nnhip_rmsnorm_forward_sum) when
    N % 4 == 0: every output bit-identical to the add and the chain run apart ("early"), the cut
    variants equal too, a written in place after y was recorded leaves y as it was."""
    rng = np.random.default_rng(F * 17 + N)
    X, A, G = normal(rng, (F, N)), normal(rng, (F, N)), uniform(rng, (F, 1), 0.5, 1.5)
    eps = 1e-5
    fused = residual_chain(hip, X, A, G, eps)
    apart = residual_chain(hip, X, A, G, eps, "early")
    ref = residual_chain(cpu, X, A, G, eps)
    for n in NAMES + ("y",):
        assert np.array_equal(bits(fused[n]), bits(apart[n])), n
        assert nrm_err(fused[n], ref[n]) <= 1e-5, n
    assert np.array_equal(bits(fused["y"]), bits(X + A))
    for cut in ("y", "write_a"):
        print(f"[rmsnorm residual] F{F} N{N} cut={cut}", flush=True)
        other = residual_chain(hip, X, A, G, eps, cut)
        for n in NAMES + ("y",):
            assert np.array_equal(bits(fused[n]), bits(other[n])), (cut, n)
        assert np.array_equal(bits(other["a"]), bits(A * (2.0 if cut == "write_a" else 1.0))), cut


def residual_bwd_chain(e, Gr, Ga, Nm, Ri, E, cut=None, swap=False):
    """The backward's calls, then out = e + dx (GPTBlock::backward's residual add; dx + e when
    `swap`); `cut`: "dx" reads dx before the add (the add then runs alone), "write_e" scales e in
    place before the add."""
    F, N = Gr.shape
    g, ga, nm, ri, ee = e.tensor(Gr), e.tensor(Ga), e.tensor(Nm), e.tensor(Ri), e.tensor(E)
    m_raw = e.eval_expr_reduce(BCOL, [g, ga, nm], F, N)
    m = e.elementwise_binary_scalar("Mul", m_raw, 1.0 / F)
    dx = e.eval_expr(BDX, [g, ga, m, nm, ri], F, N)
    gg = e.eval_expr_reduce(BROW, [g, ga, nm], F, N)
    if cut == "dx":
        dx.numpy()
    if cut == "write_e":
        e.scale_inplace(ee, 2.0)
    out = e.elementwise_binary("Add", dx, ee) if swap else e.elementwise_binary("Add", ee, dx)
    res = dict(zip(BNAMES, (t.numpy() for t in (m_raw, m, dx, gg))))
    res["out"] = out.numpy()
    return res


@pytest.mark.parametrize("F,N", [(768, 8192), (128, 36), (1100, 40), (300, 100)])
def test_rmsnorm_backward_then_residual_add(hip, cpu, F, N):
    """The recorded dx and the add of the incoming gradient run as one pass
    (nnhip_rmsnorm_backward_add): dx and the sum bit-identical to the calls run apart."""
    rng = np.random.default_rng(F * 3 + N)
    Gr, Nm, E = normal(rng, (F, N)), normal(rng, (F, N)), normal(rng, (F, N))
    Ga, Ri = uniform(rng, (F, 1), 0.5, 1.5), uniform(rng, (1, N), 0.5, 2.0)
    fused = residual_bwd_chain(hip, Gr, Ga, Nm, Ri, E)
    apart = residual_bwd_chain(hip, Gr, Ga, Nm, Ri, E, "dx")
    ref = residual_bwd_chain(cpu, Gr, Ga, Nm, Ri, E)
    for n in BNAMES + ("out",):
        assert np.array_equal(bits(fused[n]), bits(apart[n])), n
        assert nrm_err(fused[n], ref[n]) <= 1e-5, n
    assert np.array_equal(bits(fused["out"]), bits(E + fused["dx"]))
    swapped = residual_bwd_chain(hip, Gr, Ga, Nm, Ri, E, swap=True)
    assert np.array_equal(bits(swapped["out"]), bits(fused["out"]))
    w = residual_bwd_chain(hip, Gr, Ga, Nm, Ri, E, "write_e")
    assert np.array_equal(bits(w["out"]), bits(E * np.float32(2.0) + fused["dx"]))
