"""GPU parity of the GPT layers' ExprSpec programs (RMSNorm, SwiGLU, softmax).

Each program is evaluated by the HIP engine (fused kernel when the shape
allows it, the generic interpreter otherwise: N % 4 != 0) and by the oracle
on the same seeded inputs, and both are checked against the float64 closed
form. Sizes include the config-4 activations (768 x 8192, 3072 x 8192).
"""
import zlib

import numpy as np
import pytest

import layer_programs as lp
from helpers import normal, nrm_err, uniform

pytestmark = pytest.mark.gpu

VEC_SHAPES = {"gamma": "col", "rinv": "row", "m": "row"}


def make_args(rng, names, F, N):
    out = {}
    for n in sorted(set(names)):
        kind = VEC_SHAPES.get(n)
        if n == "gamma":
            out[n] = uniform(rng, (F, 1), 0.5, 1.5)
        elif n == "rinv":
            out[n] = uniform(rng, (1, N), 0.5, 2.0)
        elif n == "m":
            out[n] = normal(rng, (1, N))
        elif n == "s":
            out[n] = uniform(rng, (F, N), 0.0, 1.0)
        else:
            assert kind is None
            out[n] = normal(rng, (F, N))
    return out


def _run(eng, spec, slots, args, F, N, vec):
    ts = {k: eng.tensor(v) for k, v in args.items()}
    ins = [ts[n] for n in slots]
    r = eng.eval_expr_reduce(spec, ins, F, N) if vec else eng.eval_expr(spec, ins, F, N)
    return r.numpy()


@pytest.mark.parametrize("name", sorted(lp.PROGRAMS))
@pytest.mark.parametrize("F,N", [(768, 8192), (24, 36), (24, 10), (5, 4)])
def test_layer_program(hip, cpu, name, F, N):
    build, vec, closed = lp.PROGRAMS[name]
    spec, slots = build()
    rng = np.random.default_rng(zlib.crc32(f"{name}{F}x{N}".encode()))
    args = make_args(rng, slots, F, N)
    h = _run(hip, spec, slots, args, F, N, vec)
    c = _run(cpu, spec, slots, args, F, N, vec)
    ref = closed({k: v.astype(np.float64) for k, v in args.items()})
    assert h.shape == ref.shape == c.shape
    assert nrm_err(h, c) <= 1e-5
    assert nrm_err(h, ref) <= 1e-5


@pytest.mark.parametrize("name", ["swiglu_grad_gate", "swiglu_grad_up"])
def test_swiglu_programs_config4(hip, cpu, name):
    build, vec, closed = lp.PROGRAMS[name]
    spec, slots = build()
    F, N = 3072, 8192
    args = make_args(np.random.default_rng(5), slots, F, N)
    h = _run(hip, spec, slots, args, F, N, vec)
    ref = closed({k: v.astype(np.float64) for k, v in args.items()})
    assert nrm_err(h, ref) <= 1e-6


@pytest.mark.parametrize("R,C", [(96, 1024), (37, 129)])
def test_softmax_programs(hip, cpu, R, C):
    rng = np.random.default_rng(R * C)
    x, g = normal(rng, (R, C), 3.0), normal(rng, (R, C))
    spec, _ = lp.softmax_rows()
    hx, cx = hip.tensor(x), cpu.tensor(x)
    y = hip.eval_expr(spec, [hx] * 4, R, C).numpy()
    yc = cpu.eval_expr(spec, [cx] * 4, R, C).numpy()
    assert nrm_err(y, yc) <= 1e-5
    bspec, _ = lp.softmax_rows_backward()
    hy, hg = hip.tensor(yc), hip.tensor(g)
    cy, cg = cpu.tensor(yc), cpu.tensor(g)
    dx = hip.eval_expr(bspec, [hy, hg, hy, hg], R, C).numpy()
    dxc = cpu.eval_expr(bspec, [cy, cg, cy, cg], R, C).numpy()
    assert nrm_err(dx, dxc) <= 1e-5


def test_same_program_distinct_tensors_uses_general_path(hip, cpu):
    """x*x folded over two different tensors is a valid program that is not the
    sum of squares: the engine must evaluate it as written."""
    spec, _ = lp.rms_sum_sq()
    rng = np.random.default_rng(3)
    a, b = normal(rng, (64, 128)), normal(rng, (64, 128))
    h = hip.eval_expr_reduce(spec, [hip.tensor(a), hip.tensor(b)], 64, 128).numpy()
    assert nrm_err(h, (a.astype(np.float64) * b).sum(0, keepdims=True)) <= 1e-5


@pytest.mark.parametrize("dk,heads,T", [(16, 4, 32), (64, 96, 1024), (8, 3, 7), (64, 12, 1)])
@pytest.mark.parametrize("backward", [False, True])
def test_rope_program(hip, cpu, dk, heads, T, backward):
    """RoPE (compute_layer.hpp:884-984) on the generic interpreter: RotateHalf (first half negated) and
    RowMod views, on (heads*dk, T) heads with (dk, T) tables; bit-exact against the oracle (each
    output is one multiply per term and one add, the same roundings)."""
    spec, slots = lp.rope(dk, backward)
    print(f"[rope] dk {dk} heads {heads} T {T} backward {backward}", flush=True)
    rng = np.random.default_rng(dk * 1000 + T + backward)
    q = normal(rng, (heads * dk, T))
    c, s = lp.rope_tables(dk, T)
    args = dict(q=q, cos=c, sin=s)
    h = _run(hip, spec, slots, args, heads * dk, T, False)
    o = _run(cpu, spec, slots, args, heads * dk, T, False)
    assert nrm_err(h, o) <= 1e-6
    half = dk // 2
    qb = q.reshape(heads, dk, T).astype(np.float64)
    rot = np.concatenate([-qb[:, half:], qb[:, :half]], axis=1) * (-1 if backward else 1)
    ref = (qb * c.astype(np.float64) + rot * s.astype(np.float64)).reshape(heads * dk, T)
    assert nrm_err(h, ref) <= 1e-6


@pytest.mark.parametrize("slot", [0, 3])
@pytest.mark.parametrize("view", ["RowReduceSum", "RowReduceMax", "ColReduceSum", "ColReduceMax"])
@pytest.mark.parametrize("R,C", [(37, 129), (768, 1024)])
def test_reduce_views_and_select(hip, cpu, view, R, C, slot):
    """The reduce views and Select on the GPU interpreter against the oracle: out = Select(x > 0,
    view(x) - 2y, y), with the reduce view at input slot 0 or 3 (each view's record is read at its own
    slot)."""
    from nnengine import ExprSpec, cst, inp, reg
    print(f"[expr] {view} slot {slot} {R}x{C}", flush=True)
    rng = np.random.default_rng(R + C)
    x, y = normal(rng, (R, C)), normal(rng, (R, C))
    s = ExprSpec()
    kinds = ["Linear"] * 4
    kinds[slot] = view
    for k in kinds:
        s.view(k)
    xr, y1, x2, y3 = (slot, 1, 2, 0) if slot == 3 else (0, 1, 2, 3)   # slots reading x (reduced), y, x, y
    c2, c0 = s.const(2.0), s.const(0.0)
    r0 = s.ins("Mul", inp(y1), cst(c2))
    r1 = s.ins("Sub", inp(xr), reg(r0))
    r2 = s.ins("Gt", inp(x2), cst(c0))
    s.ins("Select", reg(r2), reg(r1), inp(y3))

    def run(e):
        ts = [None] * 4
        ts[xr], ts[y1], ts[x2], ts[y3] = e.tensor(x), e.tensor(y), e.tensor(x), e.tensor(y)
        return e.eval_expr(s, ts, R, C).numpy()
    h, c = run(hip), run(cpu)
    assert nrm_err(h, c) <= 1e-5
    red = {"RowReduceSum": x.astype(np.float64).sum(1, keepdims=True), "RowReduceMax": x.max(1, keepdims=True),
           "ColReduceSum": x.astype(np.float64).sum(0, keepdims=True), "ColReduceMax": x.max(0, keepdims=True)}[view]
    ref = np.where(x > 0, red - 2.0 * y.astype(np.float64), y)
    assert nrm_err(h, ref) <= 1e-5
