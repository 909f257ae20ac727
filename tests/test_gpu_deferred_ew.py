"""Deferred elementwise runs of the HIP engine, through the C-ABI.

The engine records consecutive same-size elementwise / in-place calls and runs
them when another kind of call arrives; the optimizers' Adam / AdamW chain
(reference compute_optimizer.hpp:252-304, :388-412) runs as one fused pass per
tensor, the chains of consecutive tensors collected into multi-tensor launches
(a tensor updated again, as in the next step, first launches what is
collected), and SwiGLU::forward's sigmoid-gate chain as one fused pass. Consecutive zero calls
(zero_grad) are cleared together.
Bars: the fused chain is bit-exact against the same calls run one by one (an
engine settle after every call stops any recording from spanning two calls);
both are within 1e-6 of max|p| of the CPU oracle. Mixed sequences match the
oracle within 1e-6 normwise and see every in-place update in call order.
"""
import numpy as np
import pytest

from helpers import nrm_err, normal, uniform

pytestmark = pytest.mark.gpu

LR, B1, B2, EPS, WD = 1e-3, 0.9, 0.999, 1e-8, 0.01


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def adam_chain(e, p, m, v, g, t, decay, after=lambda: None, keep=None):
    """The per-tensor call sequence of the optimizer's adam_update_ (AdamW: decay first)."""
    ib1 = 1.0 / (1.0 - B1 ** t)
    ib2 = 1.0 / (1.0 - B2 ** t)
    if decay:
        e.scale_inplace(p, 1.0 - LR * WD); after()
    e.scale_inplace(m, B1); after()
    e.axpy_inplace(m, 1.0 - B1, g); after()
    e.scale_inplace(v, B2); after()
    g2 = e.elementwise_binary("Mul", g, g); after()
    e.scale_inplace(g2, 1.0 - B2); after()
    e.add_inplace(v, g2); after()
    mh = e.clone(m); after()
    e.scale_inplace(mh, ib1); after()
    vh = e.clone(v); after()
    e.scale_inplace(vh, ib2); after()
    sq = e.elementwise_unary("Sqrt", vh); after()
    den = e.elementwise_binary_scalar("Add", sq, EPS); after()
    ratio = e.elementwise_binary("Div", mh, den); after()
    e.scale_inplace(ratio, -LR); after()
    e.add_inplace(p, ratio); after()
    if keep is not None:
        keep.extend([g2, mh, vh, sq, den, ratio])


def adam_state(rng, shapes):
    out = []
    for s in shapes:
        out.append((normal(rng, s, 0.02), normal(rng, s, 1e-3), np.abs(normal(rng, s, 1e-6)), normal(rng, s, 0.05)))
    return out


def run_adam(e, state, steps, decay, settle_each, keep=None):
    ts = [[e.tensor(a) for a in st] for st in state]
    after = e.settle if settle_each else (lambda: None)
    for t in range(1, steps + 1):
        for p, m, v, g in ts:
            adam_chain(e, p, m, v, g, t, decay, after, keep)
    return [[x.numpy() for x in (p, m, v)] for p, m, v, _ in ts]


SHAPES = [[(1, 1)], [(1, 7)], [(768, 1)], [(10, 100)], [(768, 768)], [(1, 6144)], [(33, 31)],
          # two chains of one size in one recording, then sizes that change
          [(64, 64), (64, 64), (1, 768), (768, 768), (1, 768)],
          # more tensors than one multi-tensor launch takes (48), ragged sizes
          [(i % 7 + 1, 3 * i + 1) for i in range(60)]]


@pytest.mark.parametrize("decay", [True, False])
@pytest.mark.parametrize("shapes", SHAPES, ids=lambda s: "+".join(f"{r}x{c}" for r, c in s))
def test_adam_fused_matches_calls(hip, cpu, shapes, decay):
    rng = np.random.default_rng(len(shapes) * 1000 + shapes[0][0] + 7 * shapes[0][1] + decay)
    state = adam_state(rng, shapes)
    fused = run_adam(hip, state, 3, decay, settle_each=False)
    calls = run_adam(hip, state, 3, decay, settle_each=True)
    ref = run_adam(cpu, state, 3, decay, settle_each=False)
    for f, c, r, st in zip(fused, calls, ref, state):
        for name, a, b, o in zip("pmv", f, c, r):
            assert np.array_equal(bits(a), bits(b)), f"{name}: fused chain differs from the calls run one by one"
            scale = max(float(np.abs(o).max()), 1e-30)
            assert float(np.abs(a - o).max()) <= 1e-6 * scale, f"{name} vs oracle"


def test_adam_kept_temporaries_run_call_by_call(hip):
    """A temporary of the chain still referenced: the chain must not fuse, and the temporary holds its value."""
    rng = np.random.default_rng(11)
    state = adam_state(rng, [(40, 50)])
    keep = []
    got = run_adam(hip, state, 1, True, settle_each=False, keep=keep)
    ref = run_adam(hip, state, 1, True, settle_each=True)
    for a, b in zip(got[0], ref[0]):
        assert np.array_equal(bits(a), bits(b))
    p, m, v, g = state[0]
    g2, mh, vh, sq, den, ratio = [k.numpy() for k in keep]
    assert np.array_equal(bits(g2), bits((g * g).astype(np.float32) * np.float32(1 - B2)))
    assert np.array_equal(bits(sq), bits(np.sqrt(vh)))
    assert np.array_equal(bits(den), bits(sq + np.float32(EPS)))


def test_mixed_sequence_in_call_order(hip, cpu):
    """In-place updates, aliases and reads by other kinds of call see every earlier call."""
    rng = np.random.default_rng(5)
    A, B = uniform(rng, (129, 65)), uniform(rng, (129, 65))
    V = uniform(rng, (1, 129 * 65 // 5))

    def run(e):
        a, b = e.tensor(A), e.tensor(B)
        c = e.clone(a)
        e.scale_inplace(a, 3.0)
        d = e.elementwise_binary("Mul", a, c)          # new a times old a
        e.add_inplace(c, d)
        e.axpy_inplace(b, -0.5, c)
        s1 = e.row_reduce_sum(b)                        # another kind of call reads b
        e.add_inplace(b, b)                             # operand aliasing the destination
        x = e.elementwise_binary_scalar("Sub", b, 2.0, scalar_first=True)
        dead = e.elementwise_unary("Exp", x)            # result dropped unread
        del dead
        y = e.elementwise_unary("Abs", x)
        v = e.tensor(V)                                 # another size: starts a new recording
        e.scale_inplace(v, -1.0)
        w = e.elementwise_binary("Max", v, v)
        e.scale_inplace(y, 0.25)
        return [a, b, c, d, s1, x, y, v, w]

    h, c = run(hip), run(cpu)
    for i, (a, b) in enumerate(zip(h, c)):
        assert nrm_err(a.numpy(), b.numpy()) <= 1e-6, f"output {i}"


def test_zero_size_and_errors(hip):
    z = hip.tensor(np.zeros((0, 5), np.float32))
    hip.scale_inplace(z, 2.0)
    assert hip.clone(z).shape == (0, 5)
    a = hip.tensor(np.ones((3, 4), np.float32))
    b = hip.tensor(np.ones((4, 3), np.float32))
    with pytest.raises(Exception):
        hip.add_inplace(a, b)
    hip.scale_inplace(a, 2.0)
    assert np.array_equal(a.numpy(), np.full((3, 4), 2.0, np.float32))


def swiglu_chain(e, gate, up, after=lambda: None):
    """SwiGLU::forward's calls on the gate and up halves (sigmoid written out as primitives)."""
    t1 = e.elementwise_unary("Neg", gate); after()
    t2 = e.elementwise_unary("Exp", t1); after()
    t3 = e.elementwise_binary_scalar("Add", t2, 1.0); after()
    s = e.elementwise_binary_scalar("Div", t3, 1.0, scalar_first=True); after()
    sw = e.elementwise_binary("Mul", gate, s); after()
    out = e.elementwise_binary("Mul", sw, up); after()
    return s, out


@pytest.mark.parametrize("shape", [(3072, 8192), (7, 13), (1, 5), (64, 64)])
def test_swiglu_forward_fused_matches_calls(hip, cpu, shape):
    rng = np.random.default_rng(shape[0] * 31 + shape[1])
    G, U = normal(rng, shape, 3.0), normal(rng, shape)

    def run(e, settle_each):
        g, u = e.tensor(G), e.tensor(U)
        s, out = swiglu_chain(e, g, u, e.settle if settle_each else (lambda: None))
        return s.numpy(), out.numpy()

    fs, fo = run(hip, False)
    cs, co = run(hip, True)
    assert np.array_equal(bits(fs), bits(cs)) and np.array_equal(bits(fo), bits(co))
    rs, ro = run(cpu, False)
    assert nrm_err(fs, rs) <= 1e-6 and nrm_err(fo, ro) <= 1e-6


def test_swiglu_forward_sigmoid_dropped(hip):
    """The sigmoid dropped before the run is launched: out alone is written."""
    rng = np.random.default_rng(2)
    G, U = normal(rng, (40, 64)), normal(rng, (40, 64))
    g, u = hip.tensor(G), hip.tensor(U)
    s, out = swiglu_chain(hip, g, u)
    del s
    ref = swiglu_chain(hip, hip.tensor(G), hip.tensor(U), hip.settle)[1].numpy()
    assert np.array_equal(bits(out.numpy()), bits(ref))


def test_zero_list(hip):
    """Consecutive zero calls over tensors of many sizes, then reads and further calls in order."""
    rng = np.random.default_rng(8)
    shapes = [(1, 1), (3, 5), (768, 1), (1, 6144), (768, 768), (17, 33), (4096, 5)] * 30
    arrs = [uniform(rng, s, 1.0, 2.0) for s in shapes]
    ts = [hip.tensor(a) for a in arrs]
    keep = hip.tensor(arrs[0])
    for t in ts:
        hip.zero(t)
    hip.add_inplace(ts[3], hip.tensor(arrs[3]))          # an elementwise call after the zeros
    s = hip.row_reduce_sum(ts[4])                          # another kind of call
    for i, t in enumerate(ts):
        got = t.numpy()
        assert np.array_equal(got, arrs[3] if i == 3 else np.zeros_like(got)), i
    assert not s.numpy().any()
    assert np.array_equal(keep.numpy(), arrs[0])


def test_zero_folded_into_first_accumulation(hip):
    """zero_grad then the Linear backward's grad_w += G X^T (and grad_b += row sums of G): a gradient
    whose zero fill is still recorded gets the product (the sums) written instead of added; the
    other zeroed tensors stay zero until read, including through a row slice of one of them."""
    rng = np.random.default_rng(13)
    G, X = uniform(rng, (96, 200)), uniform(rng, (64, 200))
    gw, gb, other = (hip.tensor(uniform(rng, s, 1.0, 2.0)) for s in ((96, 64), (96, 1), (50, 7)))
    for t in (gw, gb, other):
        hip.zero(t)
    g, x = hip.tensor(G), hip.tensor(X)
    hip.add_inplace(gw, hip.matmul(g, x, False, True))     # Linear::backward's weight gradient
    hip.add_inplace(gb, hip.row_reduce_sum(g))              # and its bias gradient
    view = hip.slice_rows(other, 10, 5)
    ref_w = G.astype(np.float64) @ X.astype(np.float64).T
    assert np.abs(gw.numpy() - ref_w).max() <= 1e-5 * np.abs(ref_w).max()
    assert np.abs(gb.numpy()[:, 0] - G.astype(np.float64).sum(1)).max() <= 1e-5 * np.abs(G).sum(1).max()
    assert not view.numpy().any() and not other.numpy().any()
    hip.add_inplace(gw, hip.matmul(g, x, False, True))     # second step: accumulates
    assert np.abs(gw.numpy() - 2 * ref_w).max() <= 1e-5 * np.abs(2 * ref_w).max()


def test_zero_then_inserts(hip):
    """SwiGLU::backward's zero + insert_rows pattern: inserted rows are not zeroed
    afterwards, rows no insert covers are, and a second zero call wins over earlier inserts."""
    rng = np.random.default_rng(12)
    R, C = 70, 36
    a, b, c = uniform(rng, (30, C)), uniform(rng, (25, C)), uniform(rng, (10, C))
    dst = hip.tensor(uniform(rng, (R, C), 5.0, 6.0))
    hip.zero(dst)
    hip.insert_rows(dst, 0, hip.tensor(a))
    hip.insert_rows(dst, 40, hip.tensor(b))     # rows 30..39 and 65..69 stay zero
    ref = np.zeros((R, C), np.float32)
    ref[0:30], ref[40:65] = a, b
    assert np.array_equal(dst.numpy(), ref)
    hip.zero(dst)
    hip.insert_rows(dst, 5, hip.tensor(c))
    hip.zero(dst)                                # the later zero clears the insert too
    hip.insert_rows(dst, 60, hip.tensor(c))
    ref = np.zeros((R, C), np.float32)
    ref[60:70] = c
    assert np.array_equal(dst.numpy(), ref)
    src = hip.tensor(a)
    hip.zero(src)                                # a pending zero on the source is applied before it is read
    hip.insert_rows(dst, 0, src)
    ref[0:30] = 0
    assert np.array_equal(dst.numpy(), ref)


def swiglu_backward(e, G, U, S, Ga, after=lambda: None, read_parts=False, dst_init=None):
    """SwiGLU::backward's calls: both gradient programs, then zero + two row inserts."""
    import layer_programs as lp
    F, N = G.shape
    spec_g, slots_g = lp.swiglu_grad_gate()
    spec_u, slots_u = lp.swiglu_grad_up()
    t = dict(g=e.tensor(G), up=e.tensor(U), s=e.tensor(S), gate=e.tensor(Ga))
    gg = e.eval_expr(spec_g, [t[n] for n in slots_g], F, N); after()
    gu = e.eval_expr(spec_u, [t[n] for n in slots_u], F, N); after()
    dst = e.tensor(dst_init) if dst_init is not None else e.create_tensor(2 * F, N)
    if dst_init is None:
        e.zero(dst); after()
    e.insert_rows(dst, 0, gg); after()
    e.insert_rows(dst, F, gu); after()
    parts = [gg.numpy(), gu.numpy()] if read_parts else []
    del gg, gu                               # as when SwiGLU::backward returns: one pass for both halves
    return [dst.numpy()] + parts


@pytest.mark.parametrize("F,N,read_parts,init", [(3072, 8192, False, False), (24, 36, True, False),
                                                 (40, 64, False, True), (8, 12, True, True)])
def test_swiglu_backward_into_gradient(hip, cpu, F, N, read_parts, init):
    rng = np.random.default_rng(F + N)
    G, U, Ga = normal(rng, (F, N)), normal(rng, (F, N)), normal(rng, (F, N))
    S = uniform(rng, (F, N), 0.0, 1.0)
    D0 = uniform(rng, (2 * F, N)) if init else None
    fused = swiglu_backward(hip, G, U, S, Ga, read_parts=read_parts, dst_init=D0)
    calls = swiglu_backward(hip, G, U, S, Ga, hip.settle, read_parts=read_parts, dst_init=D0)
    for a, b in zip(fused, calls):
        assert np.array_equal(bits(a), bits(b))
    ref = swiglu_backward(cpu, G, U, S, Ga, read_parts=read_parts, dst_init=D0)
    for a, b in zip(fused, ref):
        assert nrm_err(a, b) <= 1e-6
