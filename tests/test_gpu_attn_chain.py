"""The reference's materialised attention path through the engine primitives.

GPT attention with ALiBi or document ids (reference compute_layer.hpp:1230-1252
forward, :1331-1361 backward) issues scores = batched_matmul(Q, K, transA),
masked = scores + mask, A = softmax rows, O = batched_matmul(V, A, transB) and,
backward, dV = batched_matmul(dO, A), P = batched_matmul(dO, V, transA),
dS = softmax backward (A, P), dQ / dK = batched_matmul(K / Q, dS). The HIP
engine records these calls and runs the one-pass kernels without forming
scores or A; the oracle runs every call as written. Bars: O normwise 1e-4,
dQ / dK / dV 1e-3 (the one-pass tolerances); tensors the engine computes on
demand (A, dS) 1e-5. Cases cover ALiBi, document and shared causal masks,
ragged sizes, reads of the recorded tensors, call orders and in-place writes.
"""
import numpy as np
import pytest

import layer_programs as lp
from helpers import normal, nrm_err

pytestmark = pytest.mark.gpu

SM, _ = lp.softmax_rows()
SMB, _ = lp.softmax_rows_backward()


def attn_mask(B, H, T, alibi=True, doc_ids=None):
    """(B*H*T, T): allowed iff j <= i (and same document); value -slope_h (i - j) with ALiBi."""
    i = np.arange(T)[:, None]
    j = np.arange(T)[None, :]
    out = np.empty((B, H, T, T), np.float32)
    for b in range(B):
        ok = j <= i
        if doc_ids is not None:
            d = doc_ids[b]
            ok = ok & (d[:, None] == d[None, :])
        for h in range(H):
            slope = 2.0 ** (-8.0 * h / H) if alibi else 0.0
            v = (-np.float32(slope) * (i - j).astype(np.float32)).astype(np.float32)
            out[b, h] = np.where(ok, v, -np.inf)
    return out.reshape(B * H * T, T)


def fwd(e, q, k, v, mk, BH, T, alpha):
    scores = e.batched_matmul(q, k, BH, True, False, alpha)
    masked = e.elementwise_binary("Add", scores, mk)
    del scores
    A = e.eval_expr(SM, [masked] * 4, BH * T, T)
    del masked
    O = e.batched_matmul(v, A, BH, False, True)
    return A, O


def bwd(e, q, k, v, A, g, BH, T, alpha, order="qk", with_dv=True):
    gv = e.batched_matmul(g, A, BH, False, False) if with_dv else None
    gA = e.batched_matmul(g, v, BH, True, False)
    gS = e.eval_expr(SMB, [A, gA, A, gA], BH * T, T)
    del gA
    if order == "qk":
        gq = e.batched_matmul(k, gS, BH, False, True, alpha)
        gk = e.batched_matmul(q, gS, BH, False, False, alpha)
    else:
        gk = e.batched_matmul(q, gS, BH, False, False, alpha)
        gq = e.batched_matmul(k, gS, BH, False, True, alpha)
    return gS, gq, gk, gv


def inputs(seed, BH, T, dk):
    rng = np.random.default_rng(seed)
    return [normal(rng, (BH * dk, T)) for _ in range(4)]


def run(e, arrs, mask, BH, T, alpha, read_A=False, read_gS=False, order="qk", with_dv=True):
    q, k, v, g = (e.tensor(a) for a in arrs)
    mk = e.tensor(mask)
    A, O = fwd(e, q, k, v, mk, BH, T, alpha)
    out = {"O": O.numpy()}
    if read_A:
        out["A"] = A.numpy()
    gS, gq, gk, gv = bwd(e, q, k, v, A, g, BH, T, alpha, order, with_dv)
    out.update(dQ=gq.numpy(), dK=gk.numpy())
    if gv is not None:
        out["dV"] = gv.numpy()
    if read_gS:
        out["dS"] = gS.numpy()
    return out


TOL = {"O": 1e-4, "dQ": 1e-3, "dK": 1e-3, "dV": 1e-3, "A": 1e-5, "dS": 1e-5}


def check(h, c):
    for name, a in h.items():
        assert a.shape == c[name].shape, name
        assert np.isfinite(a).all(), name
        assert nrm_err(a, c[name]) <= TOL[name], f"{name}: {nrm_err(a, c[name])}"


@pytest.mark.parametrize("B,H,T,dk", [(1, 1, 32, 64), (2, 3, 100, 64), (1, 4, 256, 64), (2, 2, 64, 32),
                                      (1, 2, 130, 16)])
@pytest.mark.parametrize("kind", ["alibi", "doc_alibi", "causal"])
def test_chain(hip, cpu, B, H, T, dk, kind):
    BH = B * H
    rng = np.random.default_rng(T * 7 + dk + BH)
    doc = None
    if kind == "doc_alibi":
        doc = [np.cumsum(rng.random(T) < 0.04) for _ in range(B)]
    mask = attn_mask(B, H, T, alibi=kind != "causal", doc_ids=doc)
    arrs = inputs(BH + T, BH, T, dk)
    alpha = 1.0 / np.sqrt(dk)
    check(run(hip, arrs, mask, BH, T, alpha), run(cpu, arrs, mask, BH, T, alpha))


@pytest.mark.parametrize("read_A,read_gS,order,with_dv", [(True, False, "qk", True), (False, True, "qk", True),
                                                          (False, False, "kq", True), (False, False, "qk", False),
                                                          (True, True, "kq", False)])
def test_chain_reads_and_orders(hip, cpu, read_A, read_gS, order, with_dv):
    B, H, T, dk = 2, 2, 96, 64
    mask = attn_mask(B, H, T)
    arrs = inputs(3, B * H, T, dk)
    kw = dict(read_A=read_A, read_gS=read_gS, order=order, with_dv=with_dv)
    check(run(hip, arrs, mask, B * H, T, 0.125, **kw), run(cpu, arrs, mask, B * H, T, 0.125, **kw))


def test_probabilities_read_after_backward(hip, cpu):
    """With whole 32 x 32 tiles the fused forward keeps its scores in A's memory for the backward;
    A read after the backward still holds the probabilities."""
    B, H, T, dk = 2, 2, 128, 64
    BH = B * H
    mask = attn_mask(B, H, T)
    arrs = inputs(5, BH, T, dk)

    def go(e):
        q, k, v, g = (e.tensor(a) for a in arrs)
        A, O = fwd(e, q, k, v, e.tensor(mask), BH, T, 0.125)
        gS, gq, gk, gv = bwd(e, q, k, v, A, g, BH, T, 0.125)
        return {"O": O.numpy(), "dQ": gq.numpy(), "dK": gk.numpy(), "dV": gv.numpy(), "A": A.numpy()}

    check(go(hip), go(cpu))


def test_two_layers_back_to_back(hip, cpu):
    """Two recorded layers between forward and backward (backward in reverse order), as in a model."""
    B, H, T, dk = 1, 3, 128, 64
    BH = B * H
    mask = attn_mask(B, H, T)

    def model(e):
        a1, a2 = inputs(1, BH, T, dk), inputs(2, BH, T, dk)
        t1 = [e.tensor(x) for x in a1]
        t2 = [e.tensor(x) for x in a2]
        mk = e.tensor(mask)
        A1, O1 = fwd(e, t1[0], t1[1], t1[2], mk, BH, T, 0.125)
        A2, O2 = fwd(e, t2[0], t2[1], t2[2], mk, BH, T, 0.125)
        r2 = bwd(e, t2[0], t2[1], t2[2], A2, t2[3], BH, T, 0.125)
        r1 = bwd(e, t1[0], t1[1], t1[2], A1, t1[3], BH, T, 0.125)
        return [O1.numpy(), O2.numpy()] + [x.numpy() for x in r2[1:] + r1[1:]]

    h, c = model(hip), model(cpu)
    for i, (a, b) in enumerate(zip(h, c)):
        assert nrm_err(a, b) <= (1e-4 if i < 2 else 1e-3), i


def test_inplace_write_between_forward_and_backward(hip, cpu):
    """Writing an input of a recorded layer (here Q) fixes A as computed from the old values."""
    B, H, T, dk = 1, 2, 64, 64
    BH = B * H
    mask = attn_mask(B, H, T)
    arrs = inputs(9, BH, T, dk)

    def go(e):
        q, k, v, g = (e.tensor(a) for a in arrs)
        mk = e.tensor(mask)
        A, O = fwd(e, q, k, v, mk, BH, T, 0.125)
        q_old = e.clone(q)
        e.scale_inplace(q, 2.0)
        gS, gq, gk, gv = bwd(e, q_old, k, v, A, g, BH, T, 0.125)
        return [O.numpy(), A.numpy(), gq.numpy(), gk.numpy(), gv.numpy(), q.numpy()]

    h, c = go(hip), go(cpu)
    for i, (a, b) in enumerate(zip(h, c)):
        assert nrm_err(a, b) <= (1e-5 if i in (1, 5) else 1e-3), i


def test_dropped_probabilities(hip, cpu):
    """A dropped right after the forward: nothing else is computed, O is right, later calls unaffected."""
    B, H, T, dk = 1, 2, 64, 64
    BH = B * H
    mask = attn_mask(B, H, T)
    arrs = inputs(4, BH, T, dk)

    def go(e):
        q, k, v, g = (e.tensor(a) for a in arrs)
        mk = e.tensor(mask)
        A, O = fwd(e, q, k, v, mk, BH, T, 0.125)
        del A
        s = e.row_reduce_sum(O)
        return [O.numpy(), s.numpy()]

    h, c = go(hip), go(cpu)
    assert nrm_err(h[0], c[0]) <= 1e-4 and nrm_err(h[1], c[1]) <= 1e-4


def test_chain_config4_shape(hip, cpu):
    """The config-4 attention of one layer (B8 x H12, T1024, d64, ALiBi): the forward
    runs one cell per step here."""
    B, H, T, dk = 8, 12, 1024, 64
    mask = attn_mask(B, H, T)
    arrs = inputs(17, B * H, T, dk)
    check(run(hip, arrs, mask, B * H, T, 0.125), run(cpu, arrs, mask, B * H, T, 0.125))
