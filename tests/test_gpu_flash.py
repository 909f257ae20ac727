"""GPU parity of the one-pass attention chains and of the engine's deferral rules.

HipEngine records the reference's two-pass attention calls (compute_layer.hpp:
1196-1221 forward, :1304-1327 backward) and runs each chain as one launch
(csrc/k_flash.hip). Every test issues the reference's call sequence on the HIP
engine and on the CPU oracle and compares all outputs, including ones read in
the middle of a chain, after in-place writes to a chain's operands, and for
products that the fused backward never materialises (dP).
Tolerances: m, l 1e-5; O, R 1e-4; dQ, dK, dV 1e-3 (normwise).
"""
import numpy as np
import pytest

from helpers import causal_mask, doc_ids_from_lengths, doc_lengths, doc_mask, normal, nrm_err

pytestmark = pytest.mark.gpu


def _mask(kind, M, N, rng):
    if kind is None:
        return None
    if kind == "causal":
        return np.where(np.arange(N)[None, :] > np.arange(M)[:, None] + (N - M), -np.inf, 0.0).astype(np.float32)
    if kind == "doc":
        ids = doc_ids_from_lengths(doc_lengths(rng, M, 8, 80))
        return doc_mask(ids)[:, :N] if N <= M else None
    if kind == "alibi":   # finite additive bias on allowed pairs, -inf above the diagonal
        i, j = np.arange(M)[:, None], np.arange(N)[None, :]
        return np.where(j > i + (N - M), -np.inf, -0.25 * np.abs(i - j)).astype(np.float32)
    raise ValueError(kind)


def _chain(e, Q, K, V, dO, Vp, G, mask, batch, alpha, alpha2=1.0, reads=()):
    """The reference's forward then backward call sequence; `reads` names tensors
    downloaded in the middle of the chain (each forces deferred work to run)."""
    q, k, mk = e.tensor(Q), e.tensor(K), (e.tensor(mask) if mask is not None else None)
    mid = {}
    m = e.batched_matmul_reduce(q, k, batch, "Max", True, False, alpha, True, mk)
    if "m" in reads:
        mid["m"] = m.numpy()
    l = e.batched_matmul_softmax_denom(q, k, m, batch, True, False, alpha, mk)
    if "l" in reads:
        mid["l"] = l.numpy()
    o = e.batched_matmul_softmax_apply(q, k, e.tensor(V), m, l, batch, True, False, alpha, mk)
    g, vp = e.tensor(dO), e.tensor(Vp)
    P = e.batched_matmul(g, vp, batch, True, False, alpha2)
    if "P" in reads:
        mid["P"] = P.numpy()
    dq, r = e.batched_matmul_softmax_backward_q(q, k, P, m, l, batch, True, False, alpha, mk)
    if "dq" in reads:
        mid["dq"] = dq.numpy()
    dk, dv = e.batched_matmul_softmax_backward_kv(q, k, P, e.tensor(G), r, m, l, batch, True, False, alpha, mk)
    out = dict(m=m.numpy(), l=l.numpy(), O=o.numpy(), dQ=dq.numpy(), R=r.numpy(), dK=dk.numpy(), dV=dv.numpy())
    if "P_after" in reads:
        out["P"] = P.numpy()
    return out, mid


TOL = dict(m=1e-5, l=1e-5, O=1e-4, R=1e-4, dQ=1e-3, dK=1e-3, dV=1e-3, P=1e-5, dq=1e-3)

SHAPES = [  # batch, M, N, K, Kd, D
    (2, 64, 64, 64, 64, 64),
    (3, 70, 70, 64, 64, 64),
    (2, 33, 95, 32, 32, 32),
    (4, 128, 128, 8, 8, 4),
    (2, 100, 64, 48, 40, 40),
    (1, 1024, 1024, 64, 64, 64),   # one batch entry: rows are split into ranges and combined
    (2, 96, 160, 16, 60, 16),      # dP's inner dim differs from the head dim
]


def _inputs(rng, batch, M, N, K, Kd, D):
    Q, Kt = normal(rng, (batch * K, M)), normal(rng, (batch * K, N))
    V = normal(rng, (batch * N, D))
    dO, Vp = normal(rng, (batch * Kd, M)), normal(rng, (batch * Kd, N))
    G = normal(rng, (batch * M, max(K, D) + 4))
    return Q, Kt, V, dO, Vp, G


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("mask_kind", [None, "causal", "doc", "alibi"])
def test_chain(hip, cpu, shape, mask_kind):
    batch, M, N, K, Kd, D = shape
    rng = np.random.default_rng(sum(shape) + len(str(mask_kind)))
    mask = _mask(mask_kind, M, N, rng)
    if mask_kind == "doc" and mask is None:
        pytest.skip("doc masks are square")
    args = _inputs(rng, batch, M, N, K, Kd, D)
    alpha = 1.0 / np.sqrt(K)
    h, _ = _chain(hip, *args, mask, batch, alpha)
    c, _ = _chain(cpu, *args, mask, batch, alpha)
    for name in h:
        assert nrm_err(h[name], c[name]) <= TOL[name], name


def test_chain_alpha2(hip, cpu):
    """A scaled dP product (batched_matmul alpha != 1) is recomputed with its scale."""
    rng = np.random.default_rng(71)
    batch, M, N, K = 3, 96, 96, 64
    args = _inputs(rng, batch, M, N, K, K, K)
    mask = causal_mask(M)
    h, _ = _chain(hip, *args, mask, batch, 0.125, alpha2=0.37)
    c, _ = _chain(cpu, *args, mask, batch, 0.125, alpha2=0.37)
    for name in h:
        assert nrm_err(h[name], c[name]) <= TOL[name], name


@pytest.mark.parametrize("reads", [("m",), ("l",), ("m", "l"), ("P",), ("dq",), ("P_after",), ("m", "P", "dq")])
def test_reads_inside_chain(hip, cpu, reads):
    """Downloading a deferred result launches its work at once; the rest of the
    chain still matches the oracle (with the general kernels or the fused ones)."""
    rng = np.random.default_rng(9)
    batch, M, N, K = 2, 128, 128, 64
    args = _inputs(rng, batch, M, N, K, K, K)
    mask = causal_mask(M)
    h, hm = _chain(hip, *args, mask, batch, 0.125, reads=reads)
    c, cm = _chain(cpu, *args, mask, batch, 0.125, reads=reads)
    for name in h:
        assert nrm_err(h[name], c[name]) <= TOL[name], name
    for name in hm:
        assert nrm_err(hm[name], cm[name]) <= TOL[name], name


def test_inplace_write_between_calls(hip, cpu):
    """In-place writes to a deferred call's operands or results take effect in
    call order, as the reference's eager primitives do."""
    rng = np.random.default_rng(10)
    batch, M, N, K = 2, 96, 96, 64
    Q, Kt, V, dO, Vp, G = _inputs(rng, batch, M, N, K, K, K)
    mask = causal_mask(M)

    def run(e):
        q, k, mk = e.tensor(Q), e.tensor(Kt), e.tensor(mask)
        m = e.batched_matmul_reduce(q, k, batch, "Max", True, False, 0.125, True, mk)
        e.scale_inplace(q, 1.5)                     # denom / apply see the new Q, m the old one
        l = e.batched_matmul_softmax_denom(q, k, m, batch, True, False, 0.125, mk)
        o = e.batched_matmul_softmax_apply(q, k, e.tensor(V), m, l, batch, True, False, 0.125, mk)
        m2 = e.batched_matmul_reduce(q, k, batch, "Max", True, False, 0.125, True, mk)
        l2 = e.batched_matmul_softmax_denom(q, k, m2, batch, True, False, 0.125, mk)
        e.add_inplace(m2, m2)                       # writes a deferred result: m2, l2 computed first
        g, vp, gg = e.tensor(dO), e.tensor(Vp), e.tensor(G)
        P = e.batched_matmul(g, vp, batch, True, False)
        e.scale_inplace(g, -2.0)                    # P is the product of the old dO
        dq, r = e.batched_matmul_softmax_backward_q(q, k, P, m, l, batch, True, False, 0.125, mk)
        dk, dv = e.batched_matmul_softmax_backward_kv(q, k, P, gg, r, m, l, batch, True, False, 0.125, mk)
        P2 = e.batched_matmul(g, vp, batch, True, False)
        dq2, r2 = e.batched_matmul_softmax_backward_q(q, k, P2, m, l, batch, True, False, 0.125, mk)
        e.scale_inplace(P2, 0.5)                    # backward_q used the old P2, backward_kv the new one
        dk2, dv2 = e.batched_matmul_softmax_backward_kv(q, k, P2, gg, r2, m, l, batch, True, False, 0.125, mk)
        P3 = e.batched_matmul(g, vp, batch, True, False)
        dq3, r3 = e.batched_matmul_softmax_backward_q(q, k, P3, m, l, batch, True, False, 0.125, mk)
        e.scale_inplace(k, 0.75)                    # backward_q saw the old K, backward_kv the new one
        dk3, dv3 = e.batched_matmul_softmax_backward_kv(q, k, P3, gg, r3, m, l, batch, True, False, 0.125, mk)
        return [t.numpy() for t in (m, l, o, m2, l2, P, dq, r, dk, dv, g, P2, dq2, r2, dk2, dv2, dq3, r3, dk3,
                                    dv3)]

    h, c = run(hip), run(cpu)
    for i, (x, y) in enumerate(zip(h, c)):
        assert nrm_err(x, y) <= 1e-3, i


def test_dropped_and_unsupported(hip, cpu):
    """Deferred results that are dropped are never needed; a value width the
    one-pass kernels do not take (D % 4 != 0) falls back to the general kernels."""
    rng = np.random.default_rng(12)
    batch, M, N, K, D = 2, 64, 80, 32, 5
    Q, Kt, V = normal(rng, (batch * K, M)), normal(rng, (batch * K, N)), normal(rng, (batch * N, D))

    def run(e):
        q, k = e.tensor(Q), e.tensor(Kt)
        dead = e.batched_matmul_reduce(q, k, batch, "Max", True, False, 0.2, True, None)
        del dead
        dead = e.batched_matmul(q, k, batch, True, False)
        del dead
        m = e.batched_matmul_reduce(q, k, batch, "Max", True, False, 0.2, True, None)
        l = e.batched_matmul_softmax_denom(q, k, m, batch, True, False, 0.2, None)
        o = e.batched_matmul_softmax_apply(q, k, e.tensor(V), m, l, batch, True, False, 0.2, None)
        e.sync()
        return [t.numpy() for t in (m, l, o)]

    for x, y in zip(run(hip), run(cpu)):
        assert nrm_err(x, y) <= 1e-4


def test_config5_rows_back_to_back(hip, cpu):
    """Two config-5-style rows issued back to back (the second row's chain starts
    while the first row's dP product is still referenced)."""
    rng = np.random.default_rng(13)
    H, T, d = 3, 256, 64
    rows = []
    for _ in range(2):
        ids = doc_ids_from_lengths(doc_lengths(rng, T, 16, 128))
        rows.append((doc_mask(ids),) + tuple(normal(rng, (H * d, T)) for _ in range(4)))

    def run(e):
        out, keep = [], []
        for mask, Q, K, V, dO in rows:
            q, k, v, g, mk = e.tensor(Q), e.tensor(K), e.tensor(V), e.tensor(dO), e.tensor(mask)
            m = e.batched_matmul_reduce(q, k, H, "Max", True, False, 0.125, True, mk)
            l = e.batched_matmul_softmax_denom(q, k, m, H, True, False, 0.125, mk)
            vt = e.rearrange_3d(e.transpose(v), T, H, d)
            o = e.batched_matmul_softmax_apply(q, k, vt, m, l, H, True, False, 0.125, mk)
            P = e.batched_matmul(g, v, H, True, False)
            G = e.rearrange_3d(e.transpose(g), T, H, d)
            dq, r = e.batched_matmul_softmax_backward_q(q, k, P, m, l, H, True, False, 0.125, mk)
            dk, dv = e.batched_matmul_softmax_backward_kv(q, k, P, G, r, m, l, H, True, False, 0.125, mk)
            keep.append(P)
            out += [o, dq, r, dk, dv]
        out.append(keep[0])
        return [t.numpy() for t in out]

    for i, (x, y) in enumerate(zip(run(hip), run(cpu))):
        assert nrm_err(x, y) <= 1e-3, i


def test_forward_long_lines_float64(hip):
    """Lines of >= 32 cells in one range (64 heads x 1024 keys: the one-cell-per-step
    forward), against a float64 softmax attention (the oracle's serial primitives
    would take minutes at this size)."""
    B, M, N, K, D = 64, 1024, 1024, 64, 64
    rng = np.random.default_rng(21)
    Q, Kt, V = normal(rng, (B * K, M)), normal(rng, (B * K, N)), normal(rng, (B * N, D))
    mask = _mask("alibi", M, N, rng)
    alpha = 0.125
    q, k, mk = hip.tensor(Q), hip.tensor(Kt), hip.tensor(mask)
    m = hip.batched_matmul_reduce(q, k, B, "Max", True, False, alpha, True, mk)
    l = hip.batched_matmul_softmax_denom(q, k, m, B, True, False, alpha, mk)
    o = hip.batched_matmul_softmax_apply(q, k, hip.tensor(V), m, l, B, True, False, alpha, mk).numpy()
    m, l = m.numpy().reshape(B, M), l.numpy().reshape(B, M)
    for b in range(0, B, 9):
        s = alpha * (Q[b * K:(b + 1) * K].astype(np.float64).T @ Kt[b * K:(b + 1) * K].astype(np.float64)) + mask
        mr = s.max(axis=1)
        w = np.exp(s - mr[:, None])
        lr = w.sum(axis=1)
        orf = (w / lr[:, None]) @ V[b * N:(b + 1) * N].astype(np.float64)
        assert nrm_err(m[b], mr) <= 1e-5 and nrm_err(l[b], lr) <= 1e-5
        assert nrm_err(o[b * M:(b + 1) * M], orf) <= 1e-4, b
