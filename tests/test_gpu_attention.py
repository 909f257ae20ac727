"""GPU parity of the fused attention primitives (compute_engine.hpp:217-276).

Small and ragged shapes, every transpose combination, head dims on both sides
of the matrix-core limit (K <= 128) and masks whose 32x32 cells are fully
blocked, all zero, or general, against the oracle; and the full BASELINE
config-2 (causal forward) and one config-5 row (document-masked forward +
backward) against a dense float64 torch computation of the same attention on
the CPU (torch's own HIP runtime cannot share a process with the engine's).
"""
import numpy as np
import pytest

from helpers import causal_mask, doc_ids_from_lengths, doc_lengths, doc_mask, normal, nrm_err, uniform

pytestmark = pytest.mark.gpu


def both(hip, cpu, fn):
    return [[t.numpy() for t in fn(e)] for e in (hip, cpu)]


def _mask(kind, M, N, rng):
    if kind is None:
        return None
    if kind == "causal":   # key j visible to query i when j <= i + (N - M)
        return np.where(np.arange(N)[None, :] > np.arange(M)[:, None] + (N - M), -np.inf, 0.0).astype(np.float32)
    u = rng.uniform(size=(M, N))
    m = np.where(u < 0.3, -np.inf, np.where(u < 0.6, rng.normal(size=(M, N)), 0.0)).astype(np.float32)
    m[: min(M, 40), : min(N, 40)] = -np.inf     # fully blocked cells
    m[: min(M, 40), min(N, 40):] = np.where(m[: min(M, 40), min(N, 40):] == -np.inf, -np.inf, 0.0)
    if M > 70 and N > 70:
        m[64:, 64:] = 0.0                        # all-zero cells
    return m


def _run_all(e, A, B, V, P, G, mask, batch, tA, tB, alpha):
    a, b = e.tensor(A), e.tensor(B)
    mk = e.tensor(mask) if mask is not None else None
    m = e.batched_matmul_reduce(a, b, batch, "Max", tA, tB, alpha, True, mk)
    l = e.batched_matmul_softmax_denom(a, b, m, batch, tA, tB, alpha, mk)
    o = e.batched_matmul_softmax_apply(a, b, e.tensor(V), m, l, batch, tA, tB, alpha, mk)
    dq, r = e.batched_matmul_softmax_backward_q(a, b, e.tensor(P), m, l, batch, tA, tB, alpha, mk)
    dk, dv = e.batched_matmul_softmax_backward_kv(a, b, e.tensor(P), e.tensor(G), r, m, l, batch, tA, tB, alpha, mk)
    return [m, l, o, dq, r, dk, dv]


SHAPES = [  # batch, M, N, K, D
    (3, 37, 53, 1, 1),
    (2, 70, 130, 31, 40),
    (2, 96, 64, 64, 64),
    (2, 96, 100, 65, 100),
    (1, 64, 200, 128, 128),
    (2, 33, 47, 129, 129),   # beyond the matrix-core limit: general path
]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("mask_kind", [None, "causal", "mixed"])
@pytest.mark.parametrize("tA,tB", [(True, False), (False, True)])
def test_attention_primitives(hip, cpu, shape, mask_kind, tA, tB):
    batch, M, N, K, D = shape
    rng = np.random.default_rng(sum(shape) * 7 + (mask_kind is None) + 2 * tA)
    A = normal(rng, (batch * (K if tA else M), M if tA else K))
    B = normal(rng, (batch * (N if tB else K), K if tB else N))
    V, P, G = normal(rng, (batch * N, D)), normal(rng, (batch * M, N)), normal(rng, (batch * M, max(D, K)))
    mask = _mask(mask_kind, M, N, rng)
    alpha = 1.0 / np.sqrt(K)
    h, c = both(hip, cpu, lambda e: _run_all(e, A, B, V, P, G, mask, batch, tA, tB, alpha))
    tol = [1e-5, 1e-5, 1e-4, 1e-3, 1e-4, 1e-3, 1e-3]
    for name, x, y, t in zip(["m", "l", "O", "dQ", "R", "dK", "dV"], h, c, tol):
        assert nrm_err(x, y) <= t, name


def test_fully_masked_rows(hip, cpu):
    rng = np.random.default_rng(4)
    batch, M, N, K, D = 2, 64, 96, 64, 64
    mask = np.zeros((M, N), np.float32)
    mask[5] = -np.inf
    mask[33:40] = -np.inf
    A, B = normal(rng, (batch * K, M)), normal(rng, (batch * K, N))
    V, P, G = normal(rng, (batch * N, D)), normal(rng, (batch * M, N)), normal(rng, (batch * M, D))
    h, c = both(hip, cpu, lambda e: _run_all(e, A, B, V, P, G, mask, batch, True, False, 0.125))
    m, l, o = h[0][:, 0].reshape(batch, M), h[1][:, 0].reshape(batch, M), h[2].reshape(batch, M, D)
    assert np.all(m[:, 5] == np.finfo(np.float32).min) and np.all(l[:, 5] == 0) and np.all(o[:, 5] == 0)
    for x, y in zip(h, c):
        assert nrm_err(x, y) <= 1e-3


# ── full-size configurations against dense float64 torch (CPU) ────────────────
def _torch_attention(Q, K, V, mask, alpha, H, d, dO=None):
    import torch
    T = Q.shape[1]

    def heads(X):
        return torch.from_numpy(X).double().reshape(H, d, T).transpose(1, 2).contiguous()
    q, k, v = (heads(X).requires_grad_(dO is not None) for X in (Q, K, V))
    s = torch.matmul(q, k.transpose(1, 2)) * alpha + torch.from_numpy(mask).double()
    w = torch.softmax(s, dim=-1)
    o = torch.matmul(w, v)
    out = {"m": s.max(-1).values, "l": torch.exp(s - s.max(-1, keepdim=True).values).sum(-1), "O": o}
    if dO is not None:
        g = heads(dO)
        o.backward(g)
        out.update(dQ=q.grad.transpose(1, 2), dK=k.grad.transpose(1, 2), dV=v.grad.transpose(1, 2))
    return {n: t.detach().numpy() for n, t in out.items()}


def test_causal_attention_config2_full(hip):
    """BH 128 (B 16 x H 8), T 512, d 64, causal, alpha 1/8."""
    rng = np.random.default_rng(2)
    BH, T, d = 128, 512, 64
    Q, K, V = (normal(rng, (BH * d, T)) for _ in range(3))
    mask = causal_mask(T)
    e = hip
    q, k, mk = e.tensor(Q), e.tensor(K), e.tensor(mask)
    vt = e.rearrange_3d(e.transpose(e.tensor(V)), T, BH, d)          # (BH*T, d)
    m = e.batched_matmul_reduce(q, k, BH, "Max", True, False, 0.125, True, mk)
    l = e.batched_matmul_softmax_denom(q, k, m, BH, True, False, 0.125, mk)
    o = e.batched_matmul_softmax_apply(q, k, vt, m, l, BH, True, False, 0.125, mk)
    ref = _torch_attention(Q, K, V, mask, 0.125, BH, d)
    assert nrm_err(m.numpy()[:, 0], ref["m"].reshape(-1)) <= 1e-5
    assert nrm_err(l.numpy()[:, 0], ref["l"].reshape(-1)) <= 1e-5
    assert nrm_err(o.numpy(), ref["O"].reshape(BH * T, d)) <= 1e-4


def test_doc_masked_attention_config5_row(hip):
    """One BASELINE config-5 row: H 12, T 2048, d 64, documents U{64..1024}, forward + backward."""
    rng = np.random.default_rng(55)
    H, T, d = 12, 2048, 64
    ids = doc_ids_from_lengths(doc_lengths(rng, T, 64, 1024))
    mask = doc_mask(ids)
    Q, K, V, dO = (normal(rng, (H * d, T)) for _ in range(4))
    e = hip
    q, k, v, g, mk = e.tensor(Q), e.tensor(K), e.tensor(V), e.tensor(dO), e.tensor(mask)
    m = e.batched_matmul_reduce(q, k, H, "Max", True, False, 0.125, True, mk)
    l = e.batched_matmul_softmax_denom(q, k, m, H, True, False, 0.125, mk)
    vt = e.rearrange_3d(e.transpose(v), T, H, d)
    o = e.batched_matmul_softmax_apply(q, k, vt, m, l, H, True, False, 0.125, mk)
    P = e.batched_matmul(g, v, H, True, False)
    G = e.rearrange_3d(e.transpose(g), T, H, d)
    dq, r = e.batched_matmul_softmax_backward_q(q, k, P, m, l, H, True, False, 0.125, mk)
    dk, dv = e.batched_matmul_softmax_backward_kv(q, k, P, G, r, m, l, H, True, False, 0.125, mk)
    ref = _torch_attention(Q, K, V, mask, 0.125, H, d, dO)
    assert nrm_err(o.numpy(), ref["O"].reshape(H * T, d)) <= 1e-4
    # R_i = sum_j W_ij P_ij = dO_i . O_i
    R_ref = (dO.astype(np.float64).reshape(H, d, T).transpose(0, 2, 1) * ref["O"]).sum(-1)
    assert nrm_err(r.numpy()[:, 0], R_ref.reshape(-1)) <= 1e-4
    for name, t in (("dQ", dq), ("dK", dk), ("dV", dv)):
        assert nrm_err(t.numpy(), ref[name].reshape(H * d, T)) <= 1e-3, name


def test_fully_masked_tiles(hip, cpu):
    """Whole 32-row query tiles and 32-column key tiles without an allowed pair: their outputs
    (lowest() maxima, zero sums, rows and gradients) are still written."""
    rng = np.random.default_rng(6)
    batch, M, N, K, D = 3, 100, 130, 64, 64
    mask = np.zeros((M, N), np.float32)
    mask[:64] = -np.inf            # query tiles 0-1 fully blocked
    mask[:, 32:64] = -np.inf       # key tile 1 fully blocked
    mask[80:, 100:] = rng.normal(size=(20, 30)).astype(np.float32)   # general cells
    A, B = normal(rng, (batch * K, M)), normal(rng, (batch * K, N))
    V, P, G = normal(rng, (batch * N, D)), normal(rng, (batch * M, N)), normal(rng, (batch * M, D))
    h, c = both(hip, cpu, lambda e: _run_all(e, A, B, V, P, G, mask, batch, True, False, 0.125))
    m = h[0][:, 0].reshape(batch, M)
    assert np.all(m[:, :64] == np.finfo(np.float32).min)
    for name, x, y in zip(["m", "l", "O", "dQ", "R", "dK", "dV"], h, c):
        assert nrm_err(x, y) <= 1e-3, name
        assert np.array_equal(x == 0, y == 0) or name in ("m",), name
