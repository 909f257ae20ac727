"""Recorded transposes and the two-pass attention chain's backward variants.

The two-pass chain turns V and dO from per batch (d_k, seq) into (seq, d_k)
with transpose + rearrange_3d (reference compute_layer.hpp:1211-1214,
:1309-1313). The HIP engine records both calls: softmax_apply reads V from its
source, backward_kv reads G from dO, and any other reader of a recorded result
gets the copy. When the forward's output O is still referenced, backward_kv
takes R_i = dO_i . O_i from it and makes one score pass instead of two; with
whole 32 x 32 tiles (T 256, 512 here) that pass reads the scores the forward
kept instead of forming them again.

Bars: the recorded layouts bit-exact against numpy, including after in-place
writes to their source or result; every backward variant within 1e-4 (O, R)
and 1e-3 (gradients) of the oracle, all variants within 1e-4 of each other.
"""
import numpy as np
import pytest

from helpers import doc_ids_from_lengths, doc_lengths, doc_mask, normal, nrm_err, uniform

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def per_batch_t(S, B, N, M):
    """rearrange_3d(transpose(S), M, B, N): per batch b, the transpose of S rows [b*N, (b+1)*N)."""
    return S.reshape(B, N, M).transpose(0, 2, 1).reshape(B * M, N)


@pytest.mark.parametrize("B,N,M", [(3, 5, 7), (12, 64, 300), (4, 33, 64)])
def test_recorded_layouts_read(hip, B, N, M):
    rng = np.random.default_rng(B * N + M)
    S = uniform(rng, (B * N, M))
    s = hip.tensor(S)
    t = hip.transpose(s)
    p = hip.rearrange_3d(t, M, B, N)
    assert np.array_equal(bits(p.numpy()), bits(per_batch_t(S, B, N, M)))
    assert np.array_equal(bits(t.numpy()), bits(S.T))
    # inverse rearrange of a recorded transpose: the plain path, (2*Mp, Np) -> (Mp, 2*Np)
    if M % 2 == 0:
        Mp, Np = M // 2, B * N
        inv = hip.rearrange_3d(hip.transpose(s), Mp, 2, Np, True)
        ref = S.T.reshape(2, Mp, Np).transpose(1, 0, 2).reshape(Mp, 2 * Np)
        assert np.array_equal(bits(inv.numpy()), bits(ref))


def test_recorded_layouts_writes(hip):
    rng = np.random.default_rng(7)
    B, N, M = 6, 40, 24
    S = uniform(rng, (B * N, M))
    s = hip.tensor(S)
    t = hip.transpose(s)
    p = hip.rearrange_3d(t, M, B, N)
    hip.scale_inplace(s, 2.0)                      # source written: the records see its old values
    assert np.array_equal(bits(p.numpy()), bits(per_batch_t(S, B, N, M)))
    assert np.array_equal(bits(t.numpy()), bits(S.T))
    assert np.array_equal(bits(s.numpy()), bits(S * 2.0))
    p2 = hip.rearrange_3d(hip.transpose(s), M, B, N)
    hip.scale_inplace(p2, 0.5)                     # result written in place
    assert np.array_equal(bits(p2.numpy()), bits(per_batch_t(S * 2.0, B, N, M) * 0.5))
    q = hip.rearrange_3d(hip.transpose(s), M * B, 1, N)   # x (M, B*N) read with other dims: the plain path
    assert np.array_equal(bits(q.numpy()), bits((S * 2.0).T.reshape(M * B, N)))


def test_many_recorded_layouts(hip):
    """More pending transposes than the engine keeps: the oldest are launched early, all read correct."""
    rng = np.random.default_rng(8)
    Ss = [uniform(rng, (2 * 16, 8 + i)) for i in range(24)]
    outs = [hip.rearrange_3d(hip.transpose(hip.tensor(S)), S.shape[1], 2, 16) for S in Ss]
    hip.settle()
    for S, o in zip(Ss, outs):
        assert np.array_equal(bits(o.numpy()), bits(per_batch_t(S, 2, 16, S.shape[1])))


def _row(e, Q, K, V, dO, mask, H, variant):
    """The reference's two-pass call sequence for one packed row (compute_layer.hpp:1196-1221,
    :1304-1327), with the variant's change: "ds" keeps O (one score pass from R = dO . O); "no_o"
    drops the caller's O (the engine keeps its own reference for the backward: still one pass);
    "read_g" reads G before backward_kv (G copied out: two score passes reading G); "v_written"
    writes V in place between forward and backward, so the forward's O no longer matches and the
    backward makes two score passes reading dO's columns for G (it uses the new V, as the
    reference would)."""
    q, k, v, g = e.tensor(Q), e.tensor(K), e.tensor(V), e.tensor(dO)
    mk = e.tensor(mask) if mask is not None else None
    T, d = Q.shape[1], Q.shape[0] // H
    m = e.batched_matmul_reduce(q, k, H, "Max", True, False, 0.125, True, mk)
    l = e.batched_matmul_softmax_denom(q, k, m, H, True, False, 0.125, mk)
    vt = e.rearrange_3d(e.transpose(v), T, H, d)
    o = e.batched_matmul_softmax_apply(q, k, vt, m, l, H, True, False, 0.125, mk)
    out = {"O": o.numpy()}
    if variant == "no_o":
        del o
    if variant == "v_written":
        e.scale_inplace(v, 0.5)
    P = e.batched_matmul(g, v, H, True, False)
    G = e.rearrange_3d(e.transpose(g), T, H, d)
    if variant == "read_g":
        out["G"] = G.numpy()
    dq, r = e.batched_matmul_softmax_backward_q(q, k, P, m, l, H, True, False, 0.125, mk)
    dk, dv = e.batched_matmul_softmax_backward_kv(q, k, P, G, r, m, l, H, True, False, 0.125, mk)
    out.update(R=r.numpy(), dQ=dq.numpy(), dK=dk.numpy(), dV=dv.numpy(), Vt=vt.numpy())
    return out


@pytest.mark.parametrize("H,T,d,masked", [(4, 300, 64, True), (3, 256, 32, False), (2, 520, 64, True),
                                            (2, 512, 64, True)])
def test_two_pass_backward_variants(hip, cpu, H, T, d, masked):
    rng = np.random.default_rng(H * T + d)
    mask = doc_mask(doc_ids_from_lengths(doc_lengths(rng, T, 20, 200))) if masked else None
    Q, K, V, dO = (normal(rng, (H * d, T)) for _ in range(4))
    runs = {}
    for variant in ("ds", "no_o", "read_g", "v_written"):
        h, c = _row(hip, Q, K, V, dO, mask, H, variant), _row(cpu, Q, K, V, dO, mask, H, variant)
        print(f"[two-pass] H{H} T{T} d{d} masked={masked} {variant}", flush=True)
        for name in ("O", "R"):
            assert nrm_err(h[name], c[name]) <= 1e-4, (variant, name)
        for name in ("dQ", "dK", "dV"):
            assert nrm_err(h[name], c[name]) <= 1e-3, (variant, name)
        assert np.array_equal(bits(h["Vt"]), bits(per_batch_t(V, H, d, T)))
        if variant == "read_g":
            assert np.array_equal(bits(h["G"]), bits(per_batch_t(dO, H, d, T)))
        runs[variant] = h
    for variant in ("no_o", "read_g"):
        for name in ("R", "dQ", "dK", "dV"):
            assert nrm_err(runs["ds"][name], runs[variant][name]) <= 1e-4, (variant, name)


def test_more_two_pass_layers_than_kept(hip, cpu):
    """66 two-pass layers forward, then backward in reverse (as a deep model runs): the engine
    keeps the forward outputs and score blocks of the last 64; the first two layers' backward
    forms its scores again. Every layer's O, R and gradients match the oracle's."""
    rng = np.random.default_rng(66)
    L, H, T, d = 66, 2, 64, 32
    mask = doc_mask(doc_ids_from_lengths(doc_lengths(rng, T, 16, 48)))
    data = [[normal(rng, (H * d, T)) for _ in range(4)] for _ in range(L)]

    def model(e):
        mk = e.tensor(mask)
        state, out = [], []
        for Q, K, V, dO in data:
            q, k, v, g = e.tensor(Q), e.tensor(K), e.tensor(V), e.tensor(dO)
            m = e.batched_matmul_reduce(q, k, H, "Max", True, False, 0.125, True, mk)
            l = e.batched_matmul_softmax_denom(q, k, m, H, True, False, 0.125, mk)
            vt = e.rearrange_3d(e.transpose(v), T, H, d)
            o = e.batched_matmul_softmax_apply(q, k, vt, m, l, H, True, False, 0.125, mk)
            state.append((q, k, v, g, m, l, o))
        for q, k, v, g, m, l, o in reversed(state):
            P = e.batched_matmul(g, v, H, True, False)
            G = e.rearrange_3d(e.transpose(g), T, H, d)
            dq, r = e.batched_matmul_softmax_backward_q(q, k, P, m, l, H, True, False, 0.125, mk)
            dk, dv = e.batched_matmul_softmax_backward_kv(q, k, P, G, r, m, l, H, True, False, 0.125, mk)
            out.append([o.numpy(), r.numpy(), dq.numpy(), dk.numpy(), dv.numpy()])
        return out

    h, c = model(hip), model(cpu)
    for i, (a, b) in enumerate(zip(h, c)):
        for j, (x, y) in enumerate(zip(a, b)):
            assert nrm_err(x, y) <= (1e-4 if j < 2 else 1e-3), (i, j)
