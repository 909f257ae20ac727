"""GEMM operands stored by sequence (include/nnhip_kernels.h nnhip_by_seq).

The attention keeps its per-head tensors as (B * H * d_k, T): row (b, h, k) holds
sequence b's T values (reference compute_layer.hpp:1001-1010). rearrange_3d(x, H d_k,
B, T, inverse) turns them into the (H d_k, B * T) matrix the Linear layers take
(:1256-1259 for the attention output, :1377-1386 for the q, k, v gradients). The
sequence-stored entry points read those rows in place instead: column c of the
logical matrix at (c / len) * step + c % len, rows len apart.

Checked here, each against the entry point it replaces run on the rearranged matrix
(same plan, same summation order, so bit for bit) and against float64:

* nnhip_gemm_epilogue_seq (B by sequence along n, with a bias) against nnhip_gemm_epilogue;
* nnhip_gemm_tn_sum_seq (every B_i by sequence along n) against nnhip_gemm_tn_sum;
* nnhip_gemm_group_acc_seq with some members' A by sequence along k (the q, k, v
  gradients) and one member's transposed B by sequence along k (the output projection's
  input), with row sums, against nnhip_gemm_group_acc_each;
* shapes that do not give whole tiles return -7 and leave the outputs alone.
Bars: bit-identical to the replaced call; float64 normwise 1e-5.
"""
import ctypes

import numpy as np
import pytest

import nnengine
from helpers import nrm_err, uniform

pytestmark = pytest.mark.gpu
SZ, P = ctypes.c_size_t, ctypes.c_void_p


class BySeq(ctypes.Structure):
    _fields_ = [("len", SZ), ("step", SZ)]


def _lib():
    lib = nnengine.hip_library()
    lib.nnhip_gemm_workspace_bytes.restype = SZ
    lib.nnhip_gemm_workspace_bytes.argtypes = [SZ] * 4
    lib.nnhip_engine_stream.restype = P
    lib.nnhip_engine_stream.argtypes = [P]
    lib.nnhip_gemm_epilogue.argtypes = [P, P, P, SZ, SZ, SZ, SZ, ctypes.c_int, ctypes.c_int, ctypes.c_float, P,
                                        ctypes.c_int, P, SZ, P]
    lib.nnhip_gemm_epilogue_seq.argtypes = [P, P, P, SZ, SZ, SZ, ctypes.c_float, P, ctypes.c_int, BySeq, P, SZ, P]
    lib.nnhip_gemm_tn_sum.argtypes = [P, P, SZ, P, SZ, SZ, SZ, ctypes.c_float, P, SZ, P]
    lib.nnhip_gemm_tn_sum_seq.argtypes = [P, P, SZ, P, SZ, SZ, SZ, ctypes.c_float, BySeq, P, SZ, P]
    lib.nnhip_gemm_group_acc_each.argtypes = [P, P, P, SZ, SZ, SZ, SZ, ctypes.c_int, ctypes.c_int, P, ctypes.c_int,
                                              P, SZ, P]
    lib.nnhip_gemm_group_acc_seq.argtypes = [P, P, P, SZ, SZ, SZ, SZ, ctypes.c_int, ctypes.c_int, P, ctypes.c_int,
                                             P, P, P, SZ, P]
    return lib


def by_seq(X, nb, T):
    """(R, nb*T) -> the (nb*R, T) rows of each sequence, as the attention stores them."""
    R = X.shape[0]
    return np.ascontiguousarray(X.reshape(R, nb, T).transpose(1, 0, 2).reshape(nb * R, T))


def _ws(hip, lib, M, N, K, count):
    wsb = lib.nnhip_gemm_workspace_bytes(M, N, K, count)
    return wsb, hip.create_tensor(max(1, wsb // 4), 1)


def _arr(ts):
    return (P * len(ts))(*[t.data_ptr() for t in ts])


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.mark.parametrize("M,K,nb,T", [(768, 768, 8, 1024), (128, 64, 3, 256), (256, 96, 2, 128)])
def test_epilogue_seq(hip, M, K, nb, T):
    lib = _lib()
    rng = np.random.default_rng(M + K + nb * T)
    N = nb * T
    A, Bm, bias = uniform(rng, (M, K)), uniform(rng, (K, N)), uniform(rng, (M, 1))
    a, b, bs, bb = hip.tensor(A), hip.tensor(Bm), hip.tensor(by_seq(Bm, nb, T)), hip.tensor(bias)
    c1, c2 = hip.create_tensor(M, N), hip.create_tensor(M, N)
    wsb, ws = _ws(hip, lib, M, N, K, 1)
    hip.sync()
    st = lib.nnhip_engine_stream(hip._e)
    print(f"[gemm_seq] epilogue M {M} K {K} nb {nb} T {T}", flush=True)
    assert lib.nnhip_gemm_epilogue(a.data_ptr(), b.data_ptr(), c1.data_ptr(), M, K, K, N, 0, 0, 1.0, bb.data_ptr(), 0,
                                   ws.data_ptr() if wsb else None, wsb, st) == 0
    assert lib.nnhip_gemm_epilogue_seq(a.data_ptr(), bs.data_ptr(), c2.data_ptr(), M, N, K, 1.0, bb.data_ptr(), 0,
                                       BySeq(T, K * T), ws.data_ptr() if wsb else None, wsb, st) == 0
    r1, r2 = c1.numpy(), c2.numpy()
    assert np.array_equal(bits(r1), bits(r2))
    ref = A.astype(np.float64) @ Bm.astype(np.float64) + bias.astype(np.float64)
    assert nrm_err(r2, ref) <= 1e-5


@pytest.mark.parametrize("M,Ke,nb,T,count", [(768, 768, 8, 1024, 3), (128, 64, 3, 256, 3), (64, 32, 2, 128, 2)])
def test_tn_sum_seq(hip, M, Ke, nb, T, count):
    lib = _lib()
    rng = np.random.default_rng(M + Ke + nb + T + count)
    N = nb * T
    As = [uniform(rng, (Ke, M)) for _ in range(count)]
    Bs = [uniform(rng, (Ke, N)) for _ in range(count)]
    a = [hip.tensor(x) for x in As]
    b = [hip.tensor(x) for x in Bs]
    bq = [hip.tensor(by_seq(x, nb, T)) for x in Bs]
    c1, c2 = hip.create_tensor(M, N), hip.create_tensor(M, N)
    wsb, ws = _ws(hip, lib, M, N, count * Ke, 1)
    hip.sync()
    st = lib.nnhip_engine_stream(hip._e)
    print(f"[gemm_seq] tn_sum M {M} Ke {Ke} nb {nb} T {T} count {count}", flush=True)
    w = ws.data_ptr() if wsb else None
    assert lib.nnhip_gemm_tn_sum(_arr(a), _arr(b), count, c1.data_ptr(), M, N, Ke, 1.0, w, wsb, st) == 0
    assert lib.nnhip_gemm_tn_sum_seq(_arr(a), _arr(bq), count, c2.data_ptr(), M, N, Ke, 1.0, BySeq(T, Ke * T), w,
                                     wsb, st) == 0
    r1, r2 = c1.numpy(), c2.numpy()
    assert np.array_equal(bits(r1), bits(r2))
    ref = sum(x.astype(np.float64).T @ y.astype(np.float64) for x, y in zip(As, Bs))
    assert nrm_err(r2, ref) <= 1e-5


@pytest.mark.parametrize("d,nb,T,rows", [(768, 8, 1024, 1), (256, 4, 256, 2), (128, 2, 512, 0)])
def test_group_acc_seq(hip, d, nb, T, rows):
    """Four members of (d, d) over K = nb*T tokens: member 0 (the output projection) with A = G_o as
    it is and a transposed B (its input, (d, K)) by sequence; members 1-3 (q, k, v) with A = G_i by
    sequence and one plain X. rows: 0 no row sums, 1 added, 2 written."""
    lib = _lib()
    rng = np.random.default_rng(d + nb + T + rows)
    K = nb * T
    Gs = [uniform(rng, (d, K)) for _ in range(4)]
    Xo, X = uniform(rng, (d, K)), uniform(rng, (d, K))
    C0 = [uniform(rng, (d, d)) for _ in range(4)]
    R0 = [uniform(rng, (d, 1)) for _ in range(4)]
    g_plain = [hip.tensor(x) for x in Gs]
    g_seq = [g_plain[0]] + [hip.tensor(by_seq(x, nb, T)) for x in Gs[1:]]
    xo, xo_seq, x = hip.tensor(Xo), hip.tensor(by_seq(Xo, nb, T)), hip.tensor(X)
    c1, c2 = [hip.tensor(c) for c in C0], [hip.tensor(c) for c in C0]
    r1, r2 = [hip.tensor(r) for r in R0], [hip.tensor(r) for r in R0]
    wsb, ws = _ws(hip, lib, d, d, K, 4)
    hip.sync()
    st = lib.nnhip_engine_stream(hip._e)
    w = ws.data_ptr() if wsb else None
    print(f"[gemm_seq] group_acc d {d} nb {nb} T {T} rows {rows}", flush=True)
    assert lib.nnhip_gemm_group_acc_each(_arr(g_plain), _arr([xo, x, x, x]), _arr(c1), 4, d, d, K, 1, 1,
                                         _arr(r1) if rows else None, int(rows == 1), w, wsb, st) == 0
    a_seq = (BySeq * 4)(BySeq(0, 0), *[BySeq(T, d * T)] * 3)
    b_seq = (BySeq * 4)(BySeq(T, d * T), *[BySeq(0, 0)] * 3)
    assert lib.nnhip_gemm_group_acc_seq(_arr(g_seq), _arr([xo_seq, x, x, x]), _arr(c2), 4, d, d, K, 1, 1,
                                        _arr(r2) if rows else None, int(rows == 1), a_seq, b_seq, w, wsb, st) == 0
    for i in range(4):
        assert np.array_equal(bits(c1[i].numpy()), bits(c2[i].numpy())), i
        assert np.array_equal(bits(r1[i].numpy()), bits(r2[i].numpy())), i
        ref = C0[i].astype(np.float64) + Gs[i].astype(np.float64) @ (Xo if i == 0 else X).astype(np.float64).T
        assert nrm_err(c2[i].numpy(), ref) <= 1e-5, i


def test_partial_tiles_refused(hip):
    """-7 when the shapes do not give whole tiles; nothing is written."""
    lib = _lib()
    rng = np.random.default_rng(5)
    M, K, nb, T = 100, 64, 2, 128
    A, Bm = uniform(rng, (M, K)), uniform(rng, (K, nb * T))
    a, bs = hip.tensor(A), hip.tensor(by_seq(Bm, nb, T))
    c = hip.tensor(np.zeros((M, nb * T), np.float32))
    hip.sync()
    st = lib.nnhip_engine_stream(hip._e)
    assert lib.nnhip_gemm_epilogue_seq(a.data_ptr(), bs.data_ptr(), c.data_ptr(), M, nb * T, K, 1.0, None, 0,
                                       BySeq(T, K * T), None, 0, st) == -7
    assert not c.numpy().any()


# ── through the engine: rearrange_3d(., inverse) recorded, read in place ─────────
def _fwd(e, W, bias, S, d, nb, T, how):
    """AttentionBase::forward's end (compute_layer.hpp:1254-1267): concat = rearrange_3d(concat_out,
    H d_k, B, T, true), then the output projection W concat + b. how: "fold" as issued; "read" concat
    read before the product; "settle" a settle between the merge and the product (the merge stays
    recorded); "write_s" concat_out scaled in place after the product was recorded."""
    s = e.tensor(S)
    concat = e.rearrange_3d(s, d, nb, T, True)
    if how == "read":
        concat.numpy()
    if how == "settle":
        e.settle()
    y = e.matmul(e.tensor(W), concat)
    e.broadcast_row_inplace(y, e.tensor(bias), "Add")
    if how == "write_s":
        e.scale_inplace(s, 2.0)
    return [y.numpy(), concat.numpy()]


@pytest.mark.parametrize("d,nb,T", [(768, 8, 1024), (128, 3, 256), (100, 2, 48)])
def test_engine_output_projection_of_merge(hip, cpu, d, nb, T):
    """(100, 2, 48): not whole tiles, the merge is made and the product runs as usual."""
    rng = np.random.default_rng(d * nb + T)
    W, bias = uniform(rng, (d, d)), uniform(rng, (d, 1))
    S = uniform(rng, (nb * d, T))
    fold = _fwd(hip, W, bias, S, d, nb, T, "fold")
    for how in ("read", "settle", "write_s"):
        print(f"[gemm_seq] engine fwd d {d} nb {nb} T {T} {how}", flush=True)
        other = _fwd(hip, W, bias, S, d, nb, T, how)
        for i in range(2):
            assert np.array_equal(bits(fold[i]), bits(other[i])), (how, i)
    ref = _fwd(cpu, W, bias, S, d, nb, T, "read")
    for a, b in zip(fold, ref):
        assert nrm_err(a, b) <= 1e-5


def _bwd(e, Ws, Go, Xo_heads, X, dS, d, nb, T, how):
    """AttentionBase::backward's Linear part (compute_layer.hpp:1377-1408 and Linear::backward):
    the output projection's grad_w += G_o concat^T with concat a merge kept from the forward, then
    gQ, gK, gV = merges of the attention's heads' rows, each Linear's dx = W^T g, grad_w += g X^T,
    grad_b += row sums of g, the three dx summed. how: "fold" as issued; "read" every merge read
    first."""
    concat = e.rearrange_3d(e.tensor(Xo_heads), d, nb, T, True)
    x = e.tensor(X)
    gw = [e.tensor(np.zeros((d, d), np.float32)) for _ in range(4)]
    gb = [e.tensor(np.zeros((d, 1), np.float32)) for _ in range(4)]
    for t in gw + gb:
        e.zero(t)
    if how == "read":
        concat.numpy()
    go = e.tensor(Go)
    e.add_inplace(gw[0], e.matmul(go, concat, False, True))
    e.add_inplace(gb[0], e.row_reduce_sum(go))
    gs = [e.rearrange_3d(e.tensor(h), d, nb, T, True) for h in dS]
    if how == "read":
        for g in gs:
            g.numpy()
    dx = None
    for i, g in enumerate(gs):
        p = e.matmul(e.tensor(Ws[i]), g, True, False)
        if dx is None:
            dx = p
        else:
            e.add_inplace(dx, p)
        e.add_inplace(gw[i + 1], e.matmul(g, x, False, True))
        e.add_inplace(gb[i + 1], e.row_reduce_sum(g))
    return [dx.numpy()] + [t.numpy() for t in gw + gb]


@pytest.mark.parametrize("d,nb,T", [(768, 8, 1024), (128, 4, 256)])
def test_engine_attention_backward_linears_of_merges(hip, cpu, d, nb, T):
    """The merges read in place by the summed input gradient (nnhip_gemm_tn_sum_seq) and the grouped
    weight gradients with their row sums (nnhip_gemm_group_acc_seq): within the GEMM tolerance of the
    calls on the made merges (the input-gradient sum differs from three products and two adds), the
    weight gradients and row sums bit-identical (same grouped launch)."""
    rng = np.random.default_rng(d + nb * T)
    K = nb * T
    Ws = [uniform(rng, (d, d)) for _ in range(3)]
    Go, X = uniform(rng, (d, K)), uniform(rng, (d, K))
    Xo_heads = uniform(rng, (nb * d, T))
    dS = [uniform(rng, (nb * d, T)) for _ in range(3)]
    fold = _bwd(hip, Ws, Go, Xo_heads, X, dS, d, nb, T, "fold")
    sep = _bwd(hip, Ws, Go, Xo_heads, X, dS, d, nb, T, "read")
    ref = _bwd(cpu, Ws, Go, Xo_heads, X, dS, d, nb, T, "read")
    for i, (a, b, r) in enumerate(zip(fold, sep, ref)):
        if i > 0:
            assert np.array_equal(bits(a), bits(b)), i
        assert nrm_err(a, r) <= 1e-5, i
