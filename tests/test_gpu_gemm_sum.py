"""The attention's input gradient as one product (reference compute_layer.hpp:1397-1408):
dx = Wq^T gQ; dx += Wk^T gK; dx += Wv^T gV. HipEngine records the two in-place adds onto the still
recorded first product and launches nnhip_gemm_tn_sum, one product over K = 3 d_model in segment
order (include/nnhip_kernels.h). Bars: float64 with the GEMM tolerance (normwise 1e-5 and the
elementwise a-priori bound |dC| <= 2K 2^-24 (sum |A_i|^T |B_i|)_ij) for the engine call pattern and
the entry point directly, the folded products still readable afterwards, a write to an operand
between the calls, and a GPT block whose backward takes this path against the oracle (the GPT
parity tests cover the whole model).

Weight-gradient accumulations (Linear::backward's grad_w += G X^T) are recorded, up to four of one
shape grouped into one launch (the attention's output, q, k and v layers: nnhip_gemm_group_acc with
one X, nnhip_gemm_group_acc_each with a B per member), and the layer's bias row sums
(grad_b += row_reduce_sum(G)) are computed by the same launch from the G tiles it stages: checked
against float64 with the summation bound |d| <= 2K 2^-24 sum|G| per row, added or written (a bias
gradient whose zero fill is still pending), with the row-sum tensors still readable."""
import ctypes

import numpy as np
import pytest

import nnengine
from helpers import nrm_err, uniform

pytestmark = pytest.mark.gpu
SZ = ctypes.c_size_t


def _check(got, As, Bs):
    ref = sum(a.astype(np.float64).T @ b.astype(np.float64) for a, b in zip(As, Bs))
    mag = sum(np.abs(a.astype(np.float64)).T @ np.abs(b.astype(np.float64)) for a, b in zip(As, Bs))
    K = sum(a.shape[0] for a in As)
    assert nrm_err(got, ref) <= 1e-5
    assert np.all(np.abs(got - ref) <= 2 * K * 2.0 ** -24 * mag + 1e-30)


@pytest.mark.parametrize("M,N,d", [(768, 8192, 768), (64, 200, 48), (96, 36, 16)])
def test_layer_pattern_sums_three_products(hip, M, N, d):
    rng = np.random.default_rng(M + N)
    Ws = [uniform(rng, (d, M)) for _ in range(3)]          # Linear weights (out d, in M)
    Gs = [uniform(rng, (d, N)) for _ in range(3)]          # output gradients
    X = uniform(rng, (M, N))
    w = [hip.tensor(a) for a in Ws]
    g = [hip.tensor(a) for a in Gs]
    x = hip.tensor(X)
    outs = []
    for i in range(3):                                      # Linear::backward's calls, then the adds
        outs.append(hip.matmul(w[i], g[i], True, False))
        _gw = hip.matmul(g[i], x, False, True)
        if i == 1:
            hip.add_inplace(outs[0], outs[1])
        if i == 2:
            hip.add_inplace(outs[0], outs[2])
    _check(outs[0].numpy(), Ws, Gs)
    for i in (1, 2):                                        # the added products still read as themselves
        _check(outs[i].numpy(), [Ws[i]], [Gs[i]])


def test_operand_written_before_read(hip):
    rng = np.random.default_rng(5)
    M, N, d = 128, 96, 64
    Ws, Gs = [uniform(rng, (d, M)) for _ in range(2)], [uniform(rng, (d, N)) for _ in range(2)]
    w, g = [hip.tensor(a) for a in Ws], [hip.tensor(a) for a in Gs]
    dx = hip.matmul(w[0], g[0], True, False)
    dk = hip.matmul(w[1], g[1], True, False)
    hip.add_inplace(dx, dk)
    hip.scale_inplace(w[1], 2.0)                            # the recorded sum runs before this write
    _check(dx.numpy(), Ws, Gs)
    assert np.allclose(w[1].numpy(), 2 * Ws[1])


@pytest.mark.parametrize("count,M,N,K", [(3, 768, 8192, 768), (2, 100, 36, 32), (1, 64, 64, 16), (3, 132, 260, 48)])
def test_entry_point(hip, count, M, N, K):
    lib = nnengine.hip_library()
    lib.nnhip_gemm_workspace_bytes.restype = SZ
    lib.nnhip_gemm_workspace_bytes.argtypes = [SZ] * 4
    lib.nnhip_gemm_tn_sum.argtypes = [ctypes.c_void_p, ctypes.c_void_p, SZ, ctypes.c_void_p, SZ, SZ, SZ,
                                      ctypes.c_float, ctypes.c_void_p, SZ, ctypes.c_void_p]
    lib.nnhip_engine_stream.restype = ctypes.c_void_p
    lib.nnhip_engine_stream.argtypes = [ctypes.c_void_p]
    rng = np.random.default_rng(count * M + K)
    As, Bs = [uniform(rng, (K, M)) for _ in range(count)], [uniform(rng, (K, N)) for _ in range(count)]
    a, b = [hip.tensor(x) for x in As], [hip.tensor(x) for x in Bs]
    c = hip.create_tensor(M, N)
    wsb = lib.nnhip_gemm_workspace_bytes(M, N, count * K, 1)
    ws = hip.create_tensor(max(1, wsb // 4), 1)
    hip.sync()
    pa = (ctypes.c_void_p * 3)(*[t.data_ptr() for t in a])
    pb = (ctypes.c_void_p * 3)(*[t.data_ptr() for t in b])
    print(f"[tn_sum] count {count} M {M} N {N} K {K} ws {wsb}", flush=True)
    rc = lib.nnhip_gemm_tn_sum(pa, pb, count, c.data_ptr(), M, N, K, 1.0, ws.data_ptr() if wsb else None, wsb,
                               lib.nnhip_engine_stream(hip._e))
    assert rc == 0
    _check(c.numpy(), As, Bs)
    assert lib.nnhip_gemm_tn_sum(pa, pb, 4, c.data_ptr(), M, N, K, 1.0, None, 0, None) == -1   # count > 3
    assert lib.nnhip_gemm_tn_sum(pa, pb, count, c.data_ptr(), M, N, 24, 1.0, None, 0, None) == -1   # K % 16


# ── grouped weight-gradient accumulations (nnhip_gemm_group_acc) ──────────────
def _acc_ref(W0, G, X):
    return W0.astype(np.float64) + G.astype(np.float64) @ X.astype(np.float64).T


def _check_acc(got, W0, G, X):
    ref = _acc_ref(W0, G, X)
    mag = np.abs(W0.astype(np.float64)) + np.abs(G.astype(np.float64)) @ np.abs(X.astype(np.float64)).T
    assert nrm_err(got, ref) <= 1e-5
    assert np.all(np.abs(got - ref) <= 2 * (X.shape[1] + 1) * 2.0 ** -24 * mag + 1e-30)


@pytest.mark.parametrize("M,K,N,cut", [(768, 768, 8192, None), (96, 64, 2048, None), (96, 64, 2048, "read"),
                                       (96, 64, 2048, "write_x")])
def test_weight_gradients_sharing_input(hip, M, K, N, cut):
    """Linear::backward's grad_w += G X^T for three layers with one input X (the q, k, v projections):
    recorded and run as one grouped launch; `cut` reads the first gradient, or writes X in place, after
    the second accumulation (the recorded ones run first)."""
    rng = np.random.default_rng(M + K + N)
    X = uniform(rng, (K, N))
    Gs = [uniform(rng, (M, N)) for _ in range(3)]
    W0 = [uniform(rng, (M, K)) for _ in range(3)]
    x = hip.tensor(X)
    gw = [hip.tensor(w) for w in W0]
    early = None
    for i in range(3):
        hip.add_inplace(gw[i], hip.matmul(hip.tensor(Gs[i]), x, False, True))
        if i == 1 and cut == "read":
            early = gw[0].numpy()
        if i == 1 and cut == "write_x":
            hip.scale_inplace(x, 0.5)
    X3 = X * (0.5 if cut == "write_x" else 1.0)
    for i in range(3):
        _check_acc(gw[i].numpy(), W0[i], Gs[i], X3 if i == 2 else X)
    if early is not None:
        _check_acc(early, W0[0], Gs[0], X)


def _rows_ref(r0, A, acc):
    return (r0.astype(np.float64) if acc else 0.0) + A.astype(np.float64).sum(axis=1, keepdims=True)


def _check_rows(got, r0, A, acc):
    """Row sums of A over k (+ r0): normwise 1e-5 and |d| <= 2K 2^-24 sum |A| (+ |r0|) per row."""
    ref = _rows_ref(r0, A, acc)
    mag = np.abs(A.astype(np.float64)).sum(axis=1, keepdims=True) + (np.abs(r0) if acc else 0.0)
    assert nrm_err(got, ref) <= 1e-5
    assert np.all(np.abs(got - ref) <= 2 * (A.shape[1] + 1) * 2.0 ** -24 * mag + 1e-30)


@pytest.mark.parametrize("count,M,N,K,tB,rows", [(3, 768, 768, 8192, True, 1), (2, 100, 36, 3000, True, 0),
                                                 (3, 64, 128, 512, False, 1), (1, 96, 64, 2048, True, 2),
                                                 (1, 100, 36, 300, True, 1), (3, 768, 3072, 8192, True, 2)])
def test_group_acc_entry_point(hip, count, M, N, K, tB, rows):
    """rows: 0 no row sums, 1 row sums added to their destination, 2 written."""
    lib = nnengine.hip_library()
    lib.nnhip_gemm_workspace_bytes.restype = SZ
    lib.nnhip_gemm_workspace_bytes.argtypes = [SZ] * 4
    lib.nnhip_gemm_group_acc.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, SZ, SZ, SZ, SZ,
                                         ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p,
                                         SZ, ctypes.c_void_p]
    lib.nnhip_engine_stream.restype = ctypes.c_void_p
    lib.nnhip_engine_stream.argtypes = [ctypes.c_void_p]
    rng = np.random.default_rng(count * M + K)
    As = [uniform(rng, (M, K)) for _ in range(count)]
    Bm = uniform(rng, (N, K) if tB else (K, N))
    C0 = [uniform(rng, (M, N)) for _ in range(count)]
    a, c = [hip.tensor(x) for x in As], [hip.tensor(x) for x in C0]
    b = hip.tensor(Bm)
    wsb = lib.nnhip_gemm_workspace_bytes(M, N, K, count)
    ws = hip.create_tensor(max(1, wsb // 4), 1)
    hip.sync()
    R0 = [uniform(rng, (M, 1)) for _ in range(count)]
    r = [hip.tensor(x) for x in R0]
    hip.sync()
    pa = (ctypes.c_void_p * count)(*[t.data_ptr() for t in a])
    pc = (ctypes.c_void_p * count)(*[t.data_ptr() for t in c])
    pr = (ctypes.c_void_p * count)(*[t.data_ptr() for t in r])
    print(f"[group_acc] count {count} M {M} N {N} K {K} tB {tB} rows {rows} ws {wsb}", flush=True)
    assert lib.nnhip_gemm_group_acc(pa, b.data_ptr(), pc, count, M, N, K, int(tB), 1, pr if rows else None,
                                    int(rows == 1), ws.data_ptr() if wsb else None, wsb,
                                    lib.nnhip_engine_stream(hip._e)) == 0
    Xt = Bm if tB else Bm.T          # (N, K): C += A X^T
    for i in range(count):
        _check_acc(c[i].numpy(), C0[i], As[i], np.ascontiguousarray(Xt))
        if rows:
            _check_rows(r[i].numpy(), R0[i], As[i], rows == 1)
        else:
            assert np.array_equal(r[i].numpy(), R0[i])


def _lib_each():
    lib = nnengine.hip_library()
    lib.nnhip_gemm_workspace_bytes.restype = SZ
    lib.nnhip_gemm_workspace_bytes.argtypes = [SZ] * 4
    P = ctypes.c_void_p
    lib.nnhip_gemm_group_acc_each.argtypes = [P, P, P, SZ, SZ, SZ, SZ, ctypes.c_int, ctypes.c_int, P, ctypes.c_int,
                                              P, SZ, P]
    lib.nnhip_engine_stream.restype = ctypes.c_void_p
    lib.nnhip_engine_stream.argtypes = [ctypes.c_void_p]
    return lib


@pytest.mark.parametrize("count,M,N,K,tB,rows", [(4, 768, 768, 8192, True, 1), (4, 96, 64, 2048, True, 2),
                                                 (2, 100, 36, 3000, True, 0), (4, 64, 128, 512, False, 1),
                                                 (3, 256, 256, 4096, True, 2)])
def test_group_acc_each_entry_point(hip, count, M, N, K, tB, rows):
    """nnhip_gemm_group_acc_each: C_i += A_i op(B_i) with a B of each member (the attention's output,
    q, k and v weight gradients); rows: 0 no row sums, 1 added to their destination, 2 written."""
    lib = _lib_each()
    rng = np.random.default_rng(count * M + K + 5)
    As = [uniform(rng, (M, K)) for _ in range(count)]
    Bs = [uniform(rng, (N, K) if tB else (K, N)) for _ in range(count)]
    C0 = [uniform(rng, (M, N)) for _ in range(count)]
    R0 = [uniform(rng, (M, 1)) for _ in range(count)]
    a, b = [hip.tensor(x) for x in As], [hip.tensor(x) for x in Bs]
    c, r = [hip.tensor(x) for x in C0], [hip.tensor(x) for x in R0]
    wsb = lib.nnhip_gemm_workspace_bytes(M, N, K, count)
    ws = hip.create_tensor(max(1, wsb // 4), 1)
    hip.sync()
    arr = lambda ts: (ctypes.c_void_p * count)(*[t.data_ptr() for t in ts])
    print(f"[group_acc_each] count {count} M {M} N {N} K {K} tB {tB} rows {rows} ws {wsb}", flush=True)
    assert lib.nnhip_gemm_group_acc_each(arr(a), arr(b), arr(c), count, M, N, K, int(tB), 1,
                                         arr(r) if rows else None, int(rows == 1), ws.data_ptr() if wsb else None,
                                         wsb, lib.nnhip_engine_stream(hip._e)) == 0
    for i in range(count):
        Xt = np.ascontiguousarray(Bs[i] if tB else Bs[i].T)
        _check_acc(c[i].numpy(), C0[i], As[i], Xt)
        if rows:
            _check_rows(r[i].numpy(), R0[i], As[i], rows == 1)
        else:
            assert np.array_equal(r[i].numpy(), R0[i])


def test_group_acc_each_argument_errors(hip):
    lib = _lib_each()
    t = hip.create_tensor(64, 64)
    p = t.data_ptr()
    five = (ctypes.c_void_p * 5)(*([p] * 5))
    assert lib.nnhip_gemm_group_acc_each(five, five, five, 5, 64, 64, 64, 1, 1, None, 0, None, 0, None) == -1
    holes = (ctypes.c_void_p * 2)(p, None)
    two = (ctypes.c_void_p * 2)(p, p)
    assert lib.nnhip_gemm_group_acc_each(two, holes, two, 2, 64, 64, 64, 1, 1, None, 0, None, 0, None) == -1
    assert lib.nnhip_gemm_group_acc_each(two, None, two, 2, 64, 64, 64, 1, 1, None, 0, None, 0, None) == -1


@pytest.mark.parametrize("cut", [None, "read", "write_b0"])
def test_attention_weight_gradients_grouped(hip, cut):
    """The backward's order: the output projection's grad_w += G_o A^T (its own input A), then the q, k
    and v layers' with the block input X, each with its bias row sums: one launch of four members. `cut`
    reads the output projection's gradient, or writes its input A in place, after the q layer's calls
    (the recorded members run first)."""
    rng = np.random.default_rng(23)
    d, N = 192, 1024
    Xo, X = uniform(rng, (d, N)), uniform(rng, (d, N))
    Gs = [uniform(rng, (d, N)) for _ in range(4)]
    W0 = [uniform(rng, (d, d)) for _ in range(4)]
    B0 = [uniform(rng, (d, 1)) for _ in range(4)]
    xo, x = hip.tensor(Xo), hip.tensor(X)
    gw, gb = [hip.tensor(w) for w in W0], [hip.tensor(b) for b in B0]
    early = None
    for i in range(4):
        g = hip.tensor(Gs[i])
        hip.add_inplace(gw[i], hip.matmul(g, xo if i == 0 else x, False, True))
        hip.add_inplace(gb[i], hip.row_reduce_sum(g))
        if i == 1 and cut == "read":
            early = gw[0].numpy()
        if i == 1 and cut == "write_b0":
            hip.scale_inplace(xo, 0.5)
    for i in range(4):
        _check_acc(gw[i].numpy(), W0[i], Gs[i], Xo if i == 0 else X)
        _check_rows(gb[i].numpy(), B0[i], Gs[i], True)
    if early is not None:
        _check_acc(early, W0[0], Gs[0], Xo)
    if cut == "write_b0":
        assert np.array_equal(xo.numpy(), Xo * np.float32(0.5))


@pytest.mark.parametrize("fresh_b", [False, True])
def test_linear_backward_bias_sums_with_weight_gradients(hip, fresh_b):
    """Linear::backward's calls for the q, k, v layers (one X) and one more layer (another X):
    grad_w += G X^T and grad_b += row_reduce_sum(G), recorded and launched with the products; the
    bias gradients' zero fill still pending (fresh_b) makes the launch write the sums. The row-sum
    tensors themselves stay readable."""
    rng = np.random.default_rng(11 + fresh_b)
    d, N = 256, 2048
    X, X2 = uniform(rng, (d, N)), uniform(rng, (d, N))
    Gs = [uniform(rng, (d, N)) for _ in range(4)]
    W0 = [uniform(rng, (d, d)) for _ in range(4)]
    B0 = [uniform(rng, (d, 1)) for _ in range(4)]
    x, x2 = hip.tensor(X), hip.tensor(X2)
    gw, gb = [hip.tensor(w) for w in W0], [hip.tensor(b) for b in B0]
    if fresh_b:
        for t in gb:
            hip.zero(t)
    sums = []
    for i in range(4):
        g = hip.tensor(Gs[i])
        hip.add_inplace(gw[i], hip.matmul(g, x if i < 3 else x2, False, True))
        rsum = hip.row_reduce_sum(g)
        hip.add_inplace(gb[i], rsum)
        sums.append(rsum)
    for i in range(4):
        _check_acc(gw[i].numpy(), W0[i], Gs[i], X if i < 3 else X2)
        _check_rows(gb[i].numpy(), B0[i], Gs[i], not fresh_b)
        _check_rows(sums[i].numpy(), B0[i], Gs[i], False)
