"""Linear layer products with their next call folded into the GEMM epilogue.

Linear::forward is matmul(W, x) then broadcast_row_inplace(out, b, Add);
Linear::backward accumulates the weight gradient with add_inplace(grad_w,
matmul(g, x, transB)) (reference compute_layer.hpp:99-196). The HIP engine
records the matmul and, when that next call follows, adds the bias or
accumulates inside the product's epilogue. Bars: bit-exact against the same
calls launched one by one (an engine settle between them), the products within
the GEMM bound of the float64 product, and the recorded product itself correct
when read afterwards.
"""
import numpy as np
import pytest

from helpers import nrm_err, uniform

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


SHAPES = [(64, 48, 40), (768, 8192, 768), (6144, 768, 8192), (37, 29, 1500), (3, 5, 7), (768, 1, 768), (5, 1, 13)]


@pytest.mark.parametrize("M,N,K", SHAPES)
def test_bias_epilogue(hip, M, N, K):
    rng = np.random.default_rng(M + N + K)
    W, X, b = uniform(rng, (M, K)), uniform(rng, (K, N)), uniform(rng, (M, 1))

    def run(settle):
        w, x, bb = hip.tensor(W), hip.tensor(X), hip.tensor(b)
        out = hip.matmul(w, x)
        if settle:
            hip.settle()
        hip.broadcast_row_inplace(out, bb, "Add")
        return out.numpy()

    fused, calls = run(False), run(True)
    assert np.array_equal(bits(fused), bits(calls))
    ref = W.astype(np.float64) @ X.astype(np.float64) + b.astype(np.float64)
    assert nrm_err(fused, ref) <= 1e-5


@pytest.mark.parametrize("M,N,K", SHAPES)
def test_accumulate_epilogue(hip, M, N, K):
    rng = np.random.default_rng(3 * M + N + K)
    G, X, acc0 = uniform(rng, (M, K)), uniform(rng, (N, K)), uniform(rng, (M, N))

    def run(settle):
        g, x, acc = hip.tensor(G), hip.tensor(X), hip.tensor(acc0)
        gw = hip.matmul(g, x, False, True)
        if settle:
            hip.settle()
        hip.add_inplace(acc, gw)
        return acc.numpy(), gw.numpy()

    (fa, fg), (ca, cg) = run(False), run(True)
    assert np.array_equal(bits(fa), bits(ca))
    assert np.array_equal(bits(fg), bits(cg)), "the recorded product read after the accumulation"
    ref = G.astype(np.float64) @ X.astype(np.float64).T
    assert nrm_err(fg, ref) <= 1e-5
    assert nrm_err(fa, ref + acc0) <= 1e-5


def test_linear_forward_backward_sequence(hip, cpu):
    """A Linear layer's calls, forward then backward, twice, against the oracle."""
    rng = np.random.default_rng(1)
    O, I, N = 96, 80, 256
    W, b, X, G = uniform(rng, (O, I)), uniform(rng, (O, 1)), uniform(rng, (I, N)), uniform(rng, (O, N))

    def run(e):
        w, bb, x, g = e.tensor(W), e.tensor(b), e.tensor(X), e.tensor(G)
        gw_acc = e.tensor(np.zeros((O, I), np.float32))
        outs = []
        for _ in range(2):
            out = e.matmul(w, x)
            e.broadcast_row_inplace(out, bb, "Add")
            dx = e.matmul(w, g, True, False)
            gw = e.matmul(g, x, False, True)
            e.add_inplace(gw_acc, gw)
            del gw
            outs += [out.numpy(), dx.numpy()]
        outs.append(gw_acc.numpy())
        return outs

    h, c = run(hip), run(cpu)
    for i, (a, r) in enumerate(zip(h, c)):
        assert nrm_err(a, r) <= 1e-5, i


def test_other_consumers(hip):
    """A product followed by a call that is not its epilogue is launched as is."""
    rng = np.random.default_rng(2)
    A, B, v = uniform(rng, (40, 30)), uniform(rng, (30, 50)), uniform(rng, (40, 1))
    a, bm, vv = hip.tensor(A), hip.tensor(B), hip.tensor(v)
    c = hip.matmul(a, bm)
    hip.broadcast_row_inplace(c, vv, "Mul")            # not an Add: plain product, then the broadcast
    ref = (A.astype(np.float64) @ B.astype(np.float64)) * v
    assert nrm_err(c.numpy(), ref) <= 1e-5
    c2 = hip.matmul(a, bm)
    t = hip.transpose(c2)                               # another kind of call reads the product
    assert nrm_err(t.numpy(), (A.astype(np.float64) @ B.astype(np.float64)).T) <= 1e-5
    c3 = hip.matmul(a, bm)
    hip.scale_inplace(a, 2.0)                           # an input written before the product ran
    assert nrm_err(c3.numpy(), A.astype(np.float64) @ B.astype(np.float64)) <= 1e-5


@pytest.mark.parametrize("M,N,K,masked", [(32000, 2048, 768, True), (4096, 4096, 128, False), (1000, 520, 64, True),
                                          (300, 200, 64, False)])
def test_ce_from_product_statistics(hip, cpu, M, N, K, masked):
    """The lm_head Linear then sparse cross-entropy (compute_layer.hpp Linear::forward, compute_loss.hpp:229-309):
    matmul(W, x), broadcast_row_inplace(logits, b), col_softmax_sparse_forward(logits, ...). When the CE call
    reads the still-recorded product, the product's epilogue yields per-tile column statistics and the CE
    reads the logits once (shapes with >= 512 output tiles of 256 x 128; the others take the plain path).
    Bars: logits bit-exact against the calls launched one by one; gradient and loss within 1e-5 of the
    unfused HIP path and of the oracle."""
    rng = np.random.default_rng(M + N + K)
    W, X = uniform(rng, (M, K), -0.2, 0.2), uniform(rng, (K, N))
    b = uniform(rng, (M, 1))
    labels = rng.integers(0, M, size=N).astype(np.float32)
    labels[::13] = M + 1                       # invalid: zero column
    mask = (rng.random(N) > 0.1).astype(np.float32) if masked else None
    inv = 1.0 / N

    def run(e, settle):
        w, x, bb = e.tensor(W), e.tensor(X), e.tensor(b)
        lab = e.tensor(labels.reshape(1, -1))
        mk = e.tensor(mask.reshape(1, -1)) if masked else None
        logits = e.matmul(w, x)
        e.broadcast_row_inplace(logits, bb, "Add")
        if settle:
            e.settle()
        g, lv = e.col_softmax_sparse_forward(logits, lab, mk, M, inv)
        return logits.numpy(), g.numpy(), lv.numpy()

    fused, calls, ref = run(hip, False), run(hip, True), run(cpu, False)
    assert np.array_equal(bits(fused[0]), bits(calls[0]))
    for a, c, r in zip(fused[1:], calls[1:], ref[1:]):
        assert nrm_err(a, c) <= 1e-5
        assert nrm_err(a, r) <= 1e-5


def _heads(e, Ws, bs, X, B, T, how):
    """AttentionBase::forward's projections and head split: q, k, v = W x + b (matmul,
    broadcast_row_inplace), then rearrange_3d(., H_dk, B, T). "fold": as issued (the products
    write the heads' layout); "read": the projections read first (the separate calls); the
    un-split projections are read at the end either way."""
    x = e.tensor(X)
    outs = []
    for W, b in zip(Ws, bs):
        y = e.matmul(e.tensor(W), x)
        e.broadcast_row_inplace(y, e.tensor(b), "Add")
        outs.append(y)
    if how == "read":
        for y in outs:
            y.numpy()
    heads = [e.rearrange_3d(y, Ws[0].shape[0], B, T, False) for y in outs]
    return [h.numpy() for h in heads] + [y.numpy() for y in outs]


@pytest.mark.parametrize("D,B,T", [(768, 8, 1024), (64, 3, 40), (96, 2, 36)])
def test_projections_into_heads(hip, cpu, D, B, T):
    """nnhip_gemm_heads: the q / k / v products written in the heads' layout, bit-identical to
    the products then rearrange_3d, and the products themselves still correct when read later."""
    rng = np.random.default_rng(D + B + T)
    X = uniform(rng, (D, B * T))
    Ws = [uniform(rng, (D, D)) for _ in range(3)]
    bs = [uniform(rng, (D, 1)) for _ in range(3)]
    fold = _heads(hip, Ws, bs, X, B, T, "fold")
    sep = _heads(hip, Ws, bs, X, B, T, "read")
    for i, (a, b) in enumerate(zip(fold, sep)):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), i
    ref = _heads(cpu, Ws, bs, X, B, T, "read")
    for a, b in zip(fold, ref):
        assert nrm_err(a, b) <= 1e-5


def _out_proj_bwd_heads(e, W, G, B, T, how):
    """AttentionBase::backward's first steps: grad_concat = matmul(W_o, G, true, false) (Linear::backward),
    then rearrange_3d(grad_concat, H_dk, B, T). "fold": as issued (the product writes the heads' layout,
    grad_concat itself recorded as a merge of those rows); "read": grad_concat read first (the separate
    calls); "write_h": the head split scaled in place before grad_concat is read (the merge must see
    the rows as they were)."""
    gc = e.matmul(e.tensor(W), e.tensor(G), True, False)
    if how == "read":
        gc.numpy()
    h = e.rearrange_3d(gc, W.shape[1], B, T, False)
    hv = h.numpy()
    if how == "write_h":
        e.scale_inplace(h, 2.0)
    return [hv, gc.numpy()] + ([h.numpy()] if how == "write_h" else [])


@pytest.mark.parametrize("D,B,T", [(768, 8, 1024), (64, 3, 40), (96, 2, 36)])
def test_output_projection_backward_into_heads(hip, cpu, D, B, T):
    """nnhip_gemm_heads_ex (transposed W): the output projection's input gradient written in the heads'
    layout, bit-identical to the product then rearrange_3d; the product itself, read afterwards, comes
    from those rows and is bit-identical too, also after the rows were overwritten."""
    rng = np.random.default_rng(3 * D + B + T)
    W, G = uniform(rng, (D, D)), uniform(rng, (D, B * T))
    fold = _out_proj_bwd_heads(hip, W, G, B, T, "fold")
    sep = _out_proj_bwd_heads(hip, W, G, B, T, "read")
    for i, (a, b) in enumerate(zip(fold, sep)):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), i
    w = _out_proj_bwd_heads(hip, W, G, B, T, "write_h")
    assert np.array_equal(w[1].view(np.uint32), sep[1].view(np.uint32))
    assert np.array_equal(w[2], sep[0] * np.float32(2.0))
    ref = _out_proj_bwd_heads(cpu, W, G, B, T, "read")
    for a, b in zip(fold, ref):
        assert nrm_err(a, b) <= 1e-5
