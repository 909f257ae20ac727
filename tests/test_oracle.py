"""Pins the CPU oracle (oracle/, the restatement of the reference CpuEngine).

Each check is an independent computation: float64 numpy closed forms, dense
formulations of the fused primitives, torch float64 autograd, brute-force
loops for the index primitives, the reference's own known-answer mask rows
(src/doc_mask_test.cpp:49-104), its finite-difference gradcheck method
(src/gpt_gradcheck.cpp:124-261) and its document-invariance test
(src/doc_attn_test.cpp:75-152). The reference ships no stored vectors; its
sources need <expected>, which this image's libstdc++ lacks, so it cannot be
compiled here and every pin below is reference-free.
"""
import ctypes
import math

import numpy as np
import pytest
import torch

import torch_gpt
from helpers import causal_mask, doc_mask, grad_errs, normal, nrm_err, uniform
from nnengine import EngineError, ExprSpec, cst, inp, red, reg


def np64(x):
    return np.asarray(x, dtype=np.float64)


# ── GEMM ────────────────────────────────────────────────────────────────────
@pytest.mark.parametrize("tA,tB", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (5, 7, 3), (64, 64, 64), (65, 130, 129), (200, 33, 300)])
def test_matmul_vs_float64(cpu, M, N, K, tA, tB):
    rng = np.random.default_rng(M + 7 * N + 13 * K)
    A = uniform(rng, (K, M) if tA else (M, K))
    B = uniform(rng, (N, K) if tB else (K, N))
    C = cpu.matmul(cpu.tensor(A), cpu.tensor(B), tA, tB).numpy()
    Ae, Be = np64(A.T if tA else A), np64(B.T if tB else B)
    ref = Ae @ Be
    assert np.all(np.abs(C - ref) <= 2 * K * 2.0 ** -24 * (np.abs(Ae) @ np.abs(Be)) + 1e-30)


def test_matmul_shape_error(cpu):
    with pytest.raises(EngineError, match="dimension mismatch"):
        cpu.matmul(cpu.tensor(np.zeros((3, 4))), cpu.tensor(np.zeros((5, 6))))


def test_batched_matmul_alpha_and_errors(cpu):
    rng = np.random.default_rng(1)
    A, B = uniform(rng, (3 * 4, 5)), uniform(rng, (3 * 5, 6))
    C = cpu.batched_matmul(cpu.tensor(A), cpu.tensor(B), 3, False, False, 0.5).numpy()
    ref = np.concatenate([0.5 * (np64(A[4 * b:4 * b + 4]) @ np64(B[5 * b:5 * b + 5])) for b in range(3)])
    assert nrm_err(C, ref) <= 1e-6
    with pytest.raises(EngineError, match="divisible"):
        cpu.batched_matmul(cpu.tensor(A), cpu.tensor(B), 5)
    with pytest.raises(EngineError, match="batch must be > 0"):
        cpu.batched_matmul(cpu.tensor(A), cpu.tensor(B), 0)


# ── fused attention primitives vs dense float64 / torch autograd ───────────
def _dense_scores(A, B, batch, tA, tB, alpha, mask):
    """(batch, M, N) alpha*op(A_b)op(B_b) + mask, float64."""
    out = []
    ar, br = A.shape[0] // batch, B.shape[0] // batch
    for b in range(batch):
        Ab, Bb = np64(A[b * ar:(b + 1) * ar]), np64(B[b * br:(b + 1) * br])
        S = alpha * ((Ab.T if tA else Ab) @ (Bb.T if tB else Bb))
        out.append(S + (np64(mask) if mask is not None else 0.0))
    return np.stack(out)


@pytest.mark.parametrize("tA,tB", [(False, False), (False, True), (True, False), (True, True)])
@pytest.mark.parametrize("masked", [False, True])
def test_fused_forward_vs_dense(cpu, tA, tB, masked):
    rng = np.random.default_rng(2026)
    batch, M, N, K, D, alpha = 2, 4, 6, 4, 5, 0.35
    A = uniform(rng, (batch * (K if tA else M), M if tA else K))
    B = uniform(rng, (batch * (N if tB else K), K if tB else N))
    V = uniform(rng, (batch * N, D))
    mask = causal_mask(max(M, N))[:M, :N] if masked else None
    S = _dense_scores(A, B, batch, tA, tB, alpha, mask)
    a, b = cpu.tensor(A), cpu.tensor(B)
    mk = cpu.tensor(mask) if masked else None
    m = cpu.batched_matmul_reduce(a, b, batch, "Max", tA, tB, alpha, True, mk).numpy().reshape(batch, M)
    assert nrm_err(m, S.max(axis=2)) <= 1e-6
    fin = np.isfinite(S)
    ssum = cpu.batched_matmul_reduce(a, b, batch, "Sum", tA, tB, alpha, True, mk).numpy().reshape(batch, M)
    assert nrm_err(ssum, np.where(fin, S, 0).sum(axis=2)) <= 1e-6
    smin = cpu.batched_matmul_reduce(a, b, batch, "Min", tA, tB, alpha, True, mk).numpy().reshape(batch, M)
    assert nrm_err(smin, np.where(fin, S, np.inf).min(axis=2)) <= 1e-6
    mcol = cpu.batched_matmul_reduce(a, b, batch, "Max", tA, tB, alpha, False, mk).numpy()
    # a fully masked column keeps the initial lowest() (max(lowest, -inf) = lowest)
    ref_col = S.max(axis=1)
    empty = ~np.isfinite(ref_col)
    assert np.all(mcol[empty] == np.finfo(np.float32).min)
    assert nrm_err(np.where(empty, 0, mcol), np.where(empty, 0, ref_col)) <= 1e-6
    l = cpu.batched_matmul_softmax_denom(a, b, cpu.tensor(m.reshape(-1, 1)), batch, tA, tB, alpha, mk).numpy()
    W = np.exp(S - S.max(axis=2, keepdims=True))
    assert nrm_err(l.reshape(batch, M), W.sum(axis=2)) <= 1e-6
    O = cpu.batched_matmul_softmax_apply(a, b, cpu.tensor(V), cpu.tensor(m.reshape(-1, 1)), cpu.tensor(l), batch, tA,
                                         tB, alpha, mk).numpy()
    P = W / W.sum(axis=2, keepdims=True)
    ref = np.concatenate([P[bb] @ np64(V[bb * N:(bb + 1) * N]) for bb in range(batch)])
    assert nrm_err(O, ref) <= 1e-6
    # identity: softmax rows sum to one -> applying to a ones V gives ones
    O1 = cpu.batched_matmul_softmax_apply(a, b, cpu.tensor(np.ones((batch * N, 3))),
                                          cpu.tensor(m.reshape(-1, 1)), cpu.tensor(l), batch, tA, tB, alpha,
                                          mk).numpy()
    assert np.abs(O1 - 1).max() <= 1e-6


def test_fully_masked_row_max_is_lowest(cpu):
    """Max reduction starts at lowest(): an all -inf row stays lowest (cpu_engine.hpp:466-470)."""
    A = np.ones((2, 2), dtype=np.float32)
    mask = np.array([[-np.inf, -np.inf], [0, -np.inf]], dtype=np.float32)
    m = cpu.batched_matmul_reduce(cpu.tensor(A), cpu.tensor(A), 1, "Max", True, False, 1.0, True,
                                  cpu.tensor(mask)).numpy()
    assert m[0, 0] == np.finfo(np.float32).min and m[1, 0] == 2.0


@pytest.mark.parametrize("masked", [False, True])
def test_fused_backward_vs_autograd(cpu, masked):
    """backward_q / backward_kv equal torch autograd of L1 = sum P*W (dQ, dK) and
    L2 = sum G*(W V) (dV) in the attention layout transA=1, transB=0."""
    rng = np.random.default_rng(7)
    batch, T, d, alpha = 3, 9, 5, 0.4
    Q, K = uniform(rng, (batch * d, T)), uniform(rng, (batch * d, T))
    Pm, G = uniform(rng, (batch * T, T)), uniform(rng, (batch * T, d))
    mask = causal_mask(T) if masked else None
    q = torch.tensor(np64(Q), requires_grad=True)
    k = torch.tensor(np64(K), requires_grad=True)
    v = torch.zeros(batch * T, d, dtype=torch.float64, requires_grad=True)
    L1 = 0
    L2 = 0
    for b in range(batch):
        S = alpha * q[b * d:(b + 1) * d].T @ k[b * d:(b + 1) * d]
        if masked:
            S = S + torch.tensor(np64(mask))
        W = torch.softmax(S, dim=1)
        L1 = L1 + (torch.tensor(np64(Pm[b * T:(b + 1) * T])) * W).sum()
        L2 = L2 + (torch.tensor(np64(G[b * T:(b + 1) * T])) * (W.detach() @ v[b * T:(b + 1) * T])).sum()
    L1.backward()
    L2.backward()
    a, kk = cpu.tensor(Q), cpu.tensor(K)
    mk = cpu.tensor(mask) if masked else None
    m = cpu.batched_matmul_reduce(a, kk, batch, "Max", True, False, alpha, True, mk)
    l = cpu.batched_matmul_softmax_denom(a, kk, m, batch, True, False, alpha, mk)
    dq, r = cpu.batched_matmul_softmax_backward_q(a, kk, cpu.tensor(Pm), m, l, batch, True, False, alpha, mk)
    dk, dv = cpu.batched_matmul_softmax_backward_kv(a, kk, cpu.tensor(Pm), cpu.tensor(G), r, m, l, batch, True,
                                                    False, alpha, mk)
    assert nrm_err(dq.numpy(), q.grad.numpy()) <= 1e-5
    assert nrm_err(dk.numpy(), k.grad.numpy()) <= 1e-5
    # dV is returned transposed per batch: (batch*K, N) with element [k][j]
    dv_ref = np.concatenate([v.grad.numpy()[b * T:(b + 1) * T].T for b in range(batch)])
    assert nrm_err(dv.numpy(), dv_ref) <= 1e-5
    # R_i = sum_j W_ij P_ij
    S = _dense_scores(Q, K, batch, True, False, alpha, mask)
    W = np.exp(S - S.max(axis=2, keepdims=True))
    W /= W.sum(axis=2, keepdims=True)
    assert nrm_err(r.numpy().reshape(batch, T), (W * np64(Pm).reshape(batch, T, T)).sum(axis=2)) <= 1e-6


# ── column softmax / sparse cross-entropy ───────────────────────────────────
def test_sparse_ce_closed_form(cpu):
    rng = np.random.default_rng(3)
    C, N, vocab = 50, 40, 45
    L = normal(rng, (C, N), 2.0)
    labels = rng.integers(0, vocab, size=N).astype(np.float32)
    labels[[1, 5]] = [vocab, vocab + 100]   # invalid
    labels[7] = -1.0                        # reads as class 0
    mask = np.ones(N, dtype=np.float32)
    mask[[2, 3]] = [0.0, 0.49]
    inv = 1.0 / 33
    g, lv = cpu.col_softmax_sparse_forward(cpu.tensor(L), cpu.tensor(labels), cpu.tensor(mask), vocab, inv)
    g, lv = g.numpy(), lv.numpy()[0]
    Ld = np64(L)
    logp = Ld - Ld.max(0) - np.log(np.exp(Ld - Ld.max(0)).sum(0))
    lab = np.where(labels >= 0, labels, 0).astype(np.int64)
    valid = (mask >= 0.5) & (lab < vocab)
    for i in range(N):
        if not valid[i]:
            assert not g[:, i].any() and lv[i] == 0
            continue
        onehot = np.zeros(C)
        onehot[lab[i]] = 1
        assert np.abs(g[:, i] - inv * (np.exp(logp[:, i]) - onehot)).max() <= 1e-7
        assert abs(g[:, i].sum()) <= 1e-7
        assert abs(lv[i] - logp[lab[i], i]) <= 1e-5
    den = cpu.col_softmax_denom(cpu.tensor(L), cpu.tensor(L.max(0, keepdims=True))).numpy()[0]
    assert nrm_err(den, np.exp(Ld - Ld.max(0)).sum(0)) <= 1e-6
    with pytest.raises(EngineError, match="2\\^24"):
        cpu.col_softmax_sparse_forward(cpu.tensor(np.zeros((2, 2))), cpu.tensor(np.zeros((1, 2))), None,
                                       (1 << 24) + 1, 1.0)


# ── index / layout primitives: brute force, bit-exact ──────────────────────
def test_gather_scatter_brute_force(cpu):
    rng = np.random.default_rng(4)
    V, D, n = 30, 7, 200
    table = normal(rng, (V, D))
    idx = rng.integers(-2, V + 3, size=n).astype(np.float32)
    idx[:3] = [-0.5, 29.9, 1e30]
    out = cpu.gather_rows(cpu.tensor(table), cpu.tensor(idx)).numpy()
    grad = normal(rng, (n, D))
    dst = cpu.tensor(table)
    cpu.scatter_add_rows(dst, cpu.tensor(idx), cpu.tensor(grad))
    exp_g = np.zeros((n, D), dtype=np.float32)
    exp_s = table.copy()
    for i in range(n):
        f = float(idx[i])
        if f > -1 and f < 2 ** 64 and int(f) < V:
            r = int(f)
            exp_g[i] = table[r]
            for c in range(D):   # serial float32 accumulation in i order
                exp_s[r, c] = np.float32(exp_s[r, c] + grad[i, c])
    assert np.array_equal(out, exp_g)
    assert np.array_equal(dst.numpy(), exp_s)


def test_layout_primitives(cpu):
    rng = np.random.default_rng(5)
    M, B, N = 6, 4, 5
    X = uniform(rng, (M, B * N))
    Y = cpu.rearrange_3d(cpu.tensor(X), M, B, N).numpy()
    assert np.array_equal(Y, X.reshape(M, B, N).transpose(1, 0, 2).reshape(B * M, N))
    Z = cpu.rearrange_3d(cpu.tensor(Y), M, B, N, True).numpy()
    assert np.array_equal(Z, X)
    A = uniform(rng, (130, 70))
    assert np.array_equal(cpu.transpose(cpu.tensor(A)).numpy(), A.T)
    s = cpu.slice_rows(cpu.tensor(A), 3, 4).numpy()
    assert np.array_equal(s, A[3:7])
    with pytest.raises(EngineError, match="out of bounds"):
        cpu.slice_rows(cpu.tensor(A), 128, 4)


def test_elementwise_and_reductions(cpu):
    rng = np.random.default_rng(6)
    A, B = uniform(rng, (33, 44), 0.1, 3), uniform(rng, (33, 44), 0.1, 3)
    f = {"Neg": np.negative, "Exp": np.exp, "Log": np.log, "Sqrt": np.sqrt, "Rsqrt": lambda x: 1 / np.sqrt(x),
         "Abs": np.abs, "Tanh": np.tanh}
    for op, fn in f.items():
        assert nrm_err(cpu.elementwise_unary(op, cpu.tensor(A)).numpy(), fn(np64(A))) <= 2e-7
    g = {"Add": np.add, "Sub": np.subtract, "Mul": np.multiply, "Div": np.divide, "Max": np.maximum,
         "Min": np.minimum}
    for op, fn in g.items():
        assert np.array_equal(cpu.elementwise_binary(op, cpu.tensor(A), cpu.tensor(B)).numpy(), fn(A, B))
        assert np.array_equal(cpu.elementwise_binary_scalar(op, cpu.tensor(A), 1.5, True).numpy(),
                              fn(np.float32(1.5), A))
    assert nrm_err(cpu.row_reduce_sum(cpu.tensor(A)).numpy()[:, 0], np64(A).sum(1)) <= 1e-6
    assert nrm_err(cpu.col_reduce_sum(cpu.tensor(A)).numpy()[0], np64(A).sum(0)) <= 1e-6
    assert np.array_equal(cpu.col_reduce_max(cpu.tensor(A)).numpy()[0], A.max(0))
    big = uniform(rng, (2048, 300))   # parallel row-block path of col_reduce
    assert nrm_err(cpu.col_reduce_sum(cpu.tensor(big)).numpy()[0], np64(big).sum(0)) <= 1e-6


# ── eval_expr programs of the GPT path (the layers' ExprSpec programs) ───────────
def _softmax_fwd_spec():
    s = ExprSpec()
    for v in ("Linear", "RowReduceMax", "Linear", "RowReduceMax"):
        s.view(v)
    r0 = s.ins("Sub", inp(0), inp(1))
    r1 = s.ins("Exp", reg(r0))
    r2 = s.ins("Sub", inp(2), inp(3))
    r3 = s.ins("Exp", reg(r2))
    r4 = s.ins("RowSum", reg(r3))
    s.ins("Div", reg(r1), red(r4))
    return s


def _softmax_bwd_spec():
    s = ExprSpec()
    for _ in range(4):
        s.view("Linear")
    r0 = s.ins("Mul", inp(2), inp(3))
    r1 = s.ins("RowSum", reg(r0))
    r2 = s.ins("Sub", inp(1), red(r1))
    s.ins("Mul", inp(0), reg(r2))
    return s


def test_expr_softmax_programs(cpu):
    rng = np.random.default_rng(8)
    X, Gr = normal(rng, (17, 23), 3), normal(rng, (17, 23))
    y = cpu.eval_expr(_softmax_fwd_spec(), [cpu.tensor(X)] * 4, 17, 23).numpy()
    e = np.exp(np64(X) - np64(X).max(1, keepdims=True))
    ref = e / e.sum(1, keepdims=True)
    assert nrm_err(y, ref) <= 1e-6
    dx = cpu.eval_expr(_softmax_bwd_spec(), [cpu.tensor(y), cpu.tensor(Gr), cpu.tensor(y), cpu.tensor(Gr)],
                       17, 23).numpy()
    ref_dx = ref * (np64(Gr) - (ref * np64(Gr)).sum(1, keepdims=True))
    assert nrm_err(dx, ref_dx) <= 1e-5


def test_expr_rmsnorm_programs(cpu):
    rng = np.random.default_rng(9)
    F, N = 24, 10
    x, g, gamma = normal(rng, (F, N)), normal(rng, (F, N)), uniform(rng, (F, 1), 0.5, 1.5)
    # A.1: ColSum(x*x) as a reduced vector
    s = ExprSpec()
    s.view("Linear"), s.view("Linear")
    r0 = s.ins("Mul", inp(0), inp(1))
    s.ins("ColSum", reg(r0))
    ss = cpu.eval_expr_reduce(s, [cpu.tensor(x)] * 2, F, N).numpy()
    assert ss.shape == (1, N) and nrm_err(ss[0], (np64(x) ** 2).sum(0)) <= 1e-6
    rms_inv = (1 / np.sqrt(ss / F + 1e-5)).astype(np.float32)
    normed = x * rms_inv
    # A.3(c): RowSum(g*gamma*normed) -> (F,1)
    s = ExprSpec()
    s.view("Linear"), s.view("RowBroadcast"), s.view("Linear")
    r0 = s.ins("Mul", inp(0), inp(1))
    r1 = s.ins("Mul", reg(r0), inp(2))
    s.ins("RowSum", reg(r1))
    gg = cpu.eval_expr_reduce(s, [cpu.tensor(g), cpu.tensor(gamma), cpu.tensor(normed)], F, N).numpy()
    assert gg.shape == (F, 1) and nrm_err(gg[:, 0], (np64(g) * gamma * normed).sum(1)) <= 1e-6
    # A.3(b): (g*gamma - colbcast(m)*normed) * colbcast(rms_inv)
    m = ((g * gamma * normed).sum(0, keepdims=True) / F).astype(np.float32)
    s = ExprSpec()
    for v in ("Linear", "RowBroadcast", "ColBroadcast", "Linear", "ColBroadcast"):
        s.view(v)
    r0 = s.ins("Mul", inp(0), inp(1))
    r1 = s.ins("Mul", inp(2), inp(3))
    r2 = s.ins("Sub", reg(r0), reg(r1))
    s.ins("Mul", reg(r2), inp(4))
    dx = cpu.eval_expr(s, [cpu.tensor(a) for a in (g, gamma, m, normed, rms_inv)], F, N).numpy()
    assert nrm_err(dx, (np64(g) * gamma - m * normed) * rms_inv) <= 1e-6


def test_expr_views_and_select(cpu):
    rng = np.random.default_rng(10)
    R, C, blk = 8, 5, 4
    x = normal(rng, (R, C))
    tab = normal(rng, (blk, C))
    s = ExprSpec()
    s.view("RotateHalf", blk, 1), s.view("RowMod", blk), s.view("Linear")
    c0 = s.const(0.0)
    r0 = s.ins("Mul", inp(0), inp(1))
    r1 = s.ins("Gt", inp(2), cst(c0))
    s.ins("Select", reg(r1), reg(r0), inp(2))
    y = cpu.eval_expr(s, [cpu.tensor(x), cpu.tensor(tab), cpu.tensor(x)], R, C).numpy()
    rot = np.empty_like(x)
    for r in range(R):
        rl = r % blk
        src = (r // blk) * blk + (rl + blk // 2 if rl < blk // 2 else rl - blk // 2)
        rot[r] = -x[src] if rl < blk // 2 else x[src]
    ref = np.where(x > 0, rot * np.tile(tab, (R // blk, 1)), x)
    assert np.array_equal(y, ref)


def test_expr_validation_errors(cpu):
    t = cpu.tensor(np.ones((2, 2)))
    s = ExprSpec()
    s.view("Linear")
    r0 = s.ins("ColSum", inp(0))
    s.ins("Add", reg(r0), inp(0))          # register read of a reduce result
    with pytest.raises(EngineError, match="reduce dst"):
        cpu.eval_expr(s, [t], 2, 2)
    s = ExprSpec()
    s.view("Linear")
    s.ins("Exp", inp(0))
    s.ins("Add", red(0), inp(0))           # Reduce operand on an elementwise result
    with pytest.raises(EngineError, match="prior reduce"):
        cpu.eval_expr(s, [t], 2, 2)
    s = ExprSpec()
    s.view("Linear")
    r0 = s.ins("ColSum", inp(0))
    s.ins("Add", red(r0), inp(0))          # reads a Linear input after the reduction
    with pytest.raises(EngineError, match="not constant"):
        cpu.eval_expr_reduce(s, [t], 2, 2)
    s = ExprSpec()
    s.view("Linear")
    s.ins("Exp", inp(0))
    with pytest.raises(EngineError, match="rows or along columns"):
        cpu.eval_expr_reduce(s, [t], 2, 2)


# ── attention mask: the reference's known-answer rows ──────────────────────
def test_build_attention_mask_known_rows(cpu):
    """src/doc_mask_test.cpp:49-104."""
    ninf = -np.inf
    m = cpu.build_attention_mask(2, 4, 2, False)
    for row in range(16):
        i = row % 4
        assert np.array_equal(m[row], [0 if j <= i else ninf for j in range(4)])
    doc = [0, 0, 1, 1, 1, 2]
    m = cpu.build_attention_mask(1, 6, 1, False, doc_ids=doc)
    for i in range(6):
        assert np.array_equal(m[i], [0 if (j <= i and doc[i] == doc[j]) else ninf for j in range(6)])
    m = cpu.build_attention_mask(1, 3, 2, True, slopes=[1.0, 0.5])
    for h, sl in enumerate([1.0, 0.5]):
        for i in range(3):
            exp = [-sl * (i - j) if j <= i else ninf for j in range(3)]
            assert np.allclose(m[h * 3 + i], exp, atol=1e-6, rtol=0) and np.array_equal(np.isinf(m[h * 3 + i]),
                                                                                        np.isinf(exp))
    doc = [0, 0, 1, 1]
    m = cpu.build_attention_mask(1, 4, 1, True, slopes=[0.25], doc_ids=doc)
    for i in range(4):
        exp = [-0.25 * (i - j) if (j <= i and doc[i] == doc[j]) else ninf for j in range(4)]
        assert np.allclose(np.nan_to_num(m[i], neginf=-9), np.nan_to_num(np.array(exp), neginf=-9))


# ── whole GPT: oracle vs independent float64 torch restatement ─────────────
def _run_gpt(eng, cfg, params, toks, doc=None, mask=None):
    g = eng.gpt(**cfg)
    assert g.param_shapes() == torch_gpt.param_shapes(cfg)
    g.set_params(params)
    if doc is not None:
        g.set_doc_ids(doc)
    T = cfg["seq_len"]
    g.load_batch(toks[:T].astype(np.float32), toks[1:].T.reshape(-1), mask)
    loss = g.forward_loss()
    logits = g.logits()
    g.backward()
    grads = g.grads()
    g.optimizer_step()
    return loss, logits, grads, g.params()


@pytest.mark.parametrize("pos", ["learned", "alibi", "sinusoidal"])
@pytest.mark.parametrize("with_doc", [False, True])
def test_gpt_vs_torch_float64(cpu, pos, with_doc):
    cfg = dict(vocab_size=40, d_model=16, seq_len=8, num_heads=2, d_ff=24, num_layers=2, pos_enc=pos)
    rng = np.random.default_rng(123)
    B = 3
    params = [rng.normal(0, 0.2, s).astype(np.float32) for s in torch_gpt.param_shapes(cfg)]
    toks = rng.integers(0, 40, size=(9, B))
    doc = np.repeat(np.arange(6), 4).astype(np.uint64) if with_doc else None
    loss_mask = (rng.random(B * 8) > 0.2).astype(np.float32)
    loss, logits, grads, new_params = _run_gpt(cpu, cfg, params, toks, doc, loss_mask)
    rloss, rlogits, rgrads = torch_gpt.loss_and_grads(params, toks[:8], toks[1:].T.reshape(-1), cfg,
                                                      doc_ids=doc, loss_mask=loss_mask)
    assert abs(loss - rloss) <= 1e-5 * abs(rloss)
    assert nrm_err(logits, rlogits) <= 1e-5
    errs = grad_errs(grads, torch_gpt.reference_gamma_grads(params, rgrads, cfg))
    assert max(errs) <= 1e-4, errs
    # one AdamW step, closed form from the oracle's own gradients
    for a, b in zip(new_params, torch_gpt.adamw_step(params, [np64(g) for g in grads])):
        assert np.abs(a - b).max() <= 1e-6 * max(1.0, np.abs(b).max())


def test_gpt_gradcheck_finite_differences(cpu):
    """The reference's gpt_gradcheck method (src/gpt_gradcheck.cpp:124-261): central differences,
    eps 1e-3, |num - ana| <= 5e-2 (1 + |num| + |ana|)."""
    cfg = dict(vocab_size=32, d_model=16, seq_len=8, num_heads=2, d_ff=32, num_layers=2, pos_enc="alibi")
    rng = np.random.default_rng(7)
    params = [rng.normal(0, 0.3, s).astype(np.float32) for s in torch_gpt.param_shapes(cfg)]
    for i in torch_gpt.gamma_indices(cfg):   # gains at 1, as the reference's gradcheck model has them
        params[i] = np.ones_like(params[i])
    toks = rng.integers(0, 32, size=(9, 2))
    g = cpu.gpt(**cfg)
    g.set_params(params)
    g.load_batch(toks[:8].astype(np.float32), toks[1:].T.reshape(-1))
    g.forward_loss()
    g.backward()
    grads = g.grads()
    eps = 1e-3
    for pi in range(len(params)):
        flat = params[pi].reshape(-1)
        for e in rng.choice(flat.size, size=min(3, flat.size), replace=False):
            vals = []
            for sgn in (1, -1):
                p2 = [p.copy() for p in params]
                p2[pi].reshape(-1)[e] += sgn * eps
                g.set_params(p2)
                vals.append(g.forward_loss())
            num = (vals[0] - vals[1]) / (2 * eps)
            ana = float(grads[pi].reshape(-1)[e])
            assert abs(num - ana) <= 5e-2 * (1 + abs(num) + abs(ana)), (pi, e, num, ana)


def test_doc_invariance(cpu):
    """src/doc_attn_test.cpp:75-152: with document ids, logits of document B do not
    depend on document A's tokens; without them they do."""
    cfg = dict(vocab_size=64, d_model=16, seq_len=8, num_heads=2, d_ff=32, num_layers=2, pos_enc="learned")
    rng = np.random.default_rng(9)
    params = [rng.normal(0, 0.3, s).astype(np.float32) for s in torch_gpt.param_shapes(cfg)]
    toks = rng.integers(0, 64, size=(8, 1))
    toks2 = toks.copy()
    toks2[:4] = (toks2[:4] + 7) % 64        # change document A (positions 0..3)
    doc = np.array([1, 1, 1, 1, 2, 2, 2, 2], dtype=np.uint64)

    def logits(tk, with_doc):
        g = cpu.gpt(**cfg)
        g.set_params(params)
        if with_doc:
            g.set_doc_ids(doc)
        g.load_batch(tk.astype(np.float32), np.zeros(8, dtype=np.uint64))
        g.forward_loss()
        return g.logits()
    assert np.abs(logits(toks, True)[:, 4:] - logits(toks2, True)[:, 4:]).max() <= 1e-4
    assert np.abs(logits(toks, False)[:, 4:] - logits(toks2, False)[:, 4:]).max() > 1e-2


@pytest.mark.parametrize("name", sorted(__import__("layer_programs").PROGRAMS))
def test_layer_programs_closed_form(cpu, name):
    """Every ExprSpec program of the GPT layers, as the DSL folds it, against its closed form."""
    import layer_programs as lp
    from test_gpu_layer_programs import make_args
    build, vec, closed = lp.PROGRAMS[name]
    spec, slots = build()
    F, N = 24, 36
    args = make_args(np.random.default_rng(11), slots, F, N)
    ts = {k: cpu.tensor(v) for k, v in args.items()}
    ins = [ts[n] for n in slots]
    got = (cpu.eval_expr_reduce if vec else cpu.eval_expr)(spec, ins, F, N).numpy()
    assert nrm_err(got, closed({k: v.astype(np.float64) for k, v in args.items()})) <= 1e-6


# ── pins for the remaining primitives: select, column broadcast, row max ───
_CMP = {"Lt": np.less, "Le": np.less_equal, "Gt": np.greater, "Ge": np.greater_equal, "Eq": np.equal,
        "Ne": np.not_equal}


@pytest.mark.parametrize("cmp", sorted(_CMP))
def test_select_scalar_cond_closed_form(cpu, cmp):
    """elementwise_select_scalar_cond (reference cpu_engine.hpp:1221-1266): out = (A cmp b) ? T : e,
    with ties (entries equal to b), signed zeros, infinities and NaN (every comparison with NaN is
    false except Ne)."""
    rng = np.random.default_rng(21)
    b = np.float32(0.25)
    A = rng.choice(np.array([-1.5, -0.0, 0.0, 0.25, 0.2500001, 0.2499999, 3.0, np.inf, -np.inf, np.nan],
                            dtype=np.float32), size=(13, 17))
    A[0, :4] = b                                  # ties in every case
    T = normal(rng, (13, 17))
    e = np.float32(-7.5)
    got = cpu.elementwise_select_scalar_cond(cmp, cpu.tensor(A), float(b), cpu.tensor(T), float(e)).numpy()
    with np.errstate(invalid="ignore"):
        cond = _CMP[cmp](A, b)
    assert np.array_equal(got, np.where(cond, T, e))
    # b = 0 against signed zeros: -0.0 == 0.0
    got0 = cpu.elementwise_select_scalar_cond(cmp, cpu.tensor(A), 0.0, cpu.tensor(T), float(e)).numpy()
    with np.errstate(invalid="ignore"):
        assert np.array_equal(got0, np.where(_CMP[cmp](A, np.float32(0.0)), T, e))
    with pytest.raises(EngineError, match="shape"):
        cpu.elementwise_select_scalar_cond(cmp, cpu.tensor(A), 0.0, cpu.tensor(T[:, :3]), 0.0)


@pytest.mark.parametrize("op", ["Add", "Sub", "Mul", "Div", "Max", "Min"])
def test_broadcast_inplace_closed_form(cpu, op):
    """broadcast_col_inplace / broadcast_row_inplace (reference cpu_engine.hpp:1092-1125): A[r][c] op= v[c]
    (v is (1, cols)) and A[r][c] op= v[r] (v is (rows, 1)); one float32 operation per element, so the
    result equals numpy's float32 broadcast bit for bit."""
    fn = {"Add": np.add, "Sub": np.subtract, "Mul": np.multiply, "Div": np.divide, "Max": np.maximum,
          "Min": np.minimum}[op]
    rng = np.random.default_rng(22)
    A = uniform(rng, (9, 14), 0.1, 2.0)
    A[0, 0] = 1.0
    vc = uniform(rng, (1, 14), 0.5, 1.5)
    vc[0, 0] = 1.0                                # ties for Max / Min
    t = cpu.tensor(A)
    cpu.broadcast_col_inplace(t, cpu.tensor(vc), op)
    assert np.array_equal(t.numpy(), fn(A, vc))
    vr = uniform(rng, (9, 1), 0.5, 1.5)
    t = cpu.tensor(A)
    cpu.broadcast_row_inplace(t, cpu.tensor(vr), op)
    assert np.array_equal(t.numpy(), fn(A, vr))
    with pytest.raises(EngineError, match="shape mismatch"):
        cpu.broadcast_col_inplace(cpu.tensor(A), cpu.tensor(vr), op)
    with pytest.raises(EngineError, match="shape mismatch"):
        cpu.broadcast_row_inplace(cpu.tensor(A), cpu.tensor(vc), op)


def test_row_reduce_max_closed_form(cpu):
    """row_reduce_max (reference cpu_engine.hpp:1068-1076 over algebra_matrix.hpp:799-821): the
    maximum over {lowest()} and the row, so a row of -inf (or an empty row) yields lowest(), not -inf."""
    rng = np.random.default_rng(23)
    A = normal(rng, (11, 37), 3.0)
    A[2] = -np.inf
    A[3, :5] = -np.inf
    A[4] = np.finfo(np.float32).min
    A[5, 7] = np.inf
    got = cpu.row_reduce_max(cpu.tensor(A)).numpy()
    lowest = np.finfo(np.float32).min
    assert got.shape == (11, 1)
    assert np.array_equal(got[:, 0], np.max(A, axis=1, initial=lowest))
    assert got[2, 0] == lowest and got[5, 0] == np.inf
    assert np.array_equal(cpu.col_reduce_max(cpu.tensor(A.T.copy())).numpy()[0], got[:, 0])
    empty = cpu.row_reduce_max(cpu.tensor(np.zeros((3, 0), dtype=np.float32))).numpy()
    assert np.array_equal(empty[:, 0], np.full(3, lowest, dtype=np.float32))


@pytest.mark.parametrize("view", ["RowReduceSum", "RowReduceMax", "ColReduceSum", "ColReduceMax"])
def test_expr_reduce_views_closed_form(cpu, view):
    """The reduce views of eval_expr (reference cpu_engine.hpp:1368-1396): each row (Row*) or column
    (Col*) of the input is summed, or maxed from lowest(), and the scalar is read at every element of
    that row / column. Checked through out = view(x) - y * 2 against float64 sums and exact maxima."""
    rng = np.random.default_rng(24)
    R, C = 19, 29
    x = normal(rng, (R, C))
    x[1] = -np.inf                                # a row of -inf: max view yields lowest()
    x[:, 2] = -np.inf                             # a column of -inf
    if view.endswith("Sum"):
        x = np.where(np.isfinite(x), x, 0.5).astype(np.float32)
    y = normal(rng, (R, C))
    s = ExprSpec()
    s.view(view), s.view("Linear")
    c2 = s.const(2.0)
    r0 = s.ins("Mul", inp(1), cst(c2))
    s.ins("Sub", inp(0), reg(r0))
    got = cpu.eval_expr(s, [cpu.tensor(x), cpu.tensor(y)], R, C).numpy()
    axis = 1 if view.startswith("Row") else 0
    if view.endswith("Sum"):
        red_v = np64(x).sum(axis=axis, keepdims=True)
        assert nrm_err(got, red_v - 2 * np64(y)) <= 1e-6
    else:
        red_v = np.max(x, axis=axis, keepdims=True, initial=np.finfo(np.float32).min)
        assert np.array_equal(got, (red_v - np.float32(2) * y).astype(np.float32))
    # as the operand of a reduce instruction along the same axis (eval_expr_reduce requires one
    # axis for views and instructions): every element of a row / column holds the same scalar
    # (finite input here: C copies of lowest() would overflow the float32 sum)
    xf = np.where(np.isfinite(x), x, 0.5).astype(np.float32)
    s = ExprSpec()
    s.view(view)
    s.ins("RowSum" if axis == 1 else "ColSum", inp(0))
    vec = cpu.eval_expr_reduce(s, [cpu.tensor(xf)], R, C).numpy()
    if view.endswith("Sum"):
        ref = np.broadcast_to(np64(xf).sum(axis=axis, keepdims=True), (R, C)).sum(axis=axis)
    else:
        ref = np.broadcast_to(np64(xf).max(axis=axis, keepdims=True), (R, C)).sum(axis=axis)
    assert nrm_err(vec.reshape(-1), ref) <= 1e-6


def test_inplace_and_copy_primitives_closed_form(cpu):
    """add_inplace / scale_inplace / axpy_inplace / zero (reference cpu_engine.hpp:1008-1040), insert_rows
    and clone (:67-110): one float32 operation per element (bit-exact against numpy float32) and
    exact copies."""
    rng = np.random.default_rng(25)
    A, B = normal(rng, (7, 9)), normal(rng, (7, 9))
    t = cpu.tensor(A)
    cpu.add_inplace(t, cpu.tensor(B))
    assert np.array_equal(t.numpy(), A + B)
    cpu.scale_inplace(t, 0.3)
    assert np.array_equal(t.numpy(), (A + B) * np.float32(0.3))
    # a + s*b is contracted to one fused multiply-add (as clang, the reference's compiler, does by
    # default): the float64 value rounded once, within half an ulp of the float32 result
    x = (A + B) * np.float32(0.3)
    cpu.axpy_inplace(t, -1.25, cpu.tensor(B))
    ref = np64(x) + -1.25 * np64(B)
    got = t.numpy()
    assert np.all(np.abs(got - ref) <= 0.5 * np.spacing(np.abs(got)))
    c = cpu.clone(t)
    cpu.zero(t)
    assert not t.numpy().any() and np.array_equal(c.numpy(), got)
    dst = cpu.tensor(A)
    cpu.insert_rows(dst, 2, cpu.tensor(B[:3]))
    ref = A.copy()
    ref[2:5] = B[:3]
    assert np.array_equal(dst.numpy(), ref)
    with pytest.raises(EngineError):
        cpu.insert_rows(dst, 6, cpu.tensor(B[:3]))
    with pytest.raises(EngineError):
        cpu.add_inplace(cpu.tensor(A), cpu.tensor(B[:3]))


def test_build_attention_mask_rejects_missing_slopes(cpu):
    """ALiBi reads one slope per head: a slope list of another length is an error, not a read past it."""
    with pytest.raises(EngineError, match="slope"):
        cpu.build_attention_mask(1, 4, 2, True, slopes=[1.0])
    with pytest.raises(EngineError, match="slope"):
        cpu.build_attention_mask(1, 4, 2, True)
    # the C-ABI itself rejects a null slope pointer with ALiBi set
    out = np.empty((8, 4), np.float32)
    assert cpu._f["build_attention_mask"](1, 4, 2, 1, None, None, 0, out.ctypes.data_as(
        ctypes.POINTER(ctypes.c_float))) != 0


# ── GPT variants: QuickGeLU, LayerNorm, RoPE (reference compute_layer.hpp:256, 479, 884) ──
@pytest.mark.parametrize("variant", [dict(pos_enc="learned", activation="gelu", norm="layernorm"),
                                     dict(pos_enc="rope", activation="swiglu", norm="rmsnorm"),
                                     dict(pos_enc="rope", activation="gelu", norm="layernorm"),
                                     dict(pos_enc="alibi", activation="gelu", norm="rmsnorm")],
                         ids=lambda v: "-".join(v.values()))
@pytest.mark.parametrize("with_doc", [False, True])
def test_gpt_variants_vs_torch_float64(cpu, variant, with_doc):
    """The other GPT variants against the independent float64 model (LayerNorm with biased variance,
    QuickGeLU x*sigmoid(1.702x), RoPE as a complex rotation of dimension pairs (j, j + d_k/2))."""
    cfg = dict(vocab_size=40, d_model=16, seq_len=8, num_heads=2, d_ff=24, num_layers=2, **variant)
    rng = np.random.default_rng(321)
    B = 3
    shapes = torch_gpt.param_shapes(cfg)
    params = [rng.normal(0, 0.2, s).astype(np.float32) for s in shapes]
    toks = rng.integers(0, 40, size=(9, B))
    doc = np.repeat(np.arange(6), 4).astype(np.uint64) if with_doc else None
    g = cpu.gpt(**cfg)
    assert g.param_shapes() == shapes
    g.set_params(params)
    if doc is not None:
        g.set_doc_ids(doc)
    g.load_batch(toks[:8].astype(np.float32), toks[1:].T.reshape(-1))
    loss = g.forward_loss()
    logits = g.logits()
    g.backward()
    grads = g.grads()
    rloss, rlogits, rgrads = torch_gpt.loss_and_grads(params, toks[:8], toks[1:].T.reshape(-1), cfg, doc_ids=doc)
    assert abs(loss - rloss) <= 1e-5 * abs(rloss)
    assert nrm_err(logits, rlogits) <= 1e-5
    errs = grad_errs(grads, torch_gpt.reference_gamma_grads(params, rgrads, cfg))
    assert max(errs) <= 1e-4, errs


def test_rope_rotation_properties(cpu):
    """RoPE's scores depend on relative position only (q_i . k_j after rotation = f(i - j)), and the
    backward rotation is the forward's inverse."""
    import layer_programs as lp
    dk, T = 8, 6
    rng = np.random.default_rng(2)
    q = normal(rng, (dk, 1)).repeat(T, axis=1)      # the same vector at every position
    k = normal(rng, (dk, 1)).repeat(T, axis=1)
    c, s = lp.rope_tables(dk, T)
    fwd, bwd = lp.rope(dk, False)[0], lp.rope(dk, True)[0]
    ct, st = cpu.tensor(c), cpu.tensor(s)
    qr = cpu.eval_expr(fwd, [cpu.tensor(q), ct, cpu.tensor(q), st], dk, T)
    kr = cpu.eval_expr(fwd, [cpu.tensor(k), ct, cpu.tensor(k), st], dk, T)
    S = qr.numpy().T.astype(np.float64) @ kr.numpy().astype(np.float64)     # (T, T)
    for d in range(-T + 1, T):
        diag = np.diagonal(S, offset=d)
        assert np.abs(diag - diag[0]).max() <= 1e-5 * max(1.0, np.abs(S).max())
    back = cpu.eval_expr(bwd, [qr, ct, qr, st], dk, T).numpy()
    assert nrm_err(back, q) <= 1e-6


# ── incremental inference (reference compute_layer.hpp:1426-1511, 2413-2437, 2906-3096) ──
def _session_with(cpu_or_hip, cfg, params):
    g = cpu_or_hip.gpt(**cfg)
    g.set_params(params)
    return g


@pytest.mark.parametrize("pos", ["learned", "sinusoidal", "alibi", "rope"])
def test_forward_step_equals_full_forward(cpu, pos):
    """The reference's attn_consistency_test method (src/attn_consistency_test.cpp): logits of token t
    from forward_step with KV caches (positions 0..t) equal column t of the full forward over the
    sequence (causal, so later tokens do not matter)."""
    cfg = dict(vocab_size=48, d_model=16, seq_len=10, num_heads=2, d_ff=24, num_layers=2, pos_enc=pos)
    rng = np.random.default_rng(5)
    params = [rng.normal(0, 0.2, s).astype(np.float32) for s in torch_gpt.param_shapes(cfg)]
    toks = rng.integers(0, 48, size=10)
    g = _session_with(cpu, cfg, params)
    g.load_batch(toks.reshape(10, 1).astype(np.float32), np.zeros(10, np.uint64))
    g.forward_loss()
    full = g.logits()                               # (V, 10)
    for t in range(10):
        step = g.forward_step(int(toks[t]), t, t)
        assert nrm_err(step, full[:, t]) <= 1e-5, t
    g.reset_cache()
    assert nrm_err(g.forward_step(int(toks[0]), 0, 0), full[:, 0]) <= 1e-5


def test_generate_greedy_is_argmax_of_full_forward(cpu):
    """generate at temperature 0 appends argmax of the last logits; checked by recomputing each step's
    logits with a full forward of the context (no caches), including a sliding-window refill once the
    caches are full (context longer than seq_len), and an eos stop."""
    cfg = dict(vocab_size=32, d_model=16, seq_len=6, num_heads=2, d_ff=24, num_layers=2, pos_enc="alibi")
    rng = np.random.default_rng(8)
    params = [rng.normal(0, 0.5, s).astype(np.float32) for s in torch_gpt.param_shapes(cfg)]
    g = _session_with(cpu, cfg, params)
    prompt = [3, 17, 5]
    out = g.generate(prompt, 7, temperature=0.0)
    assert len(out) == 7
    ctx = list(prompt)
    for tok in out:
        window = ctx if len(ctx) < 6 else ctx[-5:]   # full caches are refilled with the last seq_len - 1 tokens
        T = len(window)
        c2 = dict(cfg, seq_len=T)
        full = _session_with(cpu, c2, params[:])
        full.load_batch(np.asarray(window, np.float32).reshape(T, 1), np.zeros(T, np.uint64))
        full.forward_loss()
        assert tok == int(np.argmax(full.logits()[:, -1])), (ctx, tok)
        ctx.append(tok)
    eos = out[2]
    stopped = g.generate(prompt, 7, temperature=0.0, eos=eos, min_new=0)
    assert stopped == out[:out.index(eos)]
    sampled = g.generate(prompt, 5, temperature=0.8, seed=11)
    assert sampled == g.generate(prompt, 5, temperature=0.8, seed=11) and all(0 <= t < 32 for t in sampled)


# ── optimizers by name (reference compute_optimizer.hpp:153-216, 415-615) ──
def _ns_closed_form(G, steps=5):
    """Newton-Schulz on G as its action on the singular values: the iteration X <- aX + (bA + cA^2)X with
    A = XX^T keeps G's singular vectors and maps each normalised singular value x to a x + b x^3 + c x^5."""
    a, b, c = 3.4445, -4.7750, 2.0315
    G = np64(G)
    U, sv, Vt = np.linalg.svd(G, full_matrices=False)
    x = sv / np.sqrt((G ** 2).sum() + 1e-14)
    for _ in range(steps):
        x = a * x + b * x ** 3 + c * x ** 5
    return (U * x) @ Vt


@pytest.mark.parametrize("name", ["sgd", "sgd_momentum", "adam", "muon"])
def test_optimizer_first_step_closed_form(cpu, name):
    """One step of each optimizer the session can use, from zero state, against its closed form: SGD
    p - lr g; momentum p - lr (1 - beta) g; Adam p - lr g / (|g| + eps); Muon (momentum 0.95, Nesterov)
    p - lr NS(1.95 g) for matrices (NS through the SVD, above) and p - lr 1.95 g for vectors."""
    cfg = dict(vocab_size=24, d_model=16, seq_len=6, num_heads=2, d_ff=12, num_layers=1, pos_enc="learned")
    rng = np.random.default_rng(13)
    params = [rng.normal(0, 0.2, s).astype(np.float32) for s in torch_gpt.param_shapes(cfg)]
    toks = rng.integers(0, 24, size=(7, 2))
    lr = 0.05
    g = cpu.gpt(**cfg, optimizer=name, lr=lr, weight_decay=0.0)
    g.set_params(params)
    g.load_batch(toks[:6].astype(np.float32), toks[1:].T.reshape(-1))
    g.forward_loss()
    g.backward()
    grads = [np64(x) for x in g.grads()]
    g.optimizer_step()
    new = g.params()
    for p, gr, q in zip(params, grads, new):
        if name == "sgd":
            ref = np64(p) - lr * gr
        elif name == "sgd_momentum":
            ref = np64(p) - lr * 0.1 * gr
        elif name == "adam":
            ref = np64(p) - lr * gr / (np.abs(gr) + 1e-8)
        else:
            upd = 1.95 * gr
            ref = np64(p) - lr * (_ns_closed_form(upd) if p.shape[0] > 1 and p.shape[1] > 1 else upd)
        tol = 2e-6 if name != "muon" else 2e-5
        assert np.abs(q - ref).max() <= tol * max(1.0, np.abs(ref).max()), (name, p.shape)
    with pytest.raises(KeyError):
        cpu.gpt(**cfg, optimizer="lion")
