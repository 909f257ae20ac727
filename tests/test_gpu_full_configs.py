"""BASELINE configs 3 and 4 at their full sizes, and the config-4 cross-entropy shape.

* Config 4: the full training-step model (12 layers, d768, 12 heads, SwiGLU
  3072, RMSNorm, ALiBi, vocab 32000, context 1024) at batch 1 of 8, the same
  seeded weights and tokens on the HIP engine and on the CPU oracle: loss,
  logits, every parameter gradient and the AdamW-updated weights (reference
  text_train.cpp:1181-1330 step; tolerances as in the small GPT tests); and at
  the full batch of 8, whose loss and gradients are the means of the 8
  batch-1 rows' (rows are independent).
* Config 3: the six GEMM sweep shapes NN, plus the GPT projection shapes in the
  reference's Linear orientation (W (out, in) times X (in, tokens)) and its two
  backward variants (TN for dX, NT for dW), against float64 with the a-priori
  elementwise bound |dC| <= 2K 2^-24 (|A||B|)_ij.
* Sparse cross-entropy over the (32000, 8192) logits of config 4, against the
  closed form: grad = inv (softmax - onehot), loss_i = log softmax[label_i],
  sum over classes of every valid column's gradient = 0.
"""
import numpy as np
import pytest

from helpers import grad_errs, nrm_err, uniform
from test_gpu_parity import check_adam_params

pytestmark = pytest.mark.gpu

C4 = dict(vocab_size=32000, d_model=768, seq_len=1024, num_heads=12, d_ff=3072, num_layers=12, pos_enc="alibi")


def _c4_params(shapes, cfg, rng):
    """The reference's init scheme for the GPT model: 2-D weights and the token embedding N(0, 0.02),
    biases 0, RMSNorm gains 1 (gain tensors: two per block and the final one, in parameters() order)."""
    base = 2 if cfg["pos_enc"] == "learned" else 1
    gains = {base + 14 * layer + 8 for layer in range(cfg["num_layers"])}
    gains |= {base + 14 * layer + 13 for layer in range(cfg["num_layers"])}
    gains.add(base + 14 * cfg["num_layers"])
    out = []
    for i, (r, c) in enumerate(shapes):
        if i in gains:
            out.append(np.ones((r, c), np.float32))
        elif c == 1:
            out.append(np.zeros((r, c), np.float32))
        else:
            out.append(rng.standard_normal((r, c), dtype=np.float32) * np.float32(0.02))
    return out


def _c4_step(e, params, toks):
    g = e.gpt(**C4)
    g.set_params(params)
    T = C4["seq_len"]
    g.load_batch(toks[:T].astype(np.float32), toks[1:].T.reshape(-1))
    loss = g.forward_loss()
    logits = g.logits()
    g.backward()
    grads = g.grads()
    g.optimizer_step()
    new = g.params()
    g.close()
    return loss, logits, grads, new


def test_config4_full_model_batch1(hip, cpu):
    print("[c4] 12L d768 H12 ff3072 ALiBi V32000 T1024 B1, seed 4", flush=True)
    rng = np.random.default_rng(4)
    g = hip.gpt(**C4)
    shapes = g.param_shapes()
    g.close()
    params = _c4_params(shapes, C4, rng)
    toks = rng.integers(0, C4["vocab_size"], size=(C4["seq_len"] + 1, 1))
    h = _c4_step(hip, params, toks)
    print(f"[c4] hip loss {h[0]:.6f}", flush=True)
    c = _c4_step(cpu, params, toks)
    print(f"[c4] oracle loss {c[0]:.6f}", flush=True)
    assert abs(h[0] - c[0]) <= 1e-5 * abs(c[0]), (h[0], c[0])
    assert nrm_err(h[1], c[1]) <= 1e-4
    errs = grad_errs(h[2], c[2])
    assert max(errs) <= 1e-3, max(errs)
    flips = check_adam_params(h[3], c[3], c[2], lr=1e-3, got_grads=h[2], params0=params)
    print(f"[c4] grad max err {max(errs):.2e}, AdamW sign flips {flips} of {sum(p.size for p in params)}",
          flush=True)


def test_config4_full_batch8_is_mean_of_rows(hip):
    """Config 4 at its full batch of 8 (the step bench.py times: K = 8192 split-K weight gradients
    with accumulate epilogues, B = 8 head layouts, per-sequence ALiBi masks). Rows are independent
    (causal attention within a sequence; every other layer acts per token) and the loss is the mean
    over all B*T tokens, so the batch-8 loss is the mean of the 8 batch-1 losses and every batch-8
    gradient the mean of the per-row gradients; each batch-1 row is the path checked against the
    oracle above. Loss relative 1e-5, gradients normwise 1e-3 per tensor."""
    print("[c4b8] 12L d768 H12 ff3072 ALiBi V32000 T1024 B8 vs 8 x B1, seed 48", flush=True)
    rng = np.random.default_rng(48)
    T, B = C4["seq_len"], 8
    g8 = hip.gpt(**C4)
    params = _c4_params(g8.param_shapes(), C4, rng)
    toks = rng.integers(0, C4["vocab_size"], size=(T + 1, B))
    g8.set_params(params)
    g8.load_batch(toks[:T].astype(np.float32), toks[1:].T.reshape(-1))
    loss8 = g8.forward_loss()
    g8.backward()
    grads8 = g8.grads()
    g8.close()
    g1 = hip.gpt(**C4)
    g1.set_params(params)
    losses, mean_grads = [], None
    for b in range(B):
        g1.zero_grad()
        g1.load_batch(toks[:T, b:b + 1].astype(np.float32), toks[1:, b])
        losses.append(g1.forward_loss())
        g1.backward()
        gr = g1.grads()
        mean_grads = [x.astype(np.float64) / B for x in gr] if mean_grads is None else \
            [m + x.astype(np.float64) / B for m, x in zip(mean_grads, gr)]
    g1.close()
    ref = float(np.mean(np.float64(losses)))
    print(f"[c4b8] batch-8 loss {loss8:.6f}, mean of rows {ref:.6f}", flush=True)
    assert abs(loss8 - ref) <= 1e-5 * abs(ref), (loss8, ref)
    errs = grad_errs(grads8, mean_grads)
    print(f"[c4b8] gradient max err {max(errs):.2e}", flush=True)
    assert max(errs) <= 1e-3, max(errs)


def _check_gemm(hip, A, B, tA, tB):
    h = hip.matmul(hip.tensor(A), hip.tensor(B), tA, tB).numpy()
    Ae = (A.T if tA else A).astype(np.float64)
    Be = (B.T if tB else B).astype(np.float64)
    ref = Ae @ Be
    assert nrm_err(h, ref) <= 1e-5
    bound = 2 * Ae.shape[1] * 2.0 ** -24 * (np.abs(Ae) @ np.abs(Be))
    assert np.all(np.abs(h - ref) <= bound + 1e-30)


@pytest.mark.parametrize("M,N,K", [(1024, 1024, 1024), (2048, 2048, 2048), (4096, 4096, 4096),
                                   (8192, 2304, 768), (8192, 3072, 768), (8192, 768, 3072)])
def test_config3_sweep_shape(hip, M, N, K):
    print(f"[c3] NN {M}x{N}x{K}", flush=True)
    rng = np.random.default_rng(M + 3 * N + 7 * K)
    _check_gemm(hip, uniform(rng, (M, K)), uniform(rng, (K, N)), False, False)


@pytest.mark.parametrize("out_f,in_f", [(2304, 768), (3072, 768), (768, 3072)])
@pytest.mark.parametrize("variant", ["fwd", "dx", "dw"])
def test_config3_linear_orientation(hip, out_f, in_f, variant):
    """Linear forward W (out, in) . X (in, N), dX = W^T G (TN), dW = G X^T (NT, K = 8192 tokens)."""
    n = 8192
    print(f"[c3] linear {variant} out {out_f} in {in_f} N {n}", flush=True)
    rng = np.random.default_rng(out_f + in_f + len(variant))
    if variant == "fwd":
        _check_gemm(hip, uniform(rng, (out_f, in_f)), uniform(rng, (in_f, n)), False, False)
    elif variant == "dx":
        _check_gemm(hip, uniform(rng, (out_f, in_f)), uniform(rng, (out_f, n)), True, False)
    else:
        _check_gemm(hip, uniform(rng, (out_f, n)), uniform(rng, (in_f, n)), False, True)


def _check_ce_closed_form(g, lv, L, labels, valid, inv):
    """Gradient and loss of every column against the float64 closed form: grad = inv (softmax -
    onehot), loss = log softmax[label], columns without a valid label zero, each column's gradient
    summing to 0."""
    assert not g[:, ~valid].any() and not lv[~valid].any()
    cols = np.flatnonzero(valid)
    lab = labels.astype(np.int64)
    for c0 in range(0, cols.size, 1024):     # column blocks: bounded memory
        cs = cols[c0:c0 + 1024]
        Ld = L[:, cs].astype(np.float64)
        mx = Ld.max(axis=0)
        lse = mx + np.log(np.exp(Ld - mx).sum(axis=0))
        p = np.exp(Ld - lse)
        p[lab[cs], np.arange(cs.size)] -= 1.0
        ref = inv * p
        gb = g[:, cs].astype(np.float64)
        assert np.abs(gb - ref).max() <= 1e-5 * np.abs(ref).max()
        assert np.abs(gb.sum(axis=0)).max() <= 1e-5 * inv
        lref = Ld[lab[cs], np.arange(cs.size)] - lse
        assert np.abs(lv[cs] - lref).max() <= 1e-5 * np.abs(lref).max()


def test_sparse_ce_ragged(hip):
    """A ragged column count (2500: the float4 kernels' last column block partly filled), with a loss
    mask and out-of-range labels, against the float64 closed form."""
    C, N = 32000, 2500
    rng = np.random.default_rng(12)
    L = rng.standard_normal((C, N), dtype=np.float32) * np.float32(3.0)
    labels = rng.integers(0, C, size=N).astype(np.float32)
    labels[7::401] = C + 1
    mask = (rng.random(N) > 0.1).astype(np.float32)
    valid = (mask >= 0.5) & (labels < C)
    inv = 1.0 / float(valid.sum())
    g, lv = hip.col_softmax_sparse_forward(hip.tensor(L), hip.tensor(labels), hip.tensor(mask), C, inv)
    _check_ce_closed_form(g.numpy(), lv.numpy()[0], L, labels, valid, inv)


def test_sparse_ce_config4_shape(hip):
    """col_softmax_sparse_forward over (32000, 8192) logits (config 4's lm_head output), with invalid
    labels and a loss mask, against the float64 closed form."""
    C, N = 32000, 8192
    print(f"[ce] {C}x{N}", flush=True)
    rng = np.random.default_rng(11)
    L = rng.standard_normal((C, N), dtype=np.float32) * np.float32(2.0)
    labels = rng.integers(0, C, size=N).astype(np.float32)
    labels[::97] = C + 3                       # invalid: column left zero
    mask = (rng.random(N) > 0.05).astype(np.float32)
    valid = (mask >= 0.5) & (labels < C)
    inv = 1.0 / float(valid.sum())
    g, lv = hip.col_softmax_sparse_forward(hip.tensor(L), hip.tensor(labels), hip.tensor(mask), C, inv)
    _check_ce_closed_form(g.numpy(), lv.numpy()[0], L, labels, valid, inv)
