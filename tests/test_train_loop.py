"""The reference training loop's step semantics (src/text_train.cpp:1181-1330)
on the oracle: gradient accumulation with the loss gradient scaled by
1 / accum_steps (:1242-1253), global-norm clipping before the update
(compute_optimizer.hpp:90-140) and the update / zero_grad cadence.

Pinned by properties the mathematics fixes, not by restating the code:
accumulated gradients are the mean of the micro-batch gradients (the
backward is linear in the loss gradient), clipping rescales the whole
gradient vector to norm max_norm and leaves it alone below that, and the
one-call loop iteration equals the same calls issued one by one.
"""
import numpy as np
import pytest

from helpers import grad_errs
import nnengine

CFG = dict(vocab_size=48, d_model=16, seq_len=8, num_heads=2, d_ff=24, num_layers=2, pos_enc="alibi")
B = 2


def _session(eng, params):
    g = eng.gpt(**CFG)
    g.set_params(params)
    return g


def _setup(eng, seed=7):
    rng = np.random.default_rng(seed)
    probe = eng.gpt(**CFG)
    params = [rng.normal(0, 0.2, s).astype(np.float32) for s in probe.param_shapes()]
    probe.close()
    T = CFG["seq_len"]
    batches = []
    for _ in range(2):
        toks = rng.integers(0, CFG["vocab_size"], size=(T + 1, B))
        batches.append((toks[:T].astype(np.float32), toks[1:].T.reshape(-1)))
    return params, batches


def _global_norm(grads):
    return float(np.sqrt(sum(float(np.sum(np.asarray(g, np.float64) ** 2)) for g in grads)))


def test_accumulated_grads_are_the_mean_of_micro_batch_grads(cpu):
    params, (a, b) = _setup(cpu)
    acc = _session(cpu, params)
    for tk, lb in (a, b):
        acc.load_batch(tk, lb)
        acc.forward_loss()
        acc.backward_scaled(0.5)
    g_acc = acc.grads()

    one = _session(cpu, params)
    per = []
    for tk, lb in (a, b):
        one.load_batch(tk, lb)
        one.forward_loss()
        one.backward()
        per.append(one.grads())
        one.zero_grad()
    mean = [0.5 * (np.asarray(x, np.float64) + np.asarray(y, np.float64)) for x, y in zip(*per)]
    errs = grad_errs(g_acc, mean)
    assert max(errs) <= 1e-5, errs
    # A plain backward would have summed them: the scale is not a no-op.
    assert _global_norm(g_acc) < 0.75 * _global_norm([2 * m for m in mean])


def test_clip_grad_norm_rescales_to_max_norm(cpu):
    params, ((tk, lb), _) = _setup(cpu)
    g = _session(cpu, params)
    g.load_batch(tk, lb)
    g.forward_loss()
    g.backward()
    before = g.grads()
    n = _global_norm(before)
    assert n > 0
    for no_op in (0.0, -1.0, 2.0 * n):
        g.clip_grad_norm(no_op)
        for x, y in zip(g.grads(), before):
            assert np.array_equal(x, y)
    g.clip_grad_norm(0.25 * n)
    after = g.grads()
    assert abs(_global_norm(after) - 0.25 * n) <= 1e-5 * n
    for x, y in zip(after, before):
        np.testing.assert_allclose(x, 0.25 * y, rtol=1e-5, atol=1e-7 * n)


def test_train_step_ex_equals_the_loop_issued_call_by_call(cpu):
    params, (a, b) = _setup(cpu)
    max_norm = 0.05
    one = _session(cpu, params)
    one.load_batch(*a)
    l1 = one.train_step_ex(accum_steps=2, max_norm=max_norm, do_update=False)
    assert any(np.abs(x).max() > 0 for x in one.grads())
    for x, y in zip(one.params(), params):   # no update yet
        assert np.array_equal(x, y)
    one.load_batch(*b)
    l2 = one.train_step_ex(accum_steps=2, max_norm=max_norm, do_update=True)

    ref = _session(cpu, params)
    losses = []
    for tk, lb in (a, b):
        ref.load_batch(tk, lb)
        losses.append(ref.forward_loss())
        ref.backward_scaled(0.5)
    assert _global_norm(ref.grads()) > max_norm   # clipping is active in this case
    ref.clip_grad_norm(max_norm)
    ref.optimizer_step()
    ref.zero_grad()

    assert (l1, l2) == tuple(losses)
    for x, y in zip(one.params(), ref.params()):
        assert np.array_equal(x, y)
    for x in one.grads():
        assert not np.any(x)
    assert any(not np.array_equal(x, y) for x, y in zip(one.params(), params))


def test_train_step_ex_rejects_zero_accum_steps(cpu):
    params, (a, _) = _setup(cpu)
    g = _session(cpu, params)
    g.load_batch(*a)
    with pytest.raises(nnengine.EngineError):
        g.train_step_ex(accum_steps=0)


def test_window_batch_hand_cases(cpu):
    """src/text_train.cpp:1137-1172 on a 7-token flow cut into windows of 4 at stride 3:
    full windows drop only their last label; the tail window holds one token."""
    flow = [10, 11, 12, 13, 14, 15, 16]
    docs = [1, 1, 1, 2, 2, 3, 3]
    pad = 0
    tokens, labels, mask, doc_ids, valid = cpu.window_batch(flow, [0, 3, 6], seq=4, pad_id=pad, flow_doc=docs)
    assert tokens.T.tolist() == [[10, 11, 12, 13], [13, 14, 15, 16], [16, pad, pad, pad]]
    assert labels.reshape(3, 4).tolist() == [[11, 12, 13, pad], [14, 15, 16, pad], [pad, pad, pad, pad]]
    assert mask.reshape(3, 4).tolist() == [[1, 1, 1, 0], [1, 1, 1, 0], [0, 0, 0, 0]]
    assert doc_ids.reshape(3, 4).tolist() == [[1, 1, 1, 2], [2, 2, 3, 3], [3, 0, 0, 0]]
    assert valid == 6
    t2, l2, m2, d2, v2 = cpu.window_batch(flow, [0, 3, 6], seq=4, pad_id=pad)
    assert d2 is None and v2 == valid and np.array_equal(t2, tokens) and np.array_equal(l2, labels)
    with pytest.raises(nnengine.EngineError):
        cpu.window_batch(flow, [7], seq=4, pad_id=pad)


def test_window_batch_feeds_a_session(cpu):
    """A flow of documents (one id per document, as the reference's line-per-document
    tokenisation gives them) through window_batch into the session: every full window
    contributes seq - 1 positions, and the doc-masked forward and backward run on it."""
    rng = np.random.default_rng(3)
    T = CFG["seq_len"]
    n_flow = 3 * T + 3
    flow = rng.integers(1, CFG["vocab_size"], size=n_flow)
    lengths = [5, 9, 4, 7]
    docs = np.repeat(np.arange(1, len(lengths) + 1), lengths)
    docs = np.concatenate([docs, np.full(n_flow - docs.size, len(lengths) + 1)])[:n_flow]
    starts = list(range(0, n_flow, T))[:B]
    tokens, labels, mask, doc_ids, valid = cpu.window_batch(flow, starts, T, pad_id=0, flow_doc=docs)
    assert valid == int(mask.sum()) and valid == B * (T - 1)
    params, _ = _setup(cpu)
    g = _session(cpu, params)
    g.set_doc_ids(doc_ids)
    g.load_batch(tokens, labels, mask)
    loss = g.forward_loss()
    g.backward()
    assert np.isfinite(loss) and loss > 0
