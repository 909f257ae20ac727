"""The reference training loop (src/text_train.cpp:1181-1330) on the HIP
engine against the oracle: two micro-batches accumulated with the loss
gradient scaled by 1 / accum_steps, global-norm clipping active, then the
AdamW update and zero_grad, all through nnhip_gpt_train_step_ex."""
import numpy as np
import pytest

from helpers import grad_errs, nrm_err
from test_gpu_parity import check_adam_params

pytestmark = pytest.mark.gpu


def _loop(eng, cfg, params, batches, max_norm):
    g = eng.gpt(**cfg)
    g.set_params(params)
    losses = []
    g.load_batch(*batches[0])
    losses.append(g.train_step_ex(accum_steps=2, max_norm=max_norm, do_update=False))
    g.load_batch(*batches[1])
    losses.append(g.forward_loss())
    g.backward_scaled(0.5)
    grads = g.grads()
    g.clip_grad_norm(max_norm)
    clipped = g.grads()
    g.optimizer_step()
    g.zero_grad()
    return losses, grads, clipped, g.params()


@pytest.mark.parametrize("pos", ["learned", "alibi"])
def test_accumulate_clip_update(hip, cpu, pos):
    cfg = dict(vocab_size=256, d_model=64, seq_len=32, num_heads=4, d_ff=128, num_layers=2, pos_enc=pos)
    rng = np.random.default_rng(11)
    probe = cpu.gpt(**cfg)
    params = [rng.normal(0, 0.05, s).astype(np.float32) for s in probe.param_shapes()]
    probe.close()
    T, B = cfg["seq_len"], 3
    batches = []
    for _ in range(2):
        toks = rng.integers(0, cfg["vocab_size"], size=(T + 1, B))
        batches.append((toks[:T].astype(np.float32), toks[1:].T.reshape(-1)))
    c = _loop(cpu, cfg, params, batches, max_norm=0.02)
    norm = float(np.sqrt(sum(float(np.sum(np.asarray(x, np.float64) ** 2)) for x in c[1])))
    assert norm > 0.02, norm   # clipping is active
    h = _loop(hip, cfg, params, batches, max_norm=0.02)
    for lh, lc in zip(h[0], c[0]):
        assert abs(lh - lc) <= 1e-5 * abs(lc)
    assert max(grad_errs(h[1], c[1])) <= 1e-3
    assert max(grad_errs(h[2], c[2])) <= 1e-3
    for x, y in zip(h[2], c[2]):
        assert nrm_err(x, y) <= 1e-3 or np.abs(y).max() <= 1e-4 * max(np.abs(z).max() for z in c[2])
    check_adam_params(h[3], c[3], c[2], lr=1e-3)


@pytest.mark.parametrize("pos", ["learned", "alibi"])
def test_window_batch_through_session(hip, cpu, pos):
    """A batch cut from a token flow as the reference cuts it (src/text_train.cpp:1137-1178): windows at
    a stride, the last one running past the flow's end (padded tokens and labels), the loss mask dropping
    each window's last position and the padding, and per-position document ids that switch the session
    to the document-masked attention path. One full iteration (forward + CE, backward, AdamW) on the HIP
    session against the oracle."""
    cfg = dict(vocab_size=256, d_model=64, seq_len=32, num_heads=4, d_ff=128, num_layers=2, pos_enc=pos)
    rng = np.random.default_rng(17)
    T = cfg["seq_len"]
    n_flow = 3 * T + 9
    flow = rng.integers(1, cfg["vocab_size"], size=n_flow)
    lengths = [11, 5, 23, 9, 40, 7]
    docs = np.repeat(np.arange(1, len(lengths) + 1), lengths)
    docs = np.concatenate([docs, np.full(n_flow - docs.size, len(lengths) + 1)])[:n_flow]
    starts = [0, T, 2 * T, n_flow - 5]        # the last window holds 5 tokens, then padding
    tokens, labels, mask, doc_ids, valid = cpu.window_batch(flow, starts, T, pad_id=0, flow_doc=docs)
    assert valid == 3 * (T - 1) + 4 and mask[-T:].sum() == 4 and doc_ids[-1] == 0
    probe = cpu.gpt(**cfg)
    params = [rng.normal(0, 0.05, s).astype(np.float32) for s in probe.param_shapes()]
    probe.close()

    def run(e):
        g = e.gpt(**cfg)
        g.set_params(params)
        g.set_doc_ids(doc_ids)
        g.load_batch(tokens, labels, mask)
        loss = g.forward_loss()
        logits = g.logits()
        g.backward()
        grads = g.grads()
        g.optimizer_step()
        return loss, logits, grads, g.params()
    c = run(cpu)
    h = run(hip)
    assert abs(h[0] - c[0]) <= 1e-5 * abs(c[0])
    assert nrm_err(h[1], c[1]) <= 1e-4
    assert max(grad_errs(h[2], c[2])) <= 1e-3
    check_adam_params(h[3], c[3], c[2], lr=1e-3)
