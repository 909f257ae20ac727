"""Independent float64 restatement of the reference GPT (test-only).

Written from the reference's layer descriptions, not from this repository's
C++ layers, so that it pins the composition of conventions the C++ stack
implements: batch-major token columns, head split, ALiBi slopes 2^(-8h/H)
starting at h = 0 (compute_layer.hpp:2179-2187), the (features, tokens)
activation layout, RMSNorm eps 1e-5 (:687), SwiGLU gate/up split (:373-400),
sparse cross-entropy averaged over valid tokens (compute_loss.hpp:284-308) and
the parameters() order (:2739-2755). torch autograd supplies the gradients.
"""
import math

import numpy as np
import torch


def _norm(cfg):
    return cfg.get("norm", "rmsnorm")


def _act(cfg):
    return cfg.get("activation", "swiglu")


def _layout(cfg):
    """(shape, role) per parameter in parameters() order; roles: 'gain' (RMSNorm / LayerNorm gamma),
    'shift' (LayerNorm beta), 'other'."""
    V, D, T, H, F, L = (cfg[k] for k in ("vocab_size", "d_model", "seq_len", "num_heads", "d_ff", "num_layers"))
    norm = [((D, 1), "gain")] + ([((D, 1), "shift")] if _norm(cfg) == "layernorm" else [])
    f1 = 2 * F if _act(cfg) == "swiglu" else F
    out = [((V, D), "other")]
    if cfg["pos_enc"] == "learned":
        out.append(((T, D), "other"))
    for _ in range(L):
        out += [((D, D), "other"), ((D, 1), "other")] * 4 + norm
        out += [((f1, D), "other"), ((f1, 1), "other"), ((D, F), "other"), ((D, 1), "other")] + norm
    out += norm + [((V, D), "other"), ((V, 1), "other")]
    return out


def param_shapes(cfg):
    return [s for s, _ in _layout(cfg)]


def gamma_indices(cfg):
    """Positions of the norm gains (RMSNorm / LayerNorm gamma) in parameters() order."""
    return [i for i, (_, r) in enumerate(_layout(cfg)) if r == "gain"]


def reference_gamma_grads(params_np, grads, cfg):
    """The reference accumulates grad_gamma += row_reduce_sum(g * gamma * normed)
    (RMSNorm compute_layer.hpp:788-795, LayerNorm :636-644), i.e. gamma times the
    true gradient sum(g * normed); the two agree at gamma = 1. Returns grads with
    that convention applied."""
    out = list(grads)
    for i in gamma_indices(cfg):
        out[i] = np.asarray(params_np[i], dtype=np.float64) * grads[i]
    return out


def _rmsnorm(x, g):
    rms_inv = 1.0 / torch.sqrt((x * x).mean(dim=0, keepdim=True) + 1e-5)
    return x * rms_inv * g


def _layernorm(x, g, b):
    """LayerNorm over features (compute_layer.hpp:479-662): biased variance, eps 1e-5."""
    mu = x.mean(dim=0, keepdim=True)
    var = ((x - mu) ** 2).mean(dim=0, keepdim=True)
    return (x - mu) / torch.sqrt(var + 1e-5) * g + b


def _rope(x, T, dk):
    """Rotary positions as complex rotation: per head block of dk rows, the pair (j, j + dk/2) is the
    complex number x_j + i x_{j+dk/2} turned by pos * 10000^(-2j/dk) (compute_layer.hpp:884-984)."""
    half = dk // 2
    j = torch.arange(half, dtype=torch.float64)
    theta = 10000.0 ** (-2.0 * j / dk)
    ang = torch.arange(T, dtype=torch.float64)[None, :] * theta[:, None]        # (half, T)
    rot = torch.polar(torch.ones_like(ang), ang)
    blocks = x.reshape(-1, dk, T)
    z = torch.complex(blocks[:, :half], blocks[:, half:]) * rot
    return torch.cat([z.real, z.imag], dim=1).reshape(x.shape)


def _sinusoidal(T, D):
    pe = np.zeros((T, D))
    for pos in range(T):
        for i in range(D):
            angle = pos / (10000.0 ** ((2 * (i // 2)) / D))
            pe[pos, i] = math.sin(angle) if i % 2 == 0 else math.cos(angle)
    return torch.tensor(pe, dtype=torch.float64)


def _mask(T, h, H, alibi, doc):
    i = torch.arange(T)[:, None]
    j = torch.arange(T)[None, :]
    allowed = j <= i
    if doc is not None:
        allowed = allowed & (doc[:, None] == doc[None, :])
    bias = torch.zeros(T, T, dtype=torch.float64)
    if alibi:
        slope = 2.0 ** (-8.0 * h / H)
        bias = -slope * (i - j).to(torch.float64)
    return torch.where(allowed, bias, torch.tensor(-math.inf, dtype=torch.float64))


def forward(params, tokens, cfg, doc_ids=None):
    """params: list of float64 torch tensors in parameters() order; tokens (T, B) ints.
    Returns logits (V, B*T) with column b*T + t."""
    V, D, T, H, F, L = (cfg[k] for k in ("vocab_size", "d_model", "seq_len", "num_heads", "d_ff", "num_layers"))
    pos = cfg["pos_enc"]
    B = tokens.shape[1]
    dk = D // H
    flat = torch.as_tensor(np.ascontiguousarray(tokens.T).reshape(-1), dtype=torch.long)   # b*T + t
    it = iter(params)
    emb = next(it)
    x = emb[flat]                                   # (N, D)
    tpos = torch.arange(B * T) % T
    if pos == "learned":
        x = x + next(it)[tpos]
    elif pos == "sinusoidal":
        x = x + _sinusoidal(T, D)[tpos]
    x = x.T                                         # (D, N)
    docs = None if doc_ids is None else torch.as_tensor(np.asarray(doc_ids, dtype=np.int64)).reshape(B, T)
    def norm(x):
        if _norm(cfg) == "layernorm":
            g, b = next(it), next(it)
            return _layernorm(x, g, b)
        return _rmsnorm(x, next(it))

    for _ in range(L):
        Wq, bq, Wk, bk, Wv, bv, Wo, bo = (next(it) for _ in range(8))
        h = norm(x)
        q, k, v = Wq @ h + bq, Wk @ h + bk, Wv @ h + bv
        out = torch.zeros_like(q)
        for b in range(B):
            cols = slice(b * T, (b + 1) * T)
            for hh in range(H):
                rows = slice(hh * dk, (hh + 1) * dk)
                Q, K_, Vv = q[rows, cols], k[rows, cols], v[rows, cols]          # (dk, T)
                if pos == "rope":
                    Q, K_ = _rope(Q, T, dk), _rope(K_, T, dk)
                S = (Q.T @ K_) / math.sqrt(dk) + _mask(T, hh, H, pos == "alibi",
                                                       None if docs is None else docs[b])
                A = torch.softmax(S, dim=1)
                out[rows, cols] = Vv @ A.T
        x = x + (Wo @ out + bo)
        W1, b1, W2, b2 = (next(it) for _ in range(4))
        h2 = norm(x)
        u = W1 @ h2 + b1
        if _act(cfg) == "swiglu":
            gate, up = u[:F], u[F:]
            act = gate * torch.sigmoid(gate) * up
        else:
            act = u * torch.sigmoid(1.702 * u)   # QuickGeLU (compute_layer.hpp:256-336)
        x = x + (W2 @ act + b2)
    xf = norm(x)
    Wl, bl = next(it), next(it)
    return Wl @ xf + bl


def loss_and_grads(params_np, tokens, labels, cfg, doc_ids=None, loss_mask=None):
    """Mean cross-entropy over valid tokens; returns (loss, logits, grads) as float64 numpy."""
    params = [torch.tensor(p, dtype=torch.float64, requires_grad=True) for p in params_np]
    logits = forward(params, tokens, cfg, doc_ids)
    lab = torch.as_tensor(np.asarray(labels, dtype=np.int64))
    logp = torch.log_softmax(logits, dim=0)
    valid = lab < cfg["vocab_size"]
    if loss_mask is not None:
        valid = valid & torch.as_tensor(np.asarray(loss_mask) >= 0.5)
    picked = logp[lab.clamp(max=cfg["vocab_size"] - 1), torch.arange(lab.numel())]
    loss = -(picked * valid).sum() / max(int(valid.sum()), 1)
    loss.backward()
    return float(loss.detach()), logits.detach().numpy(), [p.grad.numpy() for p in params]


def adamw_step(params, grads, lr=1e-3, b1=0.9, b2=0.999, eps=1e-8, wd=0.01, t=1):
    """Closed-form first AdamW step from zero moments (compute_optimizer.hpp:252-304, 388-412)."""
    out = []
    for p, g in zip(params, grads):
        p = p.astype(np.float64) * (1 - lr * wd)
        m = (1 - b1) * g
        v = (1 - b2) * g * g
        mh = m / (1 - b1 ** t)
        vh = v / (1 - b2 ** t)
        out.append(p - lr * mh / (np.sqrt(vh) + eps))
    return out
