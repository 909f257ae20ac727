"""Attention of one query per head (incremental inference, reference compute_layer.hpp:1426-1511).

AttentionBase::forward_step scores the new token's query against the KV cache rows, adds the ALiBi
row, takes the softmax and weights the value rows. HipEngine runs that chain as one launch of
nnhip_attn_query, which reads the cache rows in place (include/nnhip_kernels.h). Checked here:

* the entry point against float64 numpy (m, l, O and the probabilities P): cache-row layout and transposed per-head layout, one chunk
  (N <= 256) and several merged chunks (N 600, 1500), no mask, one mask row shared by every head,
  a head whose keys are all masked (m = lowest(), l = 0, O = 0, as the one-pass forward leaves
  such rows), head dims that are not multiples of 4 (scalar path), and argument errors;
* forward_step through the engine at a context long enough for several chunks (ALiBi, 2 layers,
  seq_len 600) against the full forward of the same tokens;
Bars: m, l, O 1e-5 normwise (float32 sums over at most 1500 terms, float64 reference).
"""
import ctypes

import numpy as np
import pytest

import nnengine
import torch_gpt
from helpers import normal, nrm_err

pytestmark = pytest.mark.gpu
SZ, L = ctypes.c_size_t, ctypes.c_long
LOWEST = np.float32(-3.40282347e38)


def _lib():
    lib = nnengine.hip_library()
    lib.nnhip_attn_query_workspace_bytes.restype = SZ
    lib.nnhip_attn_query_workspace_bytes.argtypes = [SZ, SZ, SZ]
    P = ctypes.c_void_p
    lib.nnhip_attn_query.argtypes = [P, P, L, L, L, P, L, L, L, P, L, P, P, P, P, SZ, SZ, SZ, SZ, ctypes.c_float, P,
                                     P]
    lib.nnhip_engine_stream.restype = ctypes.c_void_p
    lib.nnhip_engine_stream.argtypes = [ctypes.c_void_p]
    return lib


def _reference(q, keys, vals, mask, alpha):
    """q (H, K), keys (H, N, K), vals (H, N, D), mask (H, N) or None: m, l, O, P in float64."""
    s = alpha * np.einsum("hk,hnk->hn", q.astype(np.float64), keys.astype(np.float64))
    if mask is not None:
        s = s + mask.astype(np.float64)
    m = s.max(axis=1)
    m = np.where(np.isfinite(m), m, LOWEST)
    w = np.exp(s - np.where(m == LOWEST, 0.0, m)[:, None])
    l = w.sum(axis=1)
    P = w / np.where(l > 0, l, 1.0)[:, None]
    O = np.einsum("hn,hnd->hd", P, vals.astype(np.float64))
    return m, l, O, P


CASES = [  # H, N, K, D, layout, mask kind
    (12, 72, 64, 64, "rows", "heads"),
    (12, 600, 64, 64, "rows", "heads"),
    (4, 1500, 64, 64, "rows", "shared"),
    (4, 1, 64, 64, "rows", "none"),
    (6, 300, 64, 64, "heads", "heads"),
    (3, 333, 20, 36, "rows", "heads"),
    (3, 257, 18, 30, "heads", "none"),
    (5, 260, 64, 64, "rows", "dead_head"),
]


@pytest.mark.parametrize("H,N,K,D,layout,mk", CASES)
def test_entry_point(hip, H, N, K, D, layout, mk):
    lib = _lib()
    rng = np.random.default_rng(H * N + K)
    q = normal(rng, (H, K))
    keys, vals = normal(rng, (H, N, K)), normal(rng, (H, N, D))
    alpha = 1.0 / np.sqrt(K)
    mask = None
    if mk in ("heads", "dead_head"):
        mask = (-np.abs(normal(rng, (H, N))) * 2).astype(np.float32)
        if mk == "dead_head":
            mask[2, :] = -np.inf
            mask[3, ::3] = -np.inf
    elif mk == "shared":
        mask = np.broadcast_to(-np.abs(normal(rng, (1, N))), (H, N)).astype(np.float32)
    if layout == "rows":          # KV cache rows (N, H*d): key j of head h at j*H*K + h*K
        ksrc = np.ascontiguousarray(keys.transpose(1, 0, 2).reshape(N, H * K))
        vsrc = np.ascontiguousarray(vals.transpose(1, 0, 2).reshape(N, H * D))
        kb, kj, kk, vb, vj, vd = K, H * K, 1, D, H * D, 1
    else:                         # per head (d, N): the transposed cache
        ksrc = np.ascontiguousarray(keys.transpose(0, 2, 1).reshape(H * K, N))
        vsrc = np.ascontiguousarray(vals.transpose(0, 2, 1).reshape(H * D, N))
        kb, kj, kk, vb, vj, vd = K * N, 1, N, D * N, 1, N
    tq, tk, tv = hip.tensor(q.reshape(H * K, 1)), hip.tensor(ksrc), hip.tensor(vsrc)
    tm = hip.tensor(mask[:1] if mk == "shared" else mask) if mask is not None else None
    mask_bs = 0 if mk == "shared" else N
    tmo, tlo, to, tp = hip.create_tensor(H, 1), hip.create_tensor(H, 1), hip.create_tensor(H * D, 1), None
    if mk != "none":
        tp = hip.create_tensor(H, N)
    wsb = lib.nnhip_attn_query_workspace_bytes(H, N, D)
    assert (wsb > 0) == (N > 256)
    ws = hip.create_tensor(max(1, wsb // 4), 1)
    hip.sync()
    print(f"[attn_query] H {H} N {N} K {K} D {D} {layout} {mk} ws {wsb}", flush=True)
    rc = lib.nnhip_attn_query(tq.data_ptr(), tk.data_ptr(), kb, kj, kk, tv.data_ptr(), vb, vj, vd,
                              tm.data_ptr() if tm is not None else None, mask_bs, tmo.data_ptr(), tlo.data_ptr(),
                              to.data_ptr(), tp.data_ptr() if tp is not None else None, H, N, K, D, alpha,
                              ws.data_ptr() if wsb else None,
                              lib.nnhip_engine_stream(hip._e))
    assert rc == 0
    m, l, O, Pr = _reference(q, keys, vals, mask, alpha)
    gm, gl, gO = tmo.numpy()[:, 0], tlo.numpy()[:, 0], to.numpy().reshape(H, D)
    alive = m != LOWEST
    assert nrm_err(gm[alive], m[alive]) <= 1e-5 and nrm_err(gl, l) <= 1e-5 and nrm_err(gO, O) <= 1e-5
    if tp is not None:
        assert nrm_err(tp.numpy(), Pr) <= 1e-5
    if mk == "dead_head":
        assert gm[2] == LOWEST and gl[2] == 0.0 and np.all(gO[2] == 0.0)


def test_argument_errors(hip):
    lib = _lib()
    t = hip.create_tensor(64, 64)
    p = t.data_ptr()
    call = lambda N, K, D, ws=None: lib.nnhip_attn_query(p, p, K, 64, 1, p, D, 64, 1, None, 0, p, p, p, None, 1, N,
                                                          K, D, 1.0, ws, None)
    assert call(0, 64, 64) == -1      # no keys
    assert call(8, 65, 64) == -1      # head dim above 64
    assert call(8, 64, 65) == -1      # value dim above 64
    assert call(300, 64, 64) == -1    # several chunks need the workspace


def test_forward_step_long_context(hip):
    """forward_step at every position of a 600-token context (keys split over 3 chunks at the end)
    against the full forward's logits (ALiBi, the bench model's layout at a small width)."""
    cfg = dict(vocab_size=96, d_model=64, seq_len=600, num_heads=4, d_ff=96, num_layers=2, pos_enc="alibi")
    rng = np.random.default_rng(11)
    params = [rng.normal(0, 0.1, s).astype(np.float32) for s in torch_gpt.param_shapes(cfg)]
    toks = rng.integers(0, 96, size=600)
    g = hip.gpt(**cfg)
    g.set_params(params)
    g.load_batch(toks.reshape(600, 1).astype(np.float32), np.zeros(600, np.uint64))
    g.forward_loss()
    full = g.logits()
    print("[attn_query] forward_step over 600 positions", flush=True)
    steps = np.stack([g.forward_step(int(toks[t]), t, t) for t in range(600)], axis=1)
    assert nrm_err(steps, full) <= 1e-4
    for t in (0, 255, 256, 257, 511, 599):
        assert nrm_err(steps[:, t], full[:, t]) <= 1e-4, t
