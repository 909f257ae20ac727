"""A token's fc1 product and SwiGLU::forward in one launch (nnhip_gemv_swiglu).

FeedForward::forward in incremental inference (reference compute_layer.hpp:1623-1689 with SwiGLU,
:360-458) runs fc1 (2 d_ff rows) on the normalised token and then SwiGLU's chain on the gate and up
halves of the result: slice_rows x2, Neg, Exp, Add 1, Div (1 / .), Mul, Mul. HipEngine keeps the
fc1 product recorded while the chain is recorded and runs both (and the RMSNorm before them when that
is recorded) in one launch. The bar is bit-identity with the separate launches:

* the entry point against nnhip_gemv_group[_rmsnorm] of the 2 half rows followed by
  nnhip_swiglu_forward (with and without RMSNorm, bias, s and the product written; K 768 / 3072 /
  5000 for the three unroll depths, K 99 for the scalar path), and argument errors;
* the engine's call pattern (matmul, bias, the chain on two slices of the result, the slices and s
  kept as SwiGLU keeps them) against the same calls with a read of the product before the chain
  (which launches it alone), and both against float64.
"""
import ctypes

import numpy as np
import pytest

import nnengine
from helpers import nrm_err, uniform

pytestmark = pytest.mark.gpu
SZ, P, F = ctypes.c_size_t, ctypes.c_void_p, ctypes.c_float


class _Rms(ctypes.Structure):
    _fields_ = [("gamma", P), ("inv_f", F), ("eps", F), ("s_raw", P), ("scaled", P),
                ("var_eps", P), ("rinv", P), ("normed", P), ("out", P)]


def _lib():
    lib = nnengine.hip_library()
    lib.nnhip_gemv_swiglu.argtypes = [P, P, ctypes.POINTER(_Rms), P, P, P, P, SZ, SZ, F, F, P]
    lib.nnhip_gemv_group.argtypes = [P, P, P, P, P, P, SZ, SZ, SZ, P]
    lib.nnhip_gemv_group_rmsnorm.argtypes = [P, P, ctypes.POINTER(_Rms), P, P, P, P, SZ, SZ, SZ, P]
    lib.nnhip_swiglu_forward.argtypes = [P, P, P, P, SZ, F, F, P]
    lib.nnhip_engine_stream.restype = ctypes.c_void_p
    lib.nnhip_engine_stream.argtypes = [ctypes.c_void_p]
    return lib


def _ref64(W, x, b, gamma=None, eps=1e-5):
    xd = x.astype(np.float64)
    if gamma is not None:
        xd = xd / np.sqrt((xd ** 2).mean() + eps) * gamma
    v = W.astype(np.float64) @ xd + (b if b is not None else 0.0)
    h = v.shape[0] // 2
    g, u = v[:h], v[h:]
    s = 1.0 / (np.exp(-g) + 1.0)
    return v, s, g * s * u


@pytest.mark.parametrize("half,K,rms,with_bias,keep", [(3072, 768, True, True, True), (3072, 768, True, False, False),
                                                       (3072, 768, False, True, True), (100, 3072, False, True, True),
                                                       (64, 5000, False, False, True), (37, 99, False, True, False)])
def test_entry_point_matches_separate_launches(hip, half, K, rms, with_bias, keep):
    lib = _lib()
    rng = np.random.default_rng(half + K + int(rms))
    W = uniform(rng, (2 * half, K), -0.05, 0.05)
    b = uniform(rng, (2 * half, 1))
    x, gamma = uniform(rng, (K, 1)) * 3, uniform(rng, (K, 1), 0.5, 1.5)
    tw, tb, tx, tg = hip.tensor(W), hip.tensor(b), hip.tensor(x), hip.tensor(gamma)
    t = {w: dict(y=hip.create_tensor(2 * half, 1), s=hip.create_tensor(half, 1), o=hip.create_tensor(half, 1),
                 r=[hip.create_tensor(1, 1) for _ in range(4)] + [hip.create_tensor(K, 1) for _ in range(2)])
         for w in ("fused", "separate")}
    hip.sync()
    st = lib.nnhip_engine_stream(hip._e)
    bias = tb.data_ptr() if with_bias else None
    inv_f, eps = 1.0 / K, 1e-5
    rn = {w: _Rms(tg.data_ptr(), inv_f, eps, *[r.data_ptr() for r in t[w]["r"]]) for w in t}
    f = t["fused"]
    print(f"[gemv_swiglu] half {half} K {K} rms {rms} bias {with_bias} keep {keep}", flush=True)
    assert lib.nnhip_gemv_swiglu(tw.data_ptr(), tx.data_ptr(), ctypes.byref(rn["fused"]) if rms else None, bias,
                                 f["y"].data_ptr() if keep else None, f["s"].data_ptr() if keep else None,
                                 f["o"].data_ptr(), half, K, 1.0, 1.0, st) == 0
    sp = t["separate"]
    R, B, Y = (P * 4)(tw.data_ptr()), (P * 4)(bias), (P * 4)(sp["y"].data_ptr())
    if rms:
        assert lib.nnhip_gemv_group_rmsnorm(R, tx.data_ptr(), ctypes.byref(rn["separate"]), B, Y, None, None, 1,
                                            2 * half, K, st) == 0
    else:
        assert lib.nnhip_gemv_group(R, tx.data_ptr(), B, Y, None, None, 1, 2 * half, K, st) == 0
    y0 = sp["y"].data_ptr()
    assert lib.nnhip_swiglu_forward(y0, y0 + 4 * half, sp["s"].data_ptr(), sp["o"].data_ptr(), half, 1.0, 1.0,
                                    st) == 0
    assert np.array_equal(f["o"].numpy(), sp["o"].numpy())
    if keep:
        assert np.array_equal(f["y"].numpy(), sp["y"].numpy())
        assert np.array_equal(f["s"].numpy(), sp["s"].numpy())
    if rms:
        for a, c in zip(f["r"], sp["r"]):
            assert np.array_equal(a.numpy(), c.numpy())
    v, s, o = _ref64(W, x, b if with_bias else None, gamma if rms else None, eps)
    assert nrm_err(f["o"].numpy(), o) <= 1e-5
    if keep:
        assert nrm_err(f["y"].numpy(), v) <= 1e-5 and nrm_err(f["s"].numpy(), s) <= 1e-6
    # errors: no vector, no output, RMSNorm over K > 1024
    assert lib.nnhip_gemv_swiglu(tw.data_ptr(), None, None, None, None, None, f["o"].data_ptr(), half, K, 1.0, 1.0,
                                 st) == -1
    assert lib.nnhip_gemv_swiglu(tw.data_ptr(), tx.data_ptr(), None, None, None, None, None, half, K, 1.0, 1.0,
                                 st) == -1
    assert lib.nnhip_gemv_swiglu(tw.data_ptr(), tx.data_ptr(), ctypes.byref(rn["fused"]), None, None, None,
                                 f["o"].data_ptr(), half, 1025, 1.0, 1.0, st) == -1


def _ffn_in(hip, tw, tb, tx, d_ff, force):
    """fc1 forward (matmul + bias) and SwiGLU::forward's calls, as compute_layer.hpp issues them."""
    h = hip.matmul(tw, tx)
    hip.broadcast_row_inplace(h, tb, "Add")
    if force:
        h.numpy()                                          # the product runs alone, before the chain
    gate = hip.slice_rows(h, 0, d_ff)
    up = hip.slice_rows(h, d_ff, d_ff)
    t1 = hip.elementwise_unary("Neg", gate)
    t2 = hip.elementwise_unary("Exp", t1)
    t3 = hip.elementwise_binary_scalar("Add", t2, 1.0)
    s = hip.elementwise_binary_scalar("Div", t3, 1.0, True)
    sw = hip.elementwise_binary("Mul", gate, s)
    out = hip.elementwise_binary("Mul", sw, up)
    return h, gate, up, s, out


@pytest.mark.parametrize("d_ff,K", [(3072, 768), (64, 96)])
def test_engine_chain_matches_unfolded(hip, d_ff, K):
    rng = np.random.default_rng(d_ff + K)
    W = uniform(rng, (2 * d_ff, K), -0.05, 0.05)
    b = uniform(rng, (2 * d_ff, 1))
    x = uniform(rng, (K, 1)) * 2
    tw, tb, tx = hip.tensor(W), hip.tensor(b), hip.tensor(x)
    got = [t.numpy() for t in _ffn_in(hip, tw, tb, tx, d_ff, False)]
    want = [t.numpy() for t in _ffn_in(hip, tw, tb, tx, d_ff, True)]
    for name, a, c in zip(("h", "gate", "up", "s", "out"), got, want):
        assert np.array_equal(a, c), name
    v, s, o = _ref64(W, x, b)
    assert nrm_err(got[0], v) <= 1e-5 and nrm_err(got[3], s) <= 1e-6 and nrm_err(got[4], o) <= 1e-5


@pytest.mark.parametrize("case", ["read_up_first", "write_source", "write_slice", "chain_then_write"])
def test_slices_of_a_recorded_product(hip, case):
    """slice_rows leaves a token's matrix-vector product recorded; the slices still behave as copies
    through every engine call: a read through the second half, an in-place write of the source after
    slicing (the slices keep the product's values), an in-place write of a slice (the source keeps
    them), and a write of the source after the SwiGLU chain was recorded on its halves. Each against
    the same calls with the product read (launched) before slicing, bit for bit."""
    rng = np.random.default_rng(7)
    d_ff, K = 96, 64
    W, b, x = uniform(rng, (2 * d_ff, K), -0.1, 0.1), uniform(rng, (2 * d_ff, 1)), uniform(rng, (K, 1))
    tw, tb, tx = hip.tensor(W), hip.tensor(b), hip.tensor(x)

    def go(force):
        h = hip.matmul(tw, tx)
        hip.broadcast_row_inplace(h, tb, "Add")
        if force:
            h.numpy()
        gate, up = hip.slice_rows(h, 0, d_ff), hip.slice_rows(h, d_ff, d_ff)
        out = {}
        if case == "read_up_first":
            out["up"] = up.numpy()
            out["gate"] = gate.numpy()
        elif case == "write_source":
            hip.scale_inplace(h, 2.0)
            out["gate"], out["up"], out["h"] = gate.numpy(), up.numpy(), h.numpy()
        elif case == "write_slice":
            hip.scale_inplace(up, 3.0)
            out["h"], out["up"], out["gate"] = h.numpy(), up.numpy(), gate.numpy()
        else:
            t1 = hip.elementwise_unary("Neg", gate)
            t2 = hip.elementwise_unary("Exp", t1)
            t3 = hip.elementwise_binary_scalar("Add", t2, 1.0)
            s = hip.elementwise_binary_scalar("Div", t3, 1.0, True)
            o = hip.elementwise_binary("Mul", hip.elementwise_binary("Mul", gate, s), up)
            hip.scale_inplace(h, 2.0)
            out["o"], out["s"], out["h"], out["gate"], out["up"] = o.numpy(), s.numpy(), h.numpy(), gate.numpy(), \
                up.numpy()
        return out

    got, want = go(False), go(True)
    for k in want:
        assert np.array_equal(got[k], want[k]), k
    v = W.astype(np.float64) @ x.astype(np.float64) + b
    assert nrm_err(got["gate"], v[:d_ff]) <= 1e-5
