"""Matrix-vector products of one vector in one launch (incremental inference's q, k, v projections).

AttentionBase::forward_step (reference compute_layer.hpp:1426-1511) runs w_q, w_k and w_v on the same
x_new: three Linear forwards, each matmul(W, x) then broadcast_row_inplace(bias). HipEngine records
them and launches the three products together (nnhip_gemv_group). The sums are those of the
single products, so the bar is bit-identity with the products launched one by one:

* the entry point against nnhip_gemm_epilogue per member (1 to 4 members, K 768 / 3072 / 5000 for the
  three unroll depths, K 99 for the scalar path, with and without biases), its second destinations (a
  copy, a residual sum x + v equal to the float32 add), and argument errors;
* the engine's Linear call pattern (three products of one x, each with its bias) against the same
  products forced out one at a time (a read after each), and a product of another x in between
  (not grouped), all against float64 within the GEMM tolerance as well;
* the engine's folds of forward_step (compute_layer.hpp:1426-1511, 2413-2437): the k and v rows
  inserted into caches through their transposes, and the residual add x + (W v + b), against the
  same calls with a read forcing each product out first; the cache rows around the insert keep
  their values, and a write to the cache between the calls runs the recorded insert first.
"""
import ctypes

import numpy as np
import pytest

import nnengine
from helpers import nrm_err, uniform

pytestmark = pytest.mark.gpu
SZ, P = ctypes.c_size_t, ctypes.c_void_p


def _lib():
    lib = nnengine.hip_library()
    lib.nnhip_gemv_group.argtypes = [P, P, P, P, P, P, SZ, SZ, SZ, P]
    lib.nnhip_gemm_epilogue.argtypes = [P, P, P, SZ, SZ, SZ, SZ, ctypes.c_int, ctypes.c_int, ctypes.c_float, P,
                                        ctypes.c_int, P, SZ, P]
    lib.nnhip_engine_stream.restype = ctypes.c_void_p
    lib.nnhip_engine_stream.argtypes = [ctypes.c_void_p]
    return lib


@pytest.mark.parametrize("count,rows,K,with_bias", [(3, 768, 768, True), (4, 37, 3072, False), (2, 130, 5000, True),
                                                    (1, 64, 99, True), (3, 200, 99, False)])
def test_entry_point_matches_single_products(hip, count, rows, K, with_bias):
    lib = _lib()
    rng = np.random.default_rng(rows + K + count)
    Ws = [uniform(rng, (rows, K)) for _ in range(count)]
    bs = [uniform(rng, (rows, 1)) for _ in range(count)]
    x = uniform(rng, (K, 1))
    tw, tb, tx = [hip.tensor(w) for w in Ws], [hip.tensor(b) for b in bs], hip.tensor(x)
    ys = [hip.create_tensor(rows, 1) for _ in range(count)]
    ref = [hip.create_tensor(rows, 1) for _ in range(count)]
    hip.sync()
    s = lib.nnhip_engine_stream(hip._e)
    adds = [uniform(rng, (rows, 1)) for _ in range(count)]
    ta = [hip.tensor(a) for a in adds]
    outs = [hip.create_tensor(rows, 1) for _ in range(count)]
    hip.sync()
    R = (P * 4)(*[t.data_ptr() for t in tw])
    B = (P * 4)(*[t.data_ptr() for t in tb])
    Y = (P * 4)(*[t.data_ptr() for t in ys])
    # second destinations: member 0 a copy, member 1 (if any) a residual sum, the rest none
    A = (P * 4)(None, ta[1].data_ptr() if count > 1 else None, None, None)
    O = (P * 4)(outs[0].data_ptr(), outs[1].data_ptr() if count > 1 else None, None, None)
    print(f"[gemv_group] count {count} rows {rows} K {K} bias {with_bias}", flush=True)
    assert lib.nnhip_gemv_group(R, tx.data_ptr(), B if with_bias else None, Y, A, O, count, rows, K, s) == 0
    for i in range(count):
        assert lib.nnhip_gemm_epilogue(tw[i].data_ptr(), tx.data_ptr(), ref[i].data_ptr(), rows, K, K, 1, 0, 0, 1.0,
                                       tb[i].data_ptr() if with_bias else None, 0, None, 0, s) == 0
    for i in range(count):
        got, want = ys[i].numpy(), ref[i].numpy()
        assert np.array_equal(got, want), i
        exact = Ws[i].astype(np.float64) @ x.astype(np.float64) + (bs[i] if with_bias else 0.0)
        assert nrm_err(got, exact) <= 1e-5
    assert np.array_equal(outs[0].numpy(), ref[0].numpy())
    if count > 1:
        assert np.array_equal(outs[1].numpy(), adds[1] + ref[1].numpy())   # float32 add, as the separate call
    assert lib.nnhip_gemv_group(R, tx.data_ptr(), None, Y, None, None, 5, rows, K, s) == -1   # more than 4
    assert lib.nnhip_gemv_group(R, None, None, Y, None, None, count, rows, K, s) == -1        # no vector
    assert lib.nnhip_gemv_group(R, tx.data_ptr(), None, None, A, None, count, rows, K, s) == -1   # add, no out


def test_engine_groups_linear_forwards(hip):
    """Three Linear forwards of one x (recorded, launched as one group) and the same with a read
    after each (launched alone): equal bit for bit; a product of another vector is not grouped."""
    rng = np.random.default_rng(3)
    d = 768
    Ws = [uniform(rng, (d, d)) for _ in range(3)]
    bs = [uniform(rng, (d, 1)) for _ in range(3)]
    x, x2 = uniform(rng, (d, 1)), uniform(rng, (d, 1))
    tw, tb, tx, tx2 = [hip.tensor(w) for w in Ws], [hip.tensor(b) for b in bs], hip.tensor(x), hip.tensor(x2)
    grouped = []
    for i in range(3):
        y = hip.matmul(tw[i], tx)
        hip.broadcast_row_inplace(y, tb[i], "Add")
        grouped.append(y)
        if i == 1:
            other = hip.matmul(tw[0], tx2)            # another vector in between
    got = [y.numpy() for y in grouped]
    alone = []
    for i in range(3):
        y = hip.matmul(tw[i], tx)
        hip.broadcast_row_inplace(y, tb[i], "Add")
        alone.append(y.numpy())
    for i in range(3):
        assert np.array_equal(got[i], alone[i]), i
        exact = Ws[i].astype(np.float64) @ x.astype(np.float64) + bs[i]
        assert nrm_err(got[i], exact) <= 1e-5
    assert nrm_err(other.numpy(), Ws[0].astype(np.float64) @ x2.astype(np.float64)) <= 1e-5


def _block_calls(hip, tw, tb, tx, kc, vc, pos, resid, force, write_between):
    """q, k, v = W_i x + b_i; insert k^T, v^T into the caches at row pos (then, if write_between, the k
    cache scaled by 2 in place); r = resid + (W_o q + b_o)."""
    ys = []
    for i in range(3):
        y = hip.matmul(tw[i], tx)
        hip.broadcast_row_inplace(y, tb[i], "Add")
        if force:
            y.numpy()
        ys.append(y)
    hip.insert_rows(kc, pos, hip.transpose(ys[1]))
    hip.insert_rows(vc, pos, hip.transpose(ys[2]))
    if write_between:
        hip.scale_inplace(kc, 2.0)                     # a recorded insert lands before the scaling
    o = hip.matmul(tw[3], ys[0])
    hip.broadcast_row_inplace(o, tb[3], "Add")
    if force:
        o.numpy()
    r = hip.elementwise_binary("Add", resid, o)
    return ys, o, r


@pytest.mark.parametrize("write_between", [False, True])
def test_engine_folds_cache_insert_and_residual(hip, write_between):
    rng = np.random.default_rng(7)
    d, seq, pos = 256, 12, 5
    Ws = [uniform(rng, (d, d)) for _ in range(4)]
    bs = [uniform(rng, (d, 1)) for _ in range(4)]
    x, resid = uniform(rng, (d, 1)), uniform(rng, (d, 1))
    cache0 = uniform(rng, (seq, d))
    res = {}
    for force in (False, True):
        tw, tb = [hip.tensor(w) for w in Ws], [hip.tensor(b) for b in bs]
        tx, tr = hip.tensor(x), hip.tensor(resid)
        kc, vc = hip.tensor(cache0), hip.tensor(cache0)
        ys, o, r = _block_calls(hip, tw, tb, tx, kc, vc, pos, tr, force, write_between)
        res[force] = dict(k=kc.numpy(), v=vc.numpy(), r=r.numpy(), o=o.numpy(), y=[y.numpy() for y in ys])
    g, s = res[False], res[True]
    kscale = 2.0 if write_between else 1.0
    assert np.array_equal(g["k"], s["k"])
    assert np.array_equal(g["v"], s["v"])
    assert np.array_equal(g["r"], s["r"]) and np.array_equal(g["o"], s["o"])
    for a, b in zip(g["y"], s["y"]):
        assert np.array_equal(a, b)
    rows = [i for i in range(seq) if i != pos]
    assert np.array_equal(s["v"][rows], cache0[rows])
    assert np.array_equal(s["k"][rows], kscale * cache0[rows])
    assert np.array_equal(s["k"][pos], kscale * s["y"][1][:, 0]) and np.array_equal(s["v"][pos], s["y"][2][:, 0])
    assert np.array_equal(s["r"], resid + s["o"])


class _Rms(ctypes.Structure):
    _fields_ = [("gamma", P), ("inv_f", ctypes.c_float), ("eps", ctypes.c_float), ("s_raw", P), ("scaled", P),
                ("var_eps", P), ("rinv", P), ("normed", P), ("out", P)]


@pytest.mark.parametrize("count,rows,K", [(3, 768, 768), (1, 6144, 768), (2, 50, 1000), (1, 33, 130)])
def test_rmsnorm_prologue_matches_separate_calls(hip, count, rows, K):
    """nnhip_gemv_group_rmsnorm against nnhip_rmsnorm_forward then nnhip_gemv_group: every RMSNorm
    output and every product equal bit for bit (the products read the normalised column)."""
    lib = _lib()
    lib.nnhip_gemv_group_rmsnorm.argtypes = [P, P, ctypes.POINTER(_Rms), P, P, P, P, SZ, SZ, SZ, P]
    lib.nnhip_rmsnorm_forward.argtypes = [P, P, ctypes.c_float, ctypes.c_float, P, P, P, P, P, P, SZ, SZ, P]
    rng = np.random.default_rng(count * rows + K)
    Ws = [uniform(rng, (rows, K)) for _ in range(count)]
    bs = [uniform(rng, (rows, 1)) for _ in range(count)]
    x, gamma = uniform(rng, (K, 1)) * 3, uniform(rng, (K, 1), 0.5, 1.5)
    tw, tb, tx, tg = [hip.tensor(w) for w in Ws], [hip.tensor(b) for b in bs], hip.tensor(x), hip.tensor(gamma)
    outs = {w: [hip.create_tensor(1, 1) for _ in range(4)] + [hip.create_tensor(K, 1) for _ in range(2)]
            for w in ("fused", "separate")}
    ys = {w: [hip.create_tensor(rows, 1) for _ in range(count)] for w in ("fused", "separate")}
    hip.sync()
    s = lib.nnhip_engine_stream(hip._e)
    R = (P * 4)(*[t.data_ptr() for t in tw])
    B = (P * 4)(*[t.data_ptr() for t in tb])
    inv_f, eps = 1.0 / K, 1e-6
    o = [t.data_ptr() for t in outs["fused"]]
    rn = _Rms(tg.data_ptr(), inv_f, eps, *o)
    print(f"[gemv_rms] count {count} rows {rows} K {K}", flush=True)
    assert lib.nnhip_gemv_group_rmsnorm(R, tx.data_ptr(), ctypes.byref(rn), B,
                                        (P * 4)(*[t.data_ptr() for t in ys["fused"]]), None, None, count, rows, K,
                                        s) == 0
    o2 = [t.data_ptr() for t in outs["separate"]]
    assert lib.nnhip_rmsnorm_forward(tx.data_ptr(), tg.data_ptr(), inv_f, eps, *o2, K, 1, s) == 0
    assert lib.nnhip_gemv_group(R, o2[5], B, (P * 4)(*[t.data_ptr() for t in ys["separate"]]), None, None, count,
                                rows, K, s) == 0
    for a, b in zip(outs["fused"], outs["separate"]):
        assert np.array_equal(a.numpy(), b.numpy())
    for a, b in zip(ys["fused"], ys["separate"]):
        assert np.array_equal(a.numpy(), b.numpy())
    xd = x.astype(np.float64)
    yref = xd / np.sqrt((xd ** 2).mean() + eps) * gamma
    assert nrm_err(outs["fused"][5].numpy(), yref) <= 1e-6
    assert lib.nnhip_gemv_group_rmsnorm(R, tx.data_ptr(), ctypes.byref(rn), B,
                                        (P * 4)(*[t.data_ptr() for t in ys["fused"]]), None, None, count, rows, 1025,
                                        s) == -1     # K above 1024
