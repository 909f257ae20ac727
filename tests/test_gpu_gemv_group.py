"""Matrix-vector products of one vector in one launch (incremental inference's q, k, v projections).

AttentionBase::forward_step (reference compute_layer.hpp:1426-1511) runs w_q, w_k and w_v on the same
x_new: three Linear forwards, each matmul(W, x) then broadcast_row_inplace(bias). HipEngine records
them and launches the three products together (nnhip_gemv_group). The sums are those of the
single products, so the bar is bit-identity with the products launched one by one:

* the entry point against nnhip_gemm_epilogue per member (1 to 4 members, K 768 / 3072 / 5000 for the
  three unroll depths, K 99 for the scalar path, with and without biases), and argument errors;
* the engine's Linear call pattern (three products of one x, each with its bias) against the same
  products forced out one at a time (a read after each), and a product of another x in between
  (not grouped), all against float64 within the GEMM tolerance as well.
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
    lib.nnhip_gemv_group.argtypes = [P, P, P, P, SZ, SZ, SZ, P]
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
    R = (P * 4)(*[t.data_ptr() for t in tw])
    B = (P * 4)(*[t.data_ptr() for t in tb])
    Y = (P * 4)(*[t.data_ptr() for t in ys])
    print(f"[gemv_group] count {count} rows {rows} K {K} bias {with_bias}", flush=True)
    assert lib.nnhip_gemv_group(R, tx.data_ptr(), B if with_bias else None, Y, count, rows, K, s) == 0
    for i in range(count):
        assert lib.nnhip_gemm_epilogue(tw[i].data_ptr(), tx.data_ptr(), ref[i].data_ptr(), rows, K, K, 1, 0, 0, 1.0,
                                       tb[i].data_ptr() if with_bias else None, 0, None, 0, s) == 0
    for i in range(count):
        got, want = ys[i].numpy(), ref[i].numpy()
        assert np.array_equal(got, want), i
        exact = Ws[i].astype(np.float64) @ x.astype(np.float64) + (bs[i] if with_bias else 0.0)
        assert nrm_err(got, exact) <= 1e-5
    assert lib.nnhip_gemv_group(R, tx.data_ptr(), None, Y, 5, rows, K, s) == -1      # more than 4 members
    assert lib.nnhip_gemv_group(R, None, None, Y, count, rows, K, s) == -1           # no vector


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
