"""nnhip_tensor_device_ptr: a raw reader's pointer holds the tensor's values.

The materialised attention path keeps the forward's score blocks in the
probability tensor A (the layer's softmax result) until A is read through the
engine; an FFI host that takes A's device pointer and reads it itself
(nnhip_tensor_data_ptr gives the pointer as it is) would see those blocks.
nnhip_tensor_device_ptr queues what a read through the engine would first, so
the memory behind the pointer holds the probabilities once the engine's
stream gets there; the backward that follows still matches the oracle.
Bars as test_gpu_attn_chain.py (A 1e-5, O 1e-4, gradients 1e-3).
"""
import ctypes

import numpy as np
import pytest

from helpers import nrm_err
from test_gpu_attn_chain import attn_mask, bwd, fwd, inputs

pytestmark = pytest.mark.gpu


def raw_read(ptr, shape):
    """hipMemcpy (device to host) of a float32 array at a device address."""
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    out = np.empty(shape, np.float32)
    assert hip.hipMemcpy(out.ctypes.data, ctypes.c_void_p(ptr), out.nbytes, 2) == 0
    return out


@pytest.mark.parametrize("read_O_first", [True, False])
def test_probabilities_through_device_ptr(hip, cpu, read_O_first):
    B, H, T, dk = 2, 2, 128, 64   # whole 32 x 32 tiles: the forward keeps score blocks in A
    BH = B * H
    mask = attn_mask(B, H, T)
    arrs = inputs(11, BH, T, dk)

    def go(e, raw):
        q, k, v, g = (e.tensor(a) for a in arrs)
        A, O = fwd(e, q, k, v, e.tensor(mask), BH, T, 0.125)
        out = {}
        if read_O_first:
            out["O"] = O.numpy()   # the fused forward runs (A now holds score blocks)
        if raw:
            p = A.device_ptr()
            assert p
            e.sync()
            out["A"] = raw_read(p, (BH * T, T))
        else:
            out["A"] = A.numpy()
        if not read_O_first:
            out["O"] = O.numpy()
        gS, gq, gk, gv = bwd(e, q, k, v, A, g, BH, T, 0.125)
        out.update(dQ=gq.numpy(), dK=gk.numpy(), dV=gv.numpy())
        return out

    h, c = go(hip, True), go(cpu, False)
    tol = {"A": 1e-5, "O": 1e-4, "dQ": 1e-3, "dK": 1e-3, "dV": 1e-3}
    for name, a in h.items():
        assert np.isfinite(a).all(), name
        assert nrm_err(a, c[name]) <= tol[name], f"{name}: {nrm_err(a, c[name])}"


def test_device_ptr_plain_tensor(hip):
    """An ordinary tensor: the same address as nnhip_tensor_data_ptr, its values as uploaded."""
    a = np.arange(12, dtype=np.float32).reshape(3, 4)
    t = hip.tensor(a)
    p = t.device_ptr()
    assert p == t.data_ptr()
    hip.sync()
    assert np.array_equal(raw_read(p, a.shape), a)
