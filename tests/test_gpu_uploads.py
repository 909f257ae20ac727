"""Host-to-device uploads and vector transposes through the HIP engine.

from_matrix and copy_from (compute_engine.hpp) copy small host data into a slot
of a pinned staging ring and return once the upload is queued (no wait for the
stream); larger data is uploaded and waited for. Checked: more uploads than the
ring has slots, each read back after all of them, against the host data bit for
bit; copy_from into a tensor that queued work still reads; the large path; and
transposes of row and column vectors (plain copies of the same floats).
"""
import numpy as np
import pytest

from helpers import normal

pytestmark = pytest.mark.gpu


def test_many_small_uploads_bit_exact(hip):
    rng = np.random.default_rng(1)
    hosts = [normal(rng, (int(rng.integers(1, 300)), int(rng.integers(1, 200)))) for _ in range(200)]
    ts = [hip.tensor(h) for h in hosts]            # 200 uploads through a 64-slot ring
    for h, t in zip(hosts, ts):
        assert np.array_equal(t.numpy().view(np.uint32), h.view(np.uint32))


def test_upload_order_against_queued_work(hip):
    """copy_from into a tensor while queued kernels still read its old contents, then one of them
    again: each product sees the contents at its call, as the stream orders them."""
    rng = np.random.default_rng(2)
    A, B1, B2 = normal(rng, (512, 512)), normal(rng, (512, 64)), normal(rng, (512, 64))
    a, b = hip.tensor(A), hip.tensor(B1)
    c1 = hip.matmul(a, b)
    b.copy_from(B2)
    c2 = hip.matmul(a, b)
    ref1 = A.astype(np.float64) @ B1.astype(np.float64)
    ref2 = A.astype(np.float64) @ B2.astype(np.float64)
    assert np.abs(c1.numpy() - ref1).max() <= 1e-4 * np.abs(ref1).max()
    assert np.abs(c2.numpy() - ref2).max() <= 1e-4 * np.abs(ref2).max()


def test_large_upload(hip):
    rng = np.random.default_rng(3)
    H = normal(rng, (1024, 1024))                 # 4 MB: the waited-for path
    assert np.array_equal(hip.tensor(H).numpy().view(np.uint32), H.view(np.uint32))


@pytest.mark.parametrize("shape", [(1, 768), (768, 1), (1, 1), (1, 5)])
def test_vector_transpose(hip, shape):
    rng = np.random.default_rng(4)
    X = normal(rng, shape)
    assert np.array_equal(hip.transpose(hip.tensor(X)).numpy().view(np.uint32), X.T.copy().view(np.uint32))
