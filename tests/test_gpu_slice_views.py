"""slice_rows copy semantics (cpu_engine.hpp:75-114: a slice is a copy) on the
HIP engine, whose slices view their source until either side is written in
place: the same call sequences on the HIP engine and the oracle, compared
bit for bit after every in-place write that could reach shared memory."""
import numpy as np
import pytest

from helpers import nrm_err

pytestmark = pytest.mark.gpu


@pytest.fixture
def data():
    rng = np.random.default_rng(5)
    return dict(h=rng.standard_normal((8, 12)).astype(np.float32),
                x=rng.standard_normal((8, 12)).astype(np.float32),
                y=rng.standard_normal((2, 12)).astype(np.float32),
                v=rng.standard_normal((8, 1)).astype(np.float32),
                w=rng.standard_normal((12, 5)).astype(np.float32))


def test_source_written_after_slicing(hip, cpu, data):
    res = []
    for eng in (hip, cpu):
        h = eng.tensor(data["h"])
        a, b = eng.slice_rows(h, 0, 4), eng.slice_rows(h, 4, 4)
        c = eng.slice_rows(a, 1, 2)                 # slice of a slice
        eng.add_inplace(h, eng.tensor(data["x"]))
        r = [t.numpy() for t in (h, a, b, c)]
        eng.zero(h)
        eng.insert_rows(h, 3, eng.tensor(data["y"]))
        eng.broadcast_row_inplace(h, eng.tensor(data["v"]), "Add")
        r += [t.numpy() for t in (h, a, b, c)]
        res.append(r)
    for got, ref in zip(res[0], res[1]):
        assert np.array_equal(got, ref)
    assert np.array_equal(res[0][1], data["h"][0:4])   # the slices kept their rows
    assert np.array_equal(res[0][3], data["h"][1:3])


def test_slice_written_leaves_the_source(hip, cpu, data):
    res, prods = [], []
    for eng in (hip, cpu):
        h = eng.tensor(data["h"])
        a = eng.slice_rows(h, 2, 4)
        c = eng.slice_rows(a, 0, 2)
        eng.scale_inplace(a, 3.0)
        r = [t.numpy() for t in (h, a, c)]
        c.copy_from(np.ones((2, 12), np.float32))
        eng.axpy_inplace(c, 2.0, eng.tensor(data["y"]))
        r += [t.numpy() for t in (h, a, c)]
        res.append(r)
        prods.append(eng.matmul(eng.slice_rows(h, 1, 3), eng.tensor(data["w"])).numpy())   # a slice as an operand
    for got, ref in zip(res[0], res[1]):
        assert np.array_equal(got, ref)
    assert nrm_err(prods[0], prods[1]) <= 1e-5
    assert np.array_equal(res[0][0], data["h"])        # the source never changed
    assert np.array_equal(res[0][2], data["h"][2:4])   # c was cut before a was scaled


def test_unaligned_views(hip, cpu):
    """Slices at float offsets that are not 16-byte aligned (7 columns, cut at row 1): the copy-on-write
    path (one float per thread), a GEMM operand without vector loads, the generic ExprSpec interpreter
    and insert_rows read through such views; results match the oracle bit for bit (GEMM and the
    expression within their tolerances)."""
    import layer_programs as lp
    rng = np.random.default_rng(9)
    src = rng.standard_normal((9, 7)).astype(np.float32)
    w = rng.standard_normal((7, 5)).astype(np.float32)
    y = rng.standard_normal((3, 7)).astype(np.float32)
    spec, _ = lp.softmax_rows()
    res = []
    for eng in (hip, cpu):
        h = eng.tensor(src)
        a = eng.slice_rows(h, 1, 5)                     # view at float offset 7
        b = eng.slice_rows(a, 2, 3)                     # offset 21
        prod = eng.matmul(a, eng.tensor(w))
        prod_t = eng.matmul(b, eng.tensor(w.T.copy()), False, True)
        sm = eng.eval_expr(spec, [b] * 4, 3, 7)
        dst = eng.tensor(np.zeros((6, 7), np.float32))
        eng.insert_rows(dst, 1, b)
        eng.scale_inplace(b, -2.0)                      # copy-on-write of an unaligned view
        eng.insert_rows(h, 4, eng.tensor(y))            # source written after the views were cut
        res.append([t.numpy() for t in (h, a, b, dst)] + [prod.numpy(), prod_t.numpy(), sm.numpy()])
    for got, ref in zip(res[0][:4], res[1][:4]):
        assert np.array_equal(got, ref)
    for got, ref in zip(res[0][4:], res[1][4:]):
        assert nrm_err(got, ref) <= 1e-5
    assert np.array_equal(res[0][1], src[1:6]) and np.array_equal(res[0][2], -2.0 * src[3:6])
