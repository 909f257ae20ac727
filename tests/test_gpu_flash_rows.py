"""GPU parity of document-masked batches issued row by row (BASELINE config 5's call pattern).

The two-pass attention primitives take one (M, N) mask shared by the whole
batch (cpu_engine.hpp:426-915), so a batch of packed rows whose documents
differ is issued as one chain per row, the row's heads as the batch
(compute_layer.hpp:1196-1221 forward, :1304-1327 backward). HipEngine records
each row's fused forward and backward and runs the rows of one shape together
(one multi-row launch per 8 rows, k_flash.hip). These tests issue rows back to
back on the HIP engine and on the CPU oracle and compare every row's outputs:
plain runs of 2, 8 and 9 rows (8 + 1 launches), reads of one row's results
between rows (they run the recorded rows early), rows of two shapes
interleaved, and no score blocks kept (the backward forms its scores again).
At full size, 8 config-5 rows (H 12, T 2048, d 64) go through one launch; the
first and the last row are checked against dense float64 attention.
Tolerances: m, l 1e-5; O, R 1e-4; dQ, dK, dV 1e-3 (normwise).
"""
import numpy as np
import pytest

from helpers import doc_ids_from_lengths, doc_lengths, doc_mask, normal, nrm_err
from test_gpu_attention import _torch_attention

pytestmark = pytest.mark.gpu

TOL = dict(m=1e-5, l=1e-5, O=1e-4, R=1e-4, dQ=1e-3, dK=1e-3, dV=1e-3)


def _rows(seed, n, H, T, d, lo, hi):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        ids = doc_ids_from_lengths(doc_lengths(rng, T, lo, hi))
        out.append(dict(Q=normal(rng, (H * d, T)), K=normal(rng, (H * d, T)), V=normal(rng, (H * d, T)),
                        dO=normal(rng, (H * d, T)), mask=doc_mask(ids), H=H, T=T, d=d))
    return out


def _issue(e, r, alpha):
    """One row's reference call sequence; its device results, kept alive by the caller."""
    H, T, d = r["H"], r["T"], r["d"]
    q, k, v, g, mk = (e.tensor(r[n]) for n in ("Q", "K", "V", "dO", "mask"))
    m = e.batched_matmul_reduce(q, k, H, "Max", True, False, alpha, True, mk)
    l = e.batched_matmul_softmax_denom(q, k, m, H, True, False, alpha, mk)
    vt = e.rearrange_3d(e.transpose(v), T, H, d)
    o = e.batched_matmul_softmax_apply(q, k, vt, m, l, H, True, False, alpha, mk)
    P = e.batched_matmul(g, v, H, True, False)
    G = e.rearrange_3d(e.transpose(g), T, H, d)
    dq, R = e.batched_matmul_softmax_backward_q(q, k, P, m, l, H, True, False, alpha, mk)
    dk, dv = e.batched_matmul_softmax_backward_kv(q, k, P, G, R, m, l, H, True, False, alpha, mk)
    return dict(m=m, l=l, O=o, dQ=dq, R=R, dK=dk, dV=dv)


def _read(res):
    return {n: t.numpy() for n, t in res.items()}


def _check(got, ref, where):
    for n, t in TOL.items():
        assert nrm_err(got[n], ref[n]) <= t, (where, n, nrm_err(got[n], ref[n]))


@pytest.mark.parametrize("n", [2, 8, 9])
def test_rows_back_to_back(hip, cpu, n):
    rows = _rows(100 + n, n, 4, 256, 64, 16, 128)
    held = [_issue(hip, r, 0.125) for r in rows]   # every row recorded before any result is read
    got = [_read(h) for h in held]
    for i, r in enumerate(rows):
        _check(got[i], _read(_issue(cpu, r, 0.125)), f"row {i}")


def test_reads_between_rows(hip, cpu):
    rows = _rows(7, 6, 4, 192, 64, 16, 96)
    held, early = [], {}
    for i, r in enumerate(rows):
        held.append(_issue(hip, r, 0.125))
        if i == 2:
            early["dQ1"] = held[1]["dQ"].numpy()   # runs rows 0-2 (forwards and backwards) now
        if i == 4:
            early["O4"] = held[4]["O"].numpy()     # a forward's result while rows 3-4 wait
    got = [_read(h) for h in held]
    refs = [_read(_issue(cpu, r, 0.125)) for r in rows]
    for i in range(len(rows)):
        _check(got[i], refs[i], f"row {i}")
    assert nrm_err(early["dQ1"], refs[1]["dQ"]) <= 1e-3
    assert nrm_err(early["O4"], refs[4]["O"]) <= 1e-4


def test_rows_of_two_shapes_interleaved(hip, cpu):
    a = _rows(11, 3, 4, 256, 64, 32, 128)
    b = _rows(12, 3, 2, 160, 32, 16, 64)
    rows = [x for pair in zip(a, b) for x in pair]
    held = [_issue(hip, r, 1.0 / np.sqrt(r["d"])) for r in rows]
    got = [_read(h) for h in held]
    for i, r in enumerate(rows):
        _check(got[i], _read(_issue(cpu, r, 1.0 / np.sqrt(r["d"]))), f"row {i}")


def test_rows_without_score_blocks(hip, cpu):
    """Score budget 0: no forward keeps its score blocks, every backward forms the scores itself."""
    rows = _rows(21, 4, 4, 256, 64, 16, 128)
    try:
        hip.set_score_budget(0)
        held = [_issue(hip, r, 0.125) for r in rows]
        got = [_read(h) for h in held]
    finally:
        hip.set_score_budget(8 << 30)
    for i, r in enumerate(rows):
        _check(got[i], _read(_issue(cpu, r, 0.125)), f"row {i}")


def test_config5_eight_rows_one_launch(hip):
    """8 rows, H 12, T 2048, d 64, documents U{64..1024}; rows 0 and 7 against
    dense float64 attention (their arrays sit at the two ends of the launch's row table)."""
    rows = _rows(55, 8, 12, 2048, 64, 64, 1024)
    held = [_issue(hip, r, 0.125) for r in rows]
    hip.settle()
    for i in (0, 7):
        r, got = rows[i], _read(held[i])
        H, T, d = 12, 2048, 64
        ref = _torch_attention(r["Q"], r["K"], r["V"], r["mask"], 0.125, H, d, r["dO"])
        assert nrm_err(got["O"], ref["O"].reshape(H * T, d)) <= 1e-4, i
        assert nrm_err(got["m"][:, 0], ref["m"].reshape(-1)) <= 1e-5, i
        assert nrm_err(got["l"][:, 0], ref["l"].reshape(-1)) <= 1e-5, i
        R_ref = (r["dO"].astype(np.float64).reshape(H, d, T).transpose(0, 2, 1) * ref["O"]).sum(-1)
        assert nrm_err(got["R"][:, 0], R_ref.reshape(-1)) <= 1e-4, i
        for n in ("dQ", "dK", "dV"):
            assert nrm_err(got[n], ref[n].reshape(H * d, T)) <= 1e-3, (i, n)
