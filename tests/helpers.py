"""Shared numeric helpers for the parity tests."""
import numpy as np


def nrm_err(got, ref):
    """Normwise error max|got - ref| / max|ref| (0 when both are all zero)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    if got.size == 0:
        return 0.0
    den = np.abs(ref).max()
    num = np.abs(got - ref).max()
    return float(num / den) if den > 0 else float(num)


def uniform(rng, shape, lo=-1.0, hi=1.0):
    return rng.uniform(lo, hi, size=shape).astype(np.float32)


def normal(rng, shape, std=1.0):
    return rng.normal(0.0, std, size=shape).astype(np.float32)


def causal_mask(T):
    m = np.zeros((T, T), dtype=np.float32)
    m[np.triu_indices(T, 1)] = -np.inf
    return m


def doc_mask(doc_ids):
    """Causal AND same-document (T,T) mask from per-position document ids."""
    d = np.asarray(doc_ids)
    T = d.size
    allowed = (np.arange(T)[None, :] <= np.arange(T)[:, None]) & (d[None, :] == d[:, None])
    return np.where(allowed, 0.0, -np.inf).astype(np.float32)


def doc_lengths(rng, T, lo, hi):
    """Document lengths drawn U{lo..hi} until they cover T, the last one truncated."""
    out, total = [], 0
    while total < T:
        L = int(rng.integers(lo, hi + 1))
        L = min(L, T - total)
        out.append(L)
        total += L
    return out


def doc_ids_from_lengths(lengths):
    return np.concatenate([np.full(L, i + 1, dtype=np.int64) for i, L in enumerate(lengths)])


def grad_errs(got, ref, floor_rel=1e-4):
    """Normwise error per gradient tensor, with the denominator floored at
    floor_rel * (largest |gradient| over all tensors). Gradients that vanish
    identically, such as the key bias (each softmax row is invariant to a
    constant added to its scores), hold only rounding noise; the floor keeps
    noise-vs-noise comparisons from dominating."""
    scale = max(float(np.abs(np.asarray(r, dtype=np.float64)).max()) for r in ref if np.asarray(r).size)
    out = []
    for a, b in zip(got, ref):
        a = np.asarray(a, dtype=np.float64)
        b = np.asarray(b, dtype=np.float64)
        den = max(float(np.abs(b).max()) if b.size else 0.0, floor_rel * scale)
        out.append(float(np.abs(a - b).max() / den) if b.size else 0.0)
    return out
