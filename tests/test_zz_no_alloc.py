"""nnhip_gemm_noalloc (include/nnhip_kernels.h), the GEMM entry point that allocates nothing: its
split-K partials live in the library's per-GPU scratch array. Called through the C-ABI on device
buffers owned by a HIP engine, on that engine's stream, and compared with nnhip_gemm given a workspace
of nnhip_gemm_workspace_bytes: same plan and summation order, so the results must be bit-identical.
Two calls in a row (the second smaller, so stale scratch contents from the first are present), shapes
with and without split-K, and the rejection of a product whose partials exceed the scratch."""
import ctypes

import numpy as np
import pytest

import nnengine
from helpers import uniform

pytestmark = pytest.mark.gpu

SZ = ctypes.c_size_t
SCRATCH = 64 << 20


def _lib():
    lib = nnengine.hip_library()
    lib.nnhip_gemm_workspace_bytes.restype = SZ
    lib.nnhip_gemm_workspace_bytes.argtypes = [SZ] * 4
    lib.nnhip_gemm.argtypes = [ctypes.c_void_p] * 3 + [SZ] * 5 + [ctypes.c_int] * 2 + [ctypes.c_float, ctypes.c_void_p,
                                                                                        SZ, ctypes.c_void_p]
    lib.nnhip_gemm_noalloc.argtypes = [ctypes.c_void_p] * 3 + [SZ] * 5 + [ctypes.c_int] * 2 + [ctypes.c_float,
                                                                                                ctypes.c_void_p]
    lib.nnhip_engine_stream.restype = ctypes.c_void_p
    lib.nnhip_engine_stream.argtypes = [ctypes.c_void_p]
    return lib


def _pair(hip, lib, M, N, K, batch, tA, tB, alpha, seed):
    """(C from nnhip_gemm with a workspace, C from nnhip_gemm_noalloc, workspace bytes)."""
    rng = np.random.default_rng(seed)
    A = uniform(rng, (batch * (K if tA else M), M if tA else K))
    B = uniform(rng, (batch * (N if tB else K), K if tB else N))
    a, b = hip.tensor(A), hip.tensor(B)
    c_ref, c_na = hip.create_tensor(batch * M, N), hip.create_tensor(batch * M, N)
    ws_bytes = lib.nnhip_gemm_workspace_bytes(M, N, K, batch)
    ws = hip.create_tensor(max(1, ws_bytes // 4), 1)
    hip.sync()
    stream = lib.nnhip_engine_stream(hip._e)
    args = (a.data_ptr(), b.data_ptr())
    dims = (A.shape[0], A.shape[1], B.shape[0], B.shape[1], batch, int(tA), int(tB), alpha)
    print(f"[noalloc] M {M} N {N} K {K} batch {batch} tA {tA} tB {tB} ws {ws_bytes}", flush=True)
    assert lib.nnhip_gemm(*args, c_ref.data_ptr(), *dims, ws.data_ptr() if ws_bytes else None, ws_bytes, stream) == 0
    assert lib.nnhip_gemm_noalloc(*args, c_na.data_ptr(), *dims, stream) == 0
    return c_ref.numpy(), c_na.numpy(), ws_bytes


@pytest.mark.parametrize("first,second", [
    ((768, 2048, 8192, 1, False, True), (256, 384, 2048, 1, False, True)),    # split-K twice, smaller second
    ((768, 768, 8192, 1, False, True), (100, 70, 3001, 1, True, False)),      # weight-gradient shape, ragged
    ((1024, 64, 1024, 12, False, True), (300, 200, 1500, 1, False, False)),   # batched split-K, ragged
    ((512, 1024, 256, 2, True, False), (37, 53, 29, 1, True, True)),          # no split at all
])
def test_noalloc_matches_gemm_twice(hip, first, second):
    lib = _lib()
    ws_seen = []
    for i, (M, N, K, batch, tA, tB) in enumerate((first, second)):
        ref, got, ws = _pair(hip, lib, M, N, K, batch, tA, tB, 0.75, seed=i + M)
        assert np.array_equal(got, ref)
        ws_seen.append(ws)
    assert max(ws_seen) <= SCRATCH


def test_noalloc_rejects_beyond_scratch(hip):
    """The 6144 x 768 weight gradient over 8192 tokens splits K into partials of 144 MiB: rejected with
    -6 on the host, nothing launched (the output keeps its contents)."""
    lib = _lib()
    M, N, K = 6144, 768, 8192
    need = lib.nnhip_gemm_workspace_bytes(M, N, K, 1)
    assert need > SCRATCH, need
    a, b = hip.create_tensor(M, K), hip.create_tensor(N, K)
    c = hip.tensor(np.full((M, N), 3.0, np.float32))
    hip.sync()
    stream = lib.nnhip_engine_stream(hip._e)
    assert lib.nnhip_gemm_noalloc(a.data_ptr(), b.data_ptr(), c.data_ptr(), M, K, N, K, 1, 0, 1, 1.0, stream) == -6
    assert np.all(c.numpy() == 3.0)
