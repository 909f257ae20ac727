"""Engine selection on a GPU (reference cli/engine_factory.hpp:45-88 with use_hip first in priority):
a HIP request yields the HIP engine, which runs primitives like any engine; CUDA / Vulkan requests
and no request still fail with an error naming the engine to use, never falling back."""
import numpy as np
import pytest

import nnengine
from helpers import nrm_err, uniform

pytestmark = pytest.mark.gpu


def test_hip_request_yields_the_hip_engine():
    e = nnengine.create_engine(use_hip=True, use_cuda=True, use_gpu=True)   # HIP first in priority
    rng = np.random.default_rng(1)
    A, B = uniform(rng, (64, 48)), uniform(rng, (48, 80))
    C = e.matmul(e.tensor(A), e.tensor(B)).numpy()
    assert nrm_err(C, A.astype(np.float64) @ B.astype(np.float64)) <= 1e-5
    e.close()
    for kw, msg in ((dict(use_cuda=True), "CUDA"), (dict(use_gpu=True), "Vulkan"), ({}, "HIP engine only")):
        with pytest.raises(nnengine.EngineError, match=msg):
            nnengine.create_engine(**kw)
