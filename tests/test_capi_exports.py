"""The C-ABI boundary, checked on the CPU (no device calls).

Every function declared in include/*.h must be exported by libnnhip.so; the
engine-level subset (nnhip_engine.h) must also be exported by the oracle
library under its own prefix, so the parity tests drive both through one
binding. The ExprSpec serialisation of the Python host mirror is checked
against the byte layout the headers document.
"""
import ctypes
import glob
import os
import re

import numpy as np
import pytest

import nnengine
from conftest import ORACLE_LIB, ROOT

HEADERS = sorted(glob.glob(os.path.join(ROOT, "include", "*.h")))
_DECL = re.compile(r"\b(nnhip_[A-Za-z0-9_]+)\s*\(")


def _declared(path):
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = set(_DECL.findall(text))
    return sorted(names)


def test_headers_present():
    names = [os.path.basename(h) for h in HEADERS]
    assert "nnhip_kernels.h" in names and "nnhip_engine.h" in names


@pytest.mark.parametrize("header", HEADERS, ids=os.path.basename)
def test_product_library_exports_every_declared_symbol(header):
    lib = nnengine.hip_library()
    names = _declared(header)
    assert len(names) > 10
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"libnnhip.so lacks {missing}"


def test_oracle_mirrors_engine_abi():
    lib = ctypes.CDLL(ORACLE_LIB)
    names = [n for n in _declared(os.path.join(ROOT, "include", "nnhip_engine.h"))
             if not n.startswith("nnhip_engine_profile")
             and n not in ("nnhip_engine_stream", "nnhip_engine_settle", "nnhip_engine_select",
                           "nnhip_engine_set_score_budget")]
    missing = [n for n in names if not hasattr(lib, "nnoracle_" + n[len("nnhip_"):])]
    assert not missing, f"oracle lacks the mirror of {missing}"


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(nnengine, "HIP_LIB_PATH", str(tmp_path / "absent.so"))
    with pytest.raises(nnengine.EngineError):
        nnengine.hip_library()


def test_op_codes_match_header():
    text = open(os.path.join(ROOT, "include", "nnhip_engine.h")).read()
    codes = {m.group(1): int(m.group(2)) for m in re.finditer(r"NNHIP_OP_([A-Z0-9_]+)\s*=\s*(\d+)", text)}
    assert codes == nnengine.OP


def test_expr_spec_serialisation_layout():
    s = nnengine.ExprSpec(num_regs=2)
    s.view("Linear")
    s.view("ColBroadcast", param=3, negate=1)
    c = s.const(0.5)
    s.ins("Mul", nnengine.inp(0), nnengine.inp(1), dst=0)
    s.ins("Add", nnengine.reg(0), nnengine.cst(c), dst=1)
    instrs, kinds, params, consts = s.serialise()
    assert instrs.dtype == np.uint8 and instrs.shape == (2, 8)
    assert list(instrs[1][:4]) == [nnengine.EXPR_OP["Add"], 1, nnengine.OPND["Reg"], 0]
    assert list(instrs[1][4:6]) == [nnengine.OPND["Const"], 0]
    assert list(kinds) == [nnengine.VIEW["Linear"], 0, nnengine.VIEW["ColBroadcast"], 1]
    assert list(params) == [0, 3] and consts.dtype == np.float32 and consts[0] == 0.5


def test_engine_selection_never_falls_back():
    """cli::create_engine's rules (reference cli/engine_factory.hpp:45-88) with use_hip added: a requested
    backend that cannot be created is an error, never another engine. This container has no GPU, so a HIP
    request fails here; CUDA / Vulkan requests and no request name the reference's engines."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present: the HIP request succeeds (tests/test_gpu_engine_select.py)")
    with pytest.raises(nnengine.EngineError, match="no fallback"):
        nnengine.create_engine(use_hip=True)
    with pytest.raises(nnengine.EngineError, match="CUDA.*no fallback"):
        nnengine.create_engine(use_cuda=True)
    with pytest.raises(nnengine.EngineError, match="Vulkan.*no fallback"):
        nnengine.create_engine(use_gpu=True)
    with pytest.raises(nnengine.EngineError, match="HIP engine only"):
        nnengine.create_engine()
