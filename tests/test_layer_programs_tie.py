"""The Python copies of the GPT layer programs (neuralnet.cpp_amd/layer_programs.py)
against the C++ ones the engine recognises (include/nn/layer_exprs.hpp, exported
serialised by nnhip_layer_program from the product library and from the oracle).

The GPU tests and the bench's memory-bound leg issue these Python programs to
reach the fused kernels; a Python program that differed from the C++ one in
any instruction, view, constant, register count or input-slot binding would be
run by the generic interpreter instead and those tests would measure the wrong
kernel. Host-only: no GPU is used.
"""
import ctypes

import numpy as np
import pytest

import layer_programs as lp
import nnengine
from conftest import ORACLE_LIB

DK = 64
BUILDERS = {name: fn for name, (fn, _, _) in lp.PROGRAMS.items()}
BUILDERS.update(softmax_rows=lp.softmax_rows, softmax_rows_backward=lp.softmax_rows_backward,
                rope=lambda: lp.rope(DK), rope_backward=lambda: lp.rope(DK, backward=True))


def _libs():
    return [("nnhip_", nnengine.hip_library()), ("nnoracle_", ctypes.CDLL(ORACLE_LIB))]


@pytest.mark.parametrize("name", sorted(lp.ARGS))
def test_python_program_equals_engine_program(name):
    spec, slots = BUILDERS[name]()
    cname, args = lp.ARGS[name]
    want_slots = [args.index(s) for s in slots]
    for prefix, lib in _libs():
        c = nnengine.layer_program(lib, cname, DK if cname.startswith("rope") else 0, prefix=prefix)
        assert c["instrs"] == [tuple(t) for t in spec.instrs], (prefix, name)
        assert c["views"] == [tuple(v) for v in spec.views], (prefix, name)
        assert np.array_equal(np.float32(c["consts"]), np.float32(spec.consts)), (prefix, name)
        assert c["num_regs"] == spec.num_regs, (prefix, name)
        assert c["slot_args"] == want_slots, (prefix, name)


def test_every_engine_program_has_a_python_copy():
    assert set(BUILDERS) >= set(lp.ARGS)
    assert {c for c, _ in lp.ARGS.values()} == {
        "rms_sum_sq", "rms_normalize", "rms_scale", "rms_bwd_colsum", "rms_bwd_dx", "rms_bwd_rowsum",
        "softmax_rows", "softmax_rows_backward", "swiglu_grad_gate", "swiglu_grad_up", "rope_forward",
        "rope_backward"}


def test_unknown_program_is_an_error():
    with pytest.raises(nnengine.EngineError, match="unknown program"):
        nnengine.layer_program(nnengine.hip_library(), "no_such_program")


def test_a_changed_program_is_detected():
    """A Python copy that differs in one operand (a planted mistake) no longer matches."""
    spec, _ = lp.swiglu_grad_up()
    i = spec.instrs[-1]              # Mul(reg r0, input 2): read input 1 instead
    assert i[4] == nnengine.OPND["Input"] and i[5] == 2
    spec.instrs[-1] = i[:5] + (1,) + i[6:]
    c = nnengine.layer_program(nnengine.hip_library(), "swiglu_grad_up")
    assert c["instrs"] != [tuple(t) for t in spec.instrs]
