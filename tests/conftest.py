"""Shared test setup.

CPU tests (default) check the oracle (the CPU restatement of the reference
CpuEngine under oracle/) against closed forms, brute force, finite differences
and an independent float64 torch restatement, plus the host logic and the
exports of the product library. GPU tests (marked ``gpu``) drive the HIP
engine and the oracle through the same C-ABI on the same seeded inputs.
"""
import ctypes
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "neuralnet.cpp_amd"))
sys.path.insert(0, os.path.join(ROOT, "tests"))

import nnengine  # noqa: E402

ORACLE_LIB = os.path.join(ROOT, "oracle", "_build", "libnnoracle.so")

# The oracle's thread pool reads NNORACLE_THREADS once, at first use: size it to
# the CPUs this process may run on, at most 16 (a GPU box's share of its host).
os.environ.setdefault("NNORACLE_THREADS", str(max(1, min(len(os.sched_getaffinity(0)), 16))))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP engine parity / kernels)")


def oracle_engine() -> "nnengine.Engine":
    if not os.path.exists(ORACLE_LIB):
        raise RuntimeError(f"{ORACLE_LIB} missing: run `make -C oracle` or __graft_entry__.build()")
    return nnengine.Engine(ctypes.CDLL(ORACLE_LIB), prefix="nnoracle_")


@pytest.fixture(scope="session")
def cpu():
    return oracle_engine()


@pytest.fixture(scope="session")
def hip():
    return nnengine.Engine()


def rng(seed):
    return np.random.default_rng(seed)
