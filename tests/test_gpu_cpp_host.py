"""Runs the C++ host-mirror parity program (tests/cpp/qmat_parity.cpp, built by
__graft_entry__.build()) on the GPU: QMat/MoE through rusty_engine.hpp against the oracle."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu
EXE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "qmat_parity")


def test_cpp_host_mirror_parity():
    assert os.path.exists(EXE), "tests/cpp/qmat_parity is not built (run __graft_entry__.build())"
    r = subprocess.run([EXE], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "ALL PASSED" in r.stdout
