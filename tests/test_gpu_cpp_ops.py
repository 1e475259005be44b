"""Runs the C++ ops:: parity test (tests/cpp/test_ops.cpp) on the GPU: the
reference-shaped C++ interface (Context/Tensor/ops::attention_*,
ops::linear_delta_*) over the C ABI, checked against the CPU oracle."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_cpp_ops_layer():
    exe = os.path.join(ROOT, "tests", "cpp", "test_ops")
    assert os.path.exists(exe), "build first: python -c 'import __graft_entry__ as g; g.build()'"
    r = subprocess.run([exe], capture_output=True, text=True, timeout=100)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "ALL OK" in r.stdout
