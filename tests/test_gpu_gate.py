"""Runs the C++ gate over the call-compatible namespace qwen layer
(tests/cpp/gate_w4a16.cpp, built by __graft_entry__.build())."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

GATE = os.path.join(os.path.dirname(__file__), "cpp", "_build", "gate_w4a16")


def test_cpp_gate_namespace_qwen():
    assert os.path.exists(GATE), "gate not built: run __graft_entry__.build()"
    r = subprocess.run([GATE], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "gate_w4a16: PASS" in r.stdout
