"""C++ hosts of the library, checked against the CPU oracle: the port of the reference lab's
correctness loop (tests/cpp/lab_check.cpp) through the C++ mirror of the reference entry
points (include/kvattn_gpt2.hpp), and the attention block of a 12-layer decode step captured
once as a HIP graph and replayed for T = 1..1024 (tests/cpp/step_check.cpp)."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))


def test_lab_check_binary(dev):
    exe = os.path.join(HERE, "cpp", "lab_check")
    if not os.path.exists(exe):
        subprocess.run(["make", "-C", os.path.join(HERE, "cpp")], check=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=110)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "-> all passed" in r.stdout


def test_decode_step_graph_binary(dev):
    exe = os.path.join(HERE, "cpp", "step_check")
    if not os.path.exists(exe):
        subprocess.run(["make", "-C", os.path.join(HERE, "cpp")], check=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=110)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "-> all passed" in r.stdout
