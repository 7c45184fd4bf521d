"""C++ hosts of the library, checked against the CPU oracle: the port of the reference lab's
correctness loop (tests/cpp/lab_check.cpp) through the C++ mirror of the reference entry
points (include/kvattn_gpt2.hpp), and the attention block of a 12-layer decode step captured
once as a HIP graph and replayed for T = 1..1024 (tests/cpp/step_check.cpp); and the eager
timing tool bench.py runs (tests/cpp/eager_timing.cpp) exits cleanly."""
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


@pytest.mark.parametrize("dtype", ["bf16", "int8"])
def test_eager_timing_binary(dev, dtype):
    """The eager-call timing tool bench.py reports: runs the 12-layer step through the C-ABI
    from C++, exits 0 with a clean workspace status and a positive per-call time."""
    import json
    exe = os.path.join(HERE, "cpp", "eager_timing")
    if not os.path.exists(exe):
        subprocess.run(["make", "-C", os.path.join(HERE, "cpp")], check=True)
    r = subprocess.run([exe, dtype, "2", "12", "1024", "700", "12", "5"], capture_output=True, text=True,
                       timeout=110)
    assert r.returncode == 0, r.stdout + r.stderr
    rec = json.loads(r.stdout.strip().splitlines()[-1])
    assert rec["workspace_status"] == 0 and rec["us_per_call"] > 0 and rec["layers"] == 12
