"""The grid and workspace layout helpers the kernels share with host code (csrc/layout.hpp),
built with the host compiler and checked on the CPU (tests/cpp/layout_check.cpp):
div_uniform against integer division; the XCD-local designated grid (12 heads on a grid padded
to 16, 40, 768 ...) as a bijection onto the real (head, segment) slots with every segment of a
head on one XCD; every workgroup of designated grids for B in {1, 2, 3, 17}, NH 1..40, S 1..64
(padding slots exit before any load, live slots' speculative rows, q row, partial and tag
indices inside their buffers); workspace layouts of one plan and of two plans sharing a buffer.
Planted mistakes (the one-sequence shortcut that faulted a GPU, a missing guess guard, a
counter region sized by the plan) must fail it.  A mapping mistake there shows up on the GPU
as slots that never publish or as padding slots that run past the buffers, so it is pinned
here first."""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))


def test_layout_helpers():
    cpp = os.path.join(HERE, "cpp")
    subprocess.run(["make", "-s", "-C", cpp, "layout_check"], check=True, capture_output=True)
    r = subprocess.run([os.path.join(cpp, "layout_check")], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and r.stdout.strip() == "ok", r.stdout + r.stderr
