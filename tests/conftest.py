import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TESTS = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, TESTS):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box)")


def _build_if_missing():
    """Build only what is missing (the driver's build() compiles everything)."""
    oracle_so = os.path.join(ROOT, "oracle", "libkvattn_oracle.so")
    if not os.path.exists(oracle_so):
        subprocess.run(["make", "-C", os.path.join(ROOT, "oracle")], check=True)
    lib_so = os.path.join(ROOT, "cuda_gpt2_inference_amd", "libkvattn.so")
    if not os.path.exists(lib_so):
        subprocess.run(["make", "-C", os.path.join(ROOT, "cuda_gpt2_inference_amd", "csrc")], check=True)


_build_if_missing()


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")
