"""pytest configuration: the `gpu` marker and import paths.

Tests marked `gpu` need an MI355X (they call the HIP library through its C
ABI); everything else runs on the CPU.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("", "oracle", "cxx-gpt_amd", "tests"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and the built HIP library")


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import cxxgpt_attn
    cxxgpt_attn.lib()  # raises if the HIP library is missing: no fallback
    return torch.device("cuda:0")
