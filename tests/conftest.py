"""Shared test setup: import paths, the `gpu` marker, and in-tree builds of
the oracle (gcc) and the product library when they are missing."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "tans-vectoradd_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)

if not os.path.exists(os.path.join(ROOT, "oracle", "liboracle.so")):
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)
if not os.path.exists(os.path.join(PKG, "rans_vectoradd", "libtans_amd.so")):
    subprocess.run([sys.executable, os.path.join(PKG, "build.py")], check=True)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (MI355X)")


@pytest.fixture(scope="session")
def lut():
    from oracle import oracle as O
    return O.add_lut()


def gpu_available() -> bool:
    import torch
    return torch.cuda.is_available()
