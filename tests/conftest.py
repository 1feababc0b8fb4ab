"""Test configuration: the ``gpu`` marker and import paths.

CPU tests (``-m "not gpu"``) pin the oracle and check the C ABI's host-side
behaviour; GPU tests (``-m gpu``) compare the HIP library with the oracle.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "vkqlora.rs_amd"), os.path.join(ROOT, "oracle"),
          os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


@pytest.fixture(scope="session")
def ctx():
    import qlora_hip
    c = qlora_hip.Context()  # raises NoDevice without a GPU: no CPU fallback
    print(f"device: {c.device_name()}", flush=True)
    yield c
