"""Shared fixtures. `-m "not gpu"` runs the oracle pins, host logic and the
ABI symbol checks on the CPU; `-m gpu` runs the HIP parity tests through the
C ABI (libqmm_hip.so), which must be built — a missing library fails loudly."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "npu880-mtk-npu-llm-runtime_amd")
ORACLE_DIR = os.path.join(ROOT, "oracle")
for p in (PKG, ORACLE_DIR):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and libqmm_hip.so")


@pytest.fixture(scope="session")
def oracle():
    import oracle as o
    return o.load_oracle()


@pytest.fixture(scope="session")
def ref():
    import oracle as o
    r = o.load_reference()
    if r is None:
        pytest.skip("compiled reference (oracle/_ref) not built here")
    return r


@pytest.fixture(scope="session")
def ctx():
    import qmm_hip
    c = qmm_hip.Context(0)  # raises if the library or the GPU is missing
    info = c.device_info()
    print(f"[gpu] {info}", flush=True)
    yield c
    c.close()
