import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "mrl-index-rust-vector_amd"), os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP library)")
    config.addinivalue_line("markers", "slow: large inputs")


_GPU = None


def gpu_available() -> bool:
    """True when the HIP library can open device 0 (no torch import needed)."""
    global _GPU
    if _GPU is None:
        try:
            import mrl_index_amd as m
            m.default_device()
            _GPU = True
        except Exception:
            _GPU = False
    return _GPU


@pytest.fixture(scope="session")
def device():
    import mrl_index_amd as m
    if not gpu_available():
        pytest.skip("no GPU")
    return m.default_device()
