import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; calls the HIP path through the C ABI")
    config.addinivalue_line("markers", "slow: long-running CPU test")


@pytest.fixture(scope="session")
def orc():
    import oracle

    oracle.build()
    return oracle


@pytest.fixture(scope="session")
def golden_dir():
    return os.path.join(ROOT, "tests", "golden")


@pytest.fixture(scope="session")
def dev():
    """The gfx950 device context (GPU tests only). No fallback: fails if the library is missing."""
    import example_matmul_metal4_amd as mtk

    d = mtk.Device(0)
    info = d.info
    print(f"\n[device] {info['name']} {info['arch']} CUs={info['compute_units']} clock={info['clock_khz']} kHz",
          flush=True)
    yield d
    d.close()
