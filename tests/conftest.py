# SPDX-License-Identifier: Apache-2.0
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "metal-flat_amd"), os.path.join(ROOT, "oracle"), os.path.dirname(__file__)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def oracle_threads():
    return max(1, min(16, os.cpu_count() or 1))


@pytest.fixture(scope="session")
def gpu_ok():
    import mflat

    mflat.load()
    idx = mflat.FlatIndex(8)
    ready = idx.ready()
    idx.close()
    if not ready:
        pytest.fail("GPU test collected but no gfx950 device is usable")
    return True
