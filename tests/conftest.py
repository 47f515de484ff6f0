import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "qwen-mobile-agent_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def orc():
    import orc as _orc
    _orc.lib()
    return _orc


@pytest.fixture(scope="session")
def qm():
    """The GPU library, initialised on device 0 (GPU tests only)."""
    import qmag as _qm
    _qm.init(0)
    return _qm


def max_rel_err(got, ref):
    import numpy as np
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.all(np.isfinite(got)), "non-finite GPU output"
    scale = np.max(np.abs(ref))
    # an all-zero reference would make any all-zero output "match": no test
    # here has a legitimately zero result, so treat it as a failure
    assert scale > 0, "degenerate all-zero reference"
    return float(np.max(np.abs(got - ref)) / scale)
