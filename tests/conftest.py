"""Shared test setup: import paths, the `gpu` marker, device fixtures."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "gpu-talored-ann_amd")
ORACLE = os.path.join(ROOT, "oracle")
for p in (PKG, ORACLE, ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP library)")


@pytest.fixture(scope="session")
def ctx():
    import gtann
    c = gtann.Context(0)
    yield c
    c.close()


def pytest_sessionfinish(session, exitstatus):
    # the float tolerance's calibration data, when float tests ran
    import helpers
    if helpers.ERR_ULPS_MAX:
        print("\n[floor] largest error in ulps of the operand magnitude, by (metric, D): " +
              ", ".join(f"{m} D={d}: {v:.2f}" for (m, d), v in sorted(helpers.ERR_ULPS_MAX.items())), flush=True)
