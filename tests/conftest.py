"""Shared pytest setup: markers, import paths, and the built libraries."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("", "oracle", "sam-rs_amd", "tests"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libsam_hip.so")


@pytest.fixture(scope="session")
def oracle_lib():
    import sam_oracle as oracle

    oracle.build()
    return oracle
