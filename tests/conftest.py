import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs an MI355X (gfx950) GPU; runs the HIP library")


@pytest.fixture(scope="session")
def oracle():
    from oracle import q8_oracle
    q8_oracle.lib()
    return q8_oracle


@pytest.fixture(scope="session")
def q8():
    import llmcp_amd
    llmcp_amd.lib()
    return llmcp_amd


@pytest.fixture(scope="session")
def ctx(q8):
    c = q8.Context(0)
    yield c
    c.close()
