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


# Every GPU test that takes `ctx` runs once per reference platform: the
# aarch64 SDOT arithmetic (fma epilogue, the library default) and the x86
# scalar path (mul+add); `ctx.epilogue` names the oracle variant to match.
@pytest.fixture(scope="session", params=["aarch64", "x86"])
def ctx(q8, request):
    c = q8.Context(0)
    c.set_platform(request.param)
    yield c
    c.close()
