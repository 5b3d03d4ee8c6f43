import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "flash-moe_amd"), os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the libfmoe C ABI on cuda:0)")


@pytest.fixture(scope="session")
def orc():
    from oracle import OracleLib
    return OracleLib()


@pytest.fixture(scope="session")
def ref():
    from oracle import RefLib, REF_SO
    if not os.path.exists(REF_SO):
        pytest.skip("oracle/_ref not built (reference tree absent)")
    return RefLib()


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import fmoe_amd
    fmoe_amd.lib()
    return torch.device("cuda:0")
