"""Shared fixtures. GPU tests carry @pytest.mark.gpu and call libtsr_hip through its C ABI; the CPU
checkers (oracle/) are used only as checkers."""
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(REPO, "oracle"))
sys.path.insert(0, os.path.join(REPO, "tesseract-npu_amd"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs libtsr_hip kernels)")


@pytest.fixture(scope="session")
def oc():
    import oracle
    return oracle.Oracle()


@pytest.fixture(scope="session")
def ref():
    import oracle
    if not oracle.ref_available():
        pytest.skip("oracle/_ref/libtsr_ref.so not built (needs /root/reference)")
    return oracle.Ref()


@pytest.fixture(scope="session")
def dev():
    import tsr_hip
    d = tsr_hip.Device(0)
    yield d
    d.close()
