import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_PARENT = os.path.join(ROOT, "lightning-unified-video-editor-via-in-context-sparse-attention_amd")
for p in (ROOT, PKG_PARENT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library on cuda:0)")
    config.addinivalue_line("markers", "cpu: runs on the host only (oracle, host logic, library load)")


@pytest.fixture(scope="session")
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from icsa_hip import _lib
    _lib.lib()   # fail loudly if the native library is missing
    return torch.device("cuda:0")
