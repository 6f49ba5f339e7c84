import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "qwen38-3090-cuda-server_amd")
for p in (ROOT, PKG, os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def orc():
    import oracle

    return oracle


@pytest.fixture(params=["rows", "streamk"])
def decode_path(request, monkeypatch):
    """Runs a decode/verify test through both skinny kernels: the default
    data-parallel k_rows and the stream-K kernel (QW4_ROWS=0, read by the
    library on every call)."""
    if request.param == "streamk":
        monkeypatch.setenv("QW4_ROWS", "0")
    else:
        monkeypatch.delenv("QW4_ROWS", raising=False)
    return request.param
