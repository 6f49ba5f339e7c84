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


@pytest.fixture(params=["rows", "regs", "streamk"])
def decode_path(request, monkeypatch):
    """Runs a decode/verify test through every skinny kernel form: the default
    data-parallel k_rows (M = 1: items loaded straight into LDS), k_rows with
    items in registers (QW4_DMA=0) and the stream-K kernel (QW4_ROWS=0); the
    library reads both variables on every call."""
    monkeypatch.delenv("QW4_ROWS", raising=False)
    monkeypatch.delenv("QW4_DMA", raising=False)
    if request.param == "streamk":
        monkeypatch.setenv("QW4_ROWS", "0")
    elif request.param == "regs":
        monkeypatch.setenv("QW4_DMA", "0")
    return request.param
