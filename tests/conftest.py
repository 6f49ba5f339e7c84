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


@pytest.fixture(params=["dec", "rows", "regs"])
def decode_path(request):
    """Runs a decode/verify test through every skinny kernel form: the default
    (M = 1: the integer-MFMA k_dec; M > 1: k_rows with LDS-DMA items, the
    activation rows staged in LDS where the policy stages them), k_rows at
    M = 1 too with the M > 1 activations loaded with each item, and k_rows
    with items in registers for every M, through the library's tuning
    override (qw4_tune_decode), reset afterwards."""
    import w4a16_hip as hip

    hip.tune_decode({"dec": 0, "rows": 1, "regs": 2}[request.param])
    yield request.param
    hip.tune_decode(0)
