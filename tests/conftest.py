import os
import sys

import torch  # noqa: F401  (import before any ctypes load of libhn_int4.so)
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def pytest_collection_modifyitems(config, items):
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def _announce(item):
    # name the case before any GPU step runs, so a crash is attributable
    print(f"\n[case] {item.nodeid}", flush=True)


@pytest.hookimpl(tryfirst=True)
def pytest_runtest_setup(item):
    if "gpu" in item.keywords:
        _announce(item)


@pytest.fixture(params=[0, 1], ids=["stream", "splitk"])
def decode_path(request):
    """Run a decode test through both kernel families: 0 = automatic (the
    persistent streaming kernels where they apply), 1 = split-K kernels only."""
    from hydranet_amd import _lib
    _lib.set_decode_path(request.param)
    yield request.param
    _lib.set_decode_path(0)
