"""pytest configuration: the `gpu` marker, import paths, and GPU-test gating."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "specdec-quant-triton_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libspecq.so on the device)")


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def built_lib():
    """Path of libspecq.so, building it in-tree first if it is missing."""
    from specq import _lib

    if not os.path.exists(_lib.LIB_PATH):
        import build  # specdec-quant-triton_amd/build.py

        build.build(quiet=True)
    return _lib.LIB_PATH


@pytest.fixture(autouse=True)
def _row_major_weights_run_row_major_kernels():
    """Tests pass row-major int8 weights to exercise the row-major kernels, so the transparent
    packing of such weights (kernels._WeightPackCache) is off unless a test turns it on."""
    import kernels as K

    K.set_weight_pack_cache(False)
    yield
    K.set_weight_pack_cache(False)
