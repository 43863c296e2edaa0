import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_ROOT = os.path.join(REPO, "vllm-grinqh-plugin_amd")
for p in (REPO, PKG_ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)

# Without a vLLM install the plugin's layer classes come from the minimal
# stand-in under tests/vllm_shim; it goes on the path once, here, so that every
# test module sees the same vLLM (real or stand-in) whatever the collection order.
VLLM_SHIM = os.path.join(REPO, "tests", "vllm_shim")
try:
    import vllm  # noqa: F401
except ImportError:
    sys.path.insert(0, VLLM_SHIM)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(autouse=True)
def _seed():
    import numpy as np
    np.random.seed(0)
    try:
        import torch
        torch.manual_seed(0)
    except ImportError:  # pragma: no cover
        pass
