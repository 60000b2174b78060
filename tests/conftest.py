import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "torch-vulkan_amd")
for p in (REPO, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels through the hrt C ABI)")


@pytest.fixture(autouse=True)
def _reset_vk_counters(request):
    """GPU tests start with empty kernel/fallback counters (reference tests/test_mm.py:20-23)."""
    if request.node.get_closest_marker("gpu") is not None:
        import torch_vulkan

        torch_vulkan.reset_fallback_counts()
    yield
