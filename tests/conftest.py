"""Test configuration: import paths, the ``gpu`` marker, shared helpers."""

import os
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(
    ROOT, "mask-routed-sparse-attention-for-long-context-diffusion-language-models_amd"
)
for p in (PKG_DIR, ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def pytest_collection_modifyitems(config, items):
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(autouse=True)
def _routed_locks_quiet(request):
    """After every GPU test: no routed-attention tile ran out of its bounded
    lock wait (tests that force the bound clear the counter themselves)."""

    yield
    if "gpu" in request.keywords and torch.cuda.is_available():
        import mrsa

        mrsa.check_routed_locks()
