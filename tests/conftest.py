import os
import sys

import pytest
# torch's HIP runtime must be loaded before libfusedtok_amd.so (which binds to
# it by soname) in every test process, whichever test module loads first
import torch  # noqa: F401

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs an AMD GPU (HIP device) - parity tests proper")


def _gpu_present():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:  # pragma: no cover
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_present():
        return
    skip = pytest.mark.skip(reason="no HIP device in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture
def tuning():
    """Set the library's FT_* tuning switches for one test through the
    binding (ft_set_tuning); every switch set is restored afterwards.
    ``tuning(name, value)`` sets, ``tuning.clear(name)`` restores one now."""
    import fusedtok_amd as ft
    touched = set()

    def set_switch(name, value):
        ft._fusedtok.set_tuning(name, int(value))
        touched.add(name)

    set_switch.clear = ft._fusedtok.clear_tuning
    yield set_switch
    for name in touched:
        ft._fusedtok.clear_tuning(name)
