import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "mini-inference_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built libmiq.so")


def pytest_collection_modifyitems(config, items):
    import torch
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture
def miq_env(monkeypatch):
    """Set MIQ_* kernel-selection variables for one test: libmiq reads them once at load,
    so the library re-reads them after every change and again after the test."""
    def reload():
        from kernels import _lib
        _lib.load().miq_tuning_reload()

    def setenv(name, value):
        monkeypatch.setenv(name, value)
        reload()

    yield setenv
    monkeypatch.undo()
    reload()


@pytest.fixture(autouse=True)
def _no_device_errors(request):
    """After every GPU test: no kernel may have set a bit of libmiq's device error word
    (a bounded wait that gave up and wrote NaN instead of a result)."""
    yield
    if "gpu" in request.keywords:
        import torch
        if torch.cuda.is_available():
            from kernels import _lib
            _lib.check_device_errors()
