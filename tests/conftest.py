import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
PKG = os.path.join(ROOT, "ncnn-compiler_amd")
if PKG not in sys.path:
    sys.path.insert(0, PKG)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (HIP device)")


@pytest.fixture
def nhip_env(monkeypatch):
    """monkeypatch for the library's NHIP_* switches.  libnhip reads them
    into a snapshot, so every change (and the restore at teardown) is
    followed by nhip_reload_settings()."""
    import nhip

    class _Env:
        def setenv(self, name, value):
            monkeypatch.setenv(name, value)
            nhip.reload_settings()

        def delenv(self, name, raising=True):
            monkeypatch.delenv(name, raising=raising)
            nhip.reload_settings()

    yield _Env()
    monkeypatch.undo()
    nhip.reload_settings()
