"""pytest configuration: the `gpu` marker, import paths and the shared GPU context."""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("not-cute-zig_amd", "oracle", "tests"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs through the C ABI")


@pytest.fixture(scope="session")
def gpu():
    """Initialise device 0 and load the embedded gfx950 code object once per session."""
    import notcute_flash as nc

    nc.load_library()
    if nc.device_count() == 0:
        pytest.skip("no GPU visible")
    nc.init()
    mod = nc.Module.load_embedded()
    yield mod
    mod.unload()
