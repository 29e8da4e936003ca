"""Test configuration: import paths and the `gpu` marker.

`-m "not gpu"` runs on any machine (oracle pinning, host logic, the C ABI
exports); `-m gpu` runs the parity tests on an MI355X through the C ABI.
"""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "msda-triton_amd", ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and libmsda_hip.so")


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture
def overrides():
    """Setter of library launch overrides (``overrides(BWD_OWNER=0)``, knob
    names of msda_triton_amd._native.KNOBS); every knob set is restored to
    the automatic choice when the test ends."""
    from msda_triton_amd import _native

    touched = []

    def setter(**knobs):
        lib = _native.load()
        for name, value in knobs.items():
            code = _native.KNOBS[name]
            touched.append(code)
            _native.check(lib.msda_set_launch_override(code, int(value)),
                          "msda_set_launch_override")

    yield setter
    if touched:
        lib = _native.load()
        for code in touched:
            lib.msda_set_launch_override(code, _native.OVERRIDE_AUTO)
