import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda", 0)


@pytest.fixture
def tuning():
    """``set(name, value)`` for the library's FLASHMAP_* tuning overrides within one test.
    The library reads them once per process, so every change is followed by
    fm_tuning_reload(); the previous values are restored, and re-read, at the end."""
    import os

    from flashmap_amd import _native

    saved = {}

    def set_(name: str, value) -> None:
        if name not in saved:
            saved[name] = os.environ.get(name)
        os.environ[name] = str(value)
        _native.call("fm_tuning_reload")

    yield set_
    for name, old in saved.items():
        if old is None:
            os.environ.pop(name, None)
        else:
            os.environ[name] = old
    if saved:
        _native.call("fm_tuning_reload")
