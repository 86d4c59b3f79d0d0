"""pytest configuration: the `gpu` marker and package import.  The suite
loads the library as built (it is the run that validates it), so it sets
SMX_ALLOW_UNVALIDATED before anything loads libsmx.so."""
import os
import sys
from pathlib import Path

import pytest

os.environ.setdefault("SMX_ALLOW_UNVALIDATED", "1")

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

import __graft_entry__  # noqa: E402

__graft_entry__.load_package()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def pytest_collection_modifyitems(config, items):
    try:
        import torch
        have_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover
        have_gpu = False
    if have_gpu:
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
