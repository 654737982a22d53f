import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def _has_gpu() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _has_gpu():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def wo():
    """The product module.  On a GPU box a missing extension is an error, not a skip."""
    import wmma_ops_amd
    return wmma_ops_amd


def report(name: str, **kw) -> None:
    """One flushed line per parity case, so a GPU log names the case that ran last."""
    items = " ".join(f"{k}={v}" for k, v in kw.items())
    print(f"[case] {name} {items}", flush=True)
