"""Shared test setup: the ``gpu`` marker, repository imports and small helpers."""

from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); run with -m gpu")


def pytest_collection_modifyitems(config, items):
    # Without a device, GPU tests cannot pass; skip them unless they were explicitly selected.
    try:
        import torch

        has_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover
        has_gpu = False
    if has_gpu:
        return
    skip = pytest.mark.skip(reason="no HIP device in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def pe():
    import packed_encoders_amd

    return packed_encoders_amd


def announce(msg: str) -> None:
    """Name the case on stdout before a GPU step, flushed, so a crash still identifies it."""
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()
    os.environ.setdefault("PE_LAST_CASE", msg)
