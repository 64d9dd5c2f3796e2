"""Test configuration: import paths, the `gpu` marker, shared helpers."""

import json
import os
import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
for p in (ROOT / "turboquant-amd_amd", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

import torch  # noqa: E402  (after the path setup; loads the HIP runtime before our library)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and the built HIP library")


def pytest_collection_modifyitems(config, items):
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def dev():
    return torch.device("cuda:0")


# Compress parity counts (index mismatches by distance from the boundary) recorded by the GPU
# tests; written as JSON to $TQ_PARITY_OUT at the end of the session when that is set.
_PARITY: dict = {}


@pytest.fixture(scope="session")
def parity_log():
    return _PARITY


def pytest_sessionfinish(session, exitstatus):
    path = os.environ.get("TQ_PARITY_OUT")
    if path and _PARITY:
        pathlib.Path(path).parent.mkdir(parents=True, exist_ok=True)
        pathlib.Path(path).write_text(json.dumps(_PARITY, indent=1, sort_keys=True))
