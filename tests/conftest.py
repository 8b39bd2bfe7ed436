"""Test setup: import paths, the ``gpu`` marker, shared helpers."""

import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PACKAGE = os.path.join(REPO, "nl2cuda-kernel-agent_amd")
for p in (PACKAGE, REPO):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (runs through the HIP libraries)")


def pytest_collection_modifyitems(config, items):
    import torch
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this process (torch.cuda.is_available() is False)")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def announce(msg):
    """Print (and flush) what the next GPU step is, so a crash names it."""
    print(f"\n[gpu-step] {msg}", flush=True)
