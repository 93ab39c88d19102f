"""Shared pytest setup.

Tests marked ``gpu`` need an MI355X: they are skipped where torch sees no GPU
(this CPU container) and run on the GPU box with ``-m gpu``.  On a machine with
a GPU they call the HIP library and fail loudly if it is missing.
"""
import pytest
import torch


def pytest_collection_modifyitems(config, items):
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible to torch in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
