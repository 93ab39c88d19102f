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


def pytest_sessionfinish(session, exitstatus):
    """With VBH_CHECK_BOUNDS=1 and VBHIP_LIB naming the bounds-checked library
    (libvbhip_debug.so), the session fails if any access of any kernel in any
    test failed its bounds check (the debug build counts them)."""
    import os

    if os.environ.get("VBH_CHECK_BOUNDS") != "1" or not torch.cuda.is_available():
        return
    from dslperfgap_amd import _lib

    failed, where = _lib.debug_bounds(clear=True)
    print(f"\n[bounds] {failed} failed bounds checks in this session"
          + (f", the first at {where}" if failed else ""), flush=True)
    if failed:
        session.exitstatus = 1
