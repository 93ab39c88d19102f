"""roctx ranges around measured regions, for rocprofv3 ``--marker-trace``.

bench.py brackets each timed region with a range named
``vbh-timed:<workload>:<steps>``; the trace summary
(``viperbench/rocprof_summary.py timed``) keeps exactly the kernel dispatches
that ran inside it.  The markers come from ROCm's rocprofiler-sdk roctx
library, which does nothing unless a profiler is attached; where that library
is absent the ranges are no-ops (nothing here touches the GPU).
"""
from __future__ import annotations

import contextlib
import ctypes
import os
from pathlib import Path

_lib = None
_loaded = False


def _load():
    global _lib, _loaded
    if _loaded:
        return _lib
    _loaded = True
    root = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
    for name in ("librocprofiler-sdk-roctx.so.1", "librocprofiler-sdk-roctx.so"):
        p = root / "lib" / name
        if p.exists():
            try:
                lib = ctypes.CDLL(str(p))
                lib.roctxRangePushA.argtypes = [ctypes.c_char_p]
                lib.roctxRangePushA.restype = ctypes.c_int
                lib.roctxRangePop.argtypes = []
                lib.roctxRangePop.restype = ctypes.c_int
                _lib = lib
            except (OSError, AttributeError):
                _lib = None
            break
    return _lib


def available() -> bool:
    return _load() is not None


@contextlib.contextmanager
def range_(name: str):
    """A roctx push/pop range named `name` (a no-op without the library)."""
    lib = _load()
    if lib is not None:
        lib.roctxRangePushA(name.encode())
    try:
        yield
    finally:
        if lib is not None:
            lib.roctxRangePop()
