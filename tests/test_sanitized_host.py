"""Host code under AddressSanitizer and UndefinedBehaviorSanitizer (CPU tier).

``dslperfgap_amd/sanitize.py`` rebuilds the C ABI's host code (capi.hip's
argument validation, size arithmetic, geometry and workspace sizing; the
launchers; vbhfast.c's argument parser) with ASan + UBSan in a copy of the
repository and runs the C-ABI and unified-API CPU tests there with the
sanitizer runtime preloaded.  The run must pass with no sanitizer report, and
both shared objects must be instrumented.  Takes about two minutes (the
device code of the copy is compiled too).
"""
import shutil

import pytest


def test_cpu_tier_is_clean_under_asan_and_ubsan():
    if shutil.which("hipcc") is None and not __import__("os").path.exists("/opt/rocm/bin/hipcc"):
        pytest.skip("hipcc is not installed")
    try:
        from dslperfgap_amd import sanitize
    except ImportError:
        pytest.skip("the sanitizer build script is not part of this tree")
    res = sanitize.run()
    text = res.stdout + res.stderr
    assert sanitize.clean(res), text[-6000:]
    assert " passed" in res.stdout and "failed" not in res.stdout, res.stdout[-3000:]
