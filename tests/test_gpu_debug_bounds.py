"""The bounds-checked debug build (libvbhip_debug.so, VBH_DEBUG_BOUNDS) on the GPU.

A child process loads the debug library (VBHIP_LIB) and runs the battery of
tests/_bounds_battery.py, which reaches every kernel of the library; every
global-memory access there is checked against the extent of its buffer before
it is made.  The test asserts that no check failed, that the debug build's
outputs are bit-identical to the release library's on the same inputs (the
checks change no arithmetic), and, with 16 bytes of slack taken off every
buffer, that the checks do fire: the last vector of a softmax is then counted,
its load and store skipped (the output keeps its sentinel there), and the
count names softmax.hip.
"""
import os
import subprocess
import sys
from pathlib import Path

import pytest
import torch

from dslperfgap_amd import _lib
from dslperfgap_amd.build import DEBUG_LIB_PATH

sys.path.insert(0, str(Path(__file__).parent))
import _bounds_battery  # noqa: E402

pytestmark = pytest.mark.gpu


def _same(a, b):
    if a.dtype != b.dtype or a.shape != b.shape:
        return False
    if a.is_floating_point():
        return torch.equal(a.isnan(), b.isnan()) and torch.equal(a[~a.isnan()], b[~b.isnan()])
    return torch.equal(a, b)


def test_debug_bounds_build_checks_every_kernel(tmp_path):
    if _lib.LIB_PATH.resolve() == DEBUG_LIB_PATH.resolve():
        pytest.skip("this session runs on the debug library itself (VBH_CHECK_BOUNDS run)")
    print("[gpu] debug bounds: release battery", flush=True)
    assert DEBUG_LIB_PATH.exists(), f"{DEBUG_LIB_PATH} is missing: run the build"
    with pytest.raises(_lib.VbhError) as e:  # the release library has no checks
        _lib.debug_bounds()
    assert e.value.code == _lib.E_UNSUPPORTED
    want = _bounds_battery.run()
    print(f"[gpu] debug bounds: debug battery ({len(want)} outputs) in a child process",
          flush=True)
    out = tmp_path / "debug.pt"
    env = dict(os.environ, VBHIP_LIB=str(DEBUG_LIB_PATH))
    res = subprocess.run([sys.executable, "-u", str(Path(__file__).parent / "_bounds_battery.py"),
                          str(out)], env=env, capture_output=True, text=True, timeout=300)
    print(res.stdout[-2000:], res.stderr[-2000:], flush=True)
    assert res.returncode == 0, res.stderr[-4000:]
    got = torch.load(out, weights_only=True)
    assert got["failed"] == 0, f"{got['failed']} failed bounds checks, first at {got['where']}"
    assert set(got["outs"]) == set(want)
    diff = [k for k in want if not _same(got["outs"][k], want[k])]
    assert not diff, f"debug and release outputs differ: {diff[:5]}"
    probe = got["probe"]
    assert probe["failed"] > 0 and probe["where"].startswith("softmax.hip:"), probe
    assert probe["tail_untouched"] and probe["rest_written"], probe
    assert got["after_failed"] == 0
