"""Build libvbhip.so (the gfx950 HIP kernels + C ABI) in-tree.

Every ``csrc/*.hip`` file is compiled with hipcc for gfx950 only, in parallel,
into ``_build/``, then linked into ``dslperfgap_amd/libvbhip.so``.  The CPython
binding of its launching entry points (``csrc/vbhfast.c``) is then compiled
with the host C compiler into ``dslperfgap_amd/_vbhfast*.so``, linked against
that library.  Both are rebuilt on every call (the caller asked for a build).

The same sources are also compiled with ``-DVBH_DEBUG_BOUNDS`` into
``_build/debug/`` and linked into ``libvbhip_debug.so``: the bounds-checked
debug build, in which every kernel checks each global-memory access against
the extent of its buffer before making it (``vbh_debug_bounds`` reads the
count of failed checks; ``VBHIP_LIB`` selects that library for a run).  Its
release counterpart is the same code with every check compiled away.

Provenance: the build writes ``libvbhip.srchash`` (and
``libvbhip_debug.srchash``) next to the libraries, the SHA-256 of every file
under ``csrc/`` and ``include/`` (names and contents) they were built from.
``_lib.lib()`` refuses a library whose hash differs from the sources on disk,
so a stale binary cannot run in place of the code in the tree.

Usage: ``python -m dslperfgap_amd.build [--no-debug]`` or ``build()`` from
Python.
"""
from __future__ import annotations

import hashlib
import os
import shutil
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
BUILD_DIR = PKG_DIR / "_build"
LIB_PATH = PKG_DIR / "libvbhip.so"
HASH_PATH = PKG_DIR / "libvbhip.srchash"
DEBUG_LIB_PATH = PKG_DIR / "libvbhip_debug.so"
DEBUG_HASH_PATH = PKG_DIR / "libvbhip_debug.srchash"
FAST_PATH = PKG_DIR / ("_vbhfast" + sysconfig.get_config_var("EXT_SUFFIX"))
REPO_ROOT = PKG_DIR.parent

ARCH = "gfx950"

# Packed fp32 VALU forms are kept out of the generated code (the compiler
# otherwise emits v_pk_fma_f32 / v_pk_mul_f32 / v_pk_add_f32 from plain float code).
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{REPO_ROOT / 'include'}",
]


def source_hash(pkg_dir: Path = PKG_DIR, include_dir: Path | None = None) -> str:
    """SHA-256 over the relative path and content of every file under the
    package's ``csrc/`` and the repository's ``include/``, in sorted order."""
    include_dir = include_dir or pkg_dir.parent / "include"
    h = hashlib.sha256()
    for base, tag in ((pkg_dir / "csrc", "csrc"), (include_dir, "include")):
        for f in sorted(p for p in base.rglob("*") if p.is_file()):
            h.update(f"{tag}/{f.relative_to(base).as_posix()}\0".encode())
            h.update(f.read_bytes())
            h.update(b"\0")
    return h.hexdigest()


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: install ROCm or set HIPCC")


def _compile(hipcc: str, src: Path, debug: bool = False) -> Path:
    out_dir = BUILD_DIR / "debug" if debug else BUILD_DIR
    obj = out_dir / (src.stem + ".o")
    cmd = [hipcc, *DEVICE_FLAGS, *(["-DVBH_DEBUG_BOUNDS"] if debug else []), "-c", str(src),
           "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stdout}\n{res.stderr}")
    # keep real diagnostics visible; drop the host-pass notice about the device-only feature
    noise = "is not a recognized feature for this target"
    msgs = [l for l in (res.stdout + res.stderr).splitlines() if l.strip() and noise not in l]
    if msgs:
        print("\n".join(msgs), file=sys.stderr)
    return obj


def _link(hipcc: str, objs: list, lib_path: Path) -> None:
    tmp = lib_path.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link of {lib_path.name} failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, lib_path)


def build(verbose: bool = True, debug: bool = True) -> Path:
    """Compile every HIP source for gfx950 and link libvbhip.so (and, with
    `debug`, the bounds-checked libvbhip_debug.so); return the release path."""
    hipcc = _hipcc()
    digest = source_hash()
    flavors = [(False, LIB_PATH, HASH_PATH)] + ([(True, DEBUG_LIB_PATH, DEBUG_HASH_PATH)]
                                                if debug else [])
    for _, _, hash_path in flavors:  # no hash while a library is being replaced
        hash_path.unlink(missing_ok=True)
    BUILD_DIR.mkdir(exist_ok=True)
    (BUILD_DIR / "debug").mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    units = [(src, dbg) for dbg, _, _ in flavors for src in sources]
    jobs = min(len(units), max(1, min(16, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(lambda u: _compile(hipcc, *u), units))
    for i, (_, lib_path, _) in enumerate(flavors):
        _link(hipcc, objs[i * len(sources):(i + 1) * len(sources)], lib_path)
    build_fast()
    for _, _, hash_path in flavors:
        hash_path.write_text(digest + "\n")
    if verbose:
        names = ", ".join(lib.name for _, lib, _ in flavors)
        print(f"built {names} from {len(sources)} sources each, and {FAST_PATH.name}",
              file=sys.stderr)
    return LIB_PATH


def build_fast() -> Path:
    """Compile the CPython binding (csrc/vbhfast.c).  It does not link the
    library: _lib binds it to the entry points of the instance it loads."""
    cc = os.environ.get("CC") or shutil.which("gcc") or shutil.which("cc")
    if not cc:
        raise RuntimeError("no host C compiler (gcc) found for the CPython binding")
    tmp = FAST_PATH.with_suffix(".so.tmp")
    cmd = [cc, "-O2", "-shared", "-fPIC", "-Wall", "-Werror",
           f"-I{sysconfig.get_paths()['include']}", f"-I{REPO_ROOT / 'include'}",
           str(CSRC / "vbhfast.c"), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"building {FAST_PATH.name} failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, FAST_PATH)
    return FAST_PATH


if __name__ == "__main__":
    build(debug="--no-debug" not in sys.argv[1:])
