"""Host-side AddressSanitizer + UndefinedBehaviorSanitizer run (CPU only).

The C ABI's host code -- argument validation, size arithmetic, launch-geometry
selection and workspace sizing in ``csrc/capi.hip``, the launchers, and the
CPython argument parser ``csrc/vbhfast.c`` -- is rebuilt with AddressSanitizer
and UndefinedBehaviorSanitizer in a copy of the repository (the release library
and the bounds-checked libvbhip_debug.so alike), and the CPU test
tier of the C ABI and the unified API runs against it with the sanitizer
runtime preloaded.  Device code is built exactly as for the product (the GPU
sanitizer is not used: only host code is instrumented, through ``-Xarch_host``
on every hipcc line).  Any sanitizer report fails the run.

    python -m dslperfgap_amd.sanitize [--keep DIR] [pytest selection ...]

Nothing here runs on a GPU: the tests it selects are the ``not gpu`` tier,
whose calls stop at argument validation or at the HIP runtime's "no device"
status.
"""
from __future__ import annotations

import argparse
import glob
import os
import shutil
import subprocess
import sys
import sysconfig
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

from . import build as b

ROOT = b.REPO_ROOT
DEFAULT_TESTS = ["tests/test_lib_abi.py", "tests/test_hip_impl_api.py"]
REPORT_MARKERS = ("ERROR: AddressSanitizer", "runtime error:", "ERROR: LeakSanitizer",
                  "SUMMARY: UndefinedBehaviorSanitizer")

# host-only instrumentation for hipcc lines: each flag behind its own -Xarch_host
HOST_SAN = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
            "-Xarch_host", "-fno-sanitize-recover=undefined", "-Xarch_host",
            "-fno-omit-frame-pointer", "-Xarch_host", "-g"]


def asan_runtime() -> str:
    pats = ["/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so",
            "/opt/rocm/llvm/lib/clang/*/lib/x86_64-unknown-linux-gnu/libclang_rt.asan.so"]
    for p in pats:
        hits = sorted(glob.glob(p))
        if hits:
            return hits[-1]
    raise RuntimeError("clang's AddressSanitizer runtime was not found under /opt/rocm/llvm")


def copy_tree(dst: Path) -> Path:
    """The package sources, include/, oracle/, tests/ and pytest.ini, without
    any built file."""
    skip = shutil.ignore_patterns("_build", "__pycache__", "*.so", "*.srchash", "results")
    shutil.copytree(ROOT / "dslperfgap_amd", dst / "dslperfgap_amd", ignore=skip)
    for d in ("include", "oracle", "tests"):
        shutil.copytree(ROOT / d, dst / d, ignore=shutil.ignore_patterns("__pycache__"))
    shutil.copy(ROOT / "pytest.ini", dst / "pytest.ini")
    return dst


LIBS = ((False, "libvbhip.so"), (True, "libvbhip_debug.so"))


def build_sanitized(tree: Path) -> None:
    pkg = tree / "dslperfgap_amd"
    obj_dir = pkg / "_build"
    (obj_dir / "debug").mkdir(parents=True, exist_ok=True)
    hipcc = b._hipcc()
    flags = [f if not f.startswith("-I") else f"-I{tree / 'include'}" for f in b.DEVICE_FLAGS]

    def compile_one(unit) -> Path:
        src, debug = unit
        obj = (obj_dir / "debug" if debug else obj_dir) / (src.stem + ".o")
        cmd = [hipcc, *flags, *HOST_SAN, *(["-DVBH_DEBUG_BOUNDS"] if debug else []), "-c",
               str(src), "-o", str(obj)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc (sanitized) failed for {src.name}:\n{res.stderr[-4000:]}")
        return obj

    sources = sorted((pkg / "csrc").glob("*.hip"))
    units = [(src, debug) for debug, _ in LIBS for src in sources]
    with ThreadPoolExecutor(max_workers=min(len(units), os.cpu_count() or 1)) as pool:
        objs = list(pool.map(compile_one, units))
    for i, (_, name) in enumerate(LIBS):
        cmd = [hipcc, f"--offload-arch={b.ARCH}", "-shared", "-fPIC", *HOST_SAN,
               "-Xarch_host", "-shared-libsan", "-o", str(pkg / name),
               *map(str, objs[i * len(sources):(i + 1) * len(sources)])]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"sanitized link of {name} failed:\n{res.stderr[-4000:]}")
    clang = "/opt/rocm/llvm/bin/clang"
    fast = pkg / ("_vbhfast" + sysconfig.get_config_var("EXT_SUFFIX"))
    cmd = [clang, "-O1", "-g", "-shared", "-fPIC", "-Wall", "-Werror", "-fno-omit-frame-pointer",
           "-fsanitize=address", "-fsanitize=undefined", "-fno-sanitize-recover=undefined",
           "-shared-libsan", f"-I{sysconfig.get_paths()['include']}", f"-I{tree / 'include'}",
           str(pkg / "csrc" / "vbhfast.c"), "-o", str(fast)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"sanitized _vbhfast build failed:\n{res.stderr[-4000:]}")
    digest = b.source_hash(pkg, tree / "include") + "\n"
    for _, name in LIBS:
        (pkg / name).with_suffix(".srchash").write_text(digest)


def instrumented(path: Path) -> bool:
    """Whether a shared object references the AddressSanitizer runtime."""
    out = subprocess.run(["nm", "-D", "--undefined-only", str(path)], capture_output=True,
                         text=True).stdout
    return "__asan_report" in out or "__asan_init" in out


def run(tests=None, keep: str | None = None) -> subprocess.CompletedProcess:
    """Build the sanitized copy and run `tests` in it; returns the pytest run
    (its stdout and stderr hold any sanitizer report)."""
    tmp = Path(keep) if keep else Path(tempfile.mkdtemp(prefix="vbh_san_"))
    try:
        tree = copy_tree(tmp / "repo")
        build_sanitized(tree)
        pkg = tree / "dslperfgap_amd"
        for so in [*(pkg / name for _, name in LIBS), *pkg.glob("_vbhfast*.so")]:
            if not instrumented(so):
                raise RuntimeError(f"{so.name} is not instrumented")
        env = {k: v for k, v in os.environ.items() if k not in ("VBHIP_LIB", "PYTHONPATH")}
        env.update(LD_PRELOAD=asan_runtime(),
                   ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=0",
                   UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
        cmd = [sys.executable, "-m", "pytest", "-q", "-m", "not gpu", "-p", "no:cacheprovider",
               *(tests or DEFAULT_TESTS)]
        return subprocess.run(cmd, cwd=tree, env=env, capture_output=True, text=True,
                              timeout=900)
    finally:
        if not keep:
            shutil.rmtree(tmp, ignore_errors=True)


def clean(res: subprocess.CompletedProcess) -> bool:
    text = res.stdout + res.stderr
    return res.returncode == 0 and not any(m in text for m in REPORT_MARKERS)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--keep", help="build in this directory and keep it")
    ap.add_argument("tests", nargs="*", help=f"pytest selection (default {DEFAULT_TESTS})")
    args = ap.parse_args(argv)
    res = run(args.tests or None, args.keep)
    sys.stdout.write(res.stdout[-6000:])
    sys.stderr.write(res.stderr[-6000:])
    ok = clean(res)
    print(f"sanitized host run: {'clean' if ok else 'FAILED'} (pytest rc {res.returncode})")
    return 0 if ok else 1


if __name__ == "__main__":
    sys.exit(main())
