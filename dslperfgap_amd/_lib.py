"""Bindings of libvbhip.so (declarations in include/vbhip.h).

The library is loaded after ``import torch`` so that it binds to the HIP
runtime torch already holds (both carry the soname libamdhip64.so.7), which
makes torch's stream handles valid for the library's launches.

Two bindings of the same C ABI: ctypes (every entry point; also checks the ABI
version and the exported symbols), and the CPython module ``_vbhfast`` built
from csrc/vbhfast.c, whose METH_FASTCALL functions the launching entry points
go through because its argument conversion costs about 0.1 us per call
against ctypes' 0.7 us.  ``_vbhfast`` does not link the library: it is bound
to the entry-point addresses of the instance ctypes loaded, so launches, the
tuning hook and the error message all reach one instance, whichever file
``VBHIP_LIB`` names.

There is no non-HIP fallback: if the library or the binding module is
missing, :func:`lib` raises ``ImportError`` naming the build command.  So does
a library built from other sources than the ones on disk: the build records
the SHA-256 of ``csrc/`` and ``include/`` in ``libvbhip.srchash`` next to the
library, and :func:`lib` compares it with the tree before loading.
"""
from __future__ import annotations

import ctypes
import functools
import os
import threading
from pathlib import Path

import torch  # noqa: F401  (loads the HIP runtime the library must share)

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("VBHIP_LIB", PKG_DIR / "libvbhip.so"))

ABI_VERSION = 1

# element type codes (VBH_DTYPE_*)
F32, F16, BF16, I32, I64 = 0, 1, 2, 3, 4
# argument-error codes (VBH_E_*)
E_INVALID, E_DTYPE, E_RANGE, E_UNSUPPORTED = -1, -2, -3, -4
# op codes for vbh_tune_override (VBH_OP_*)
OP_LAYER_NORM, OP_RMS_NORM, OP_SOFTMAX, OP_LOGSUMEXP, OP_CROSS_ENTROPY, OP_REDUCE = 0, 1, 2, 3, 4, 5
# reduction codes (VBH_REDUCE_*)
REDUCE_MEAN, REDUCE_MAX, REDUCE_ARGMAX = 0, 1, 2

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float

# name -> (restype, argtypes); kept in the order of include/vbhip.h
SIGNATURES = {
    "vbh_abi_version": (_i32, []),
    "vbh_last_error": (ctypes.c_char_p, []),
    "vbh_layer_norm_fwd": (_i32, [_vp, _vp, _vp, _vp, _i64, _i64, _f32, _i32, _i32, _vp]),
    "vbh_rms_norm_fwd": (_i32, [_vp, _vp, _vp, _i64, _i64, _f32, _i32, _i32, _vp]),
    "vbh_softmax_fwd": (_i32, [_vp, _vp, _i64, _i64, _i32, _i32, _i32, _vp]),
    "vbh_softmax_fwd_ws": (_i32, [_vp, _vp, _i64, _i64, _i32, _i32, _i32, _vp, _i64, _vp]),
    "vbh_softmax_workspace_bytes": (_i64, [_i64, _i64, _i32]),
    "vbh_softmax_dim_fwd": (_i32, [_vp, _vp, _i64, _i64, _i64, _i32, _i32, _i32, _vp]),
    "vbh_logsumexp_fwd": (_i32, [_vp, _vp, _i64, _i64, _i32, _i32, _vp]),
    "vbh_logsumexp_fwd_ws": (_i32, [_vp, _vp, _i64, _i64, _i32, _i32, _vp, _i64, _vp]),
    "vbh_logsumexp_workspace_bytes": (_i64, [_i64, _i64, _i32]),
    "vbh_cross_entropy_fwd": (
        _i32,
        [_vp, _vp, _i32, _i32, _vp, _vp, _vp, _i64, _i64, _i64, _f32, _f32, _f32, _i64, _i64,
         _i64, _i64, _i32, _i32, _vp],
    ),
    "vbh_cross_entropy_fwd_ws": (
        _i32,
        [_vp, _vp, _i32, _i32, _vp, _vp, _vp, _i64, _i64, _i64, _f32, _f32, _f32, _i64, _i64,
         _i64, _i64, _i32, _i32, _vp, _i64, _vp],
    ),
    "vbh_cross_entropy_workspace_bytes": (_i64, [_i64, _i64, _i64, _i32]),
    "vbh_cross_entropy_fwd_noalloc": (
        _i32,
        [_vp, _vp, _i32, _i32, _vp, _vp, _vp, _i64, _i64, _i64, _f32, _f32, _f32, _i64, _i64,
         _i64, _i64, _i32, _i32, _vp],
    ),
    "vbh_cross_entropy_bwd": (
        _i32,
        [_vp, _vp, _vp, _vp, _vp, _i32, _i32, _i64, _i64, _i64, _i64, _i64, _f32, _f32, _f32,
         _i64, _i64, _i64, _i32, _vp],
    ),
    "vbh_reduce_fwd": (_i32, [_vp, _vp, _vp, _i64, _i64, _i64, _i32, _i32, _i32, _vp]),
    "vbh_reduce_fwd_ws": (_i32, [_vp, _vp, _vp, _i64, _i64, _i64, _i32, _i32, _i32, _vp, _i64,
                                 _vp]),
    "vbh_reduce_workspace_bytes": (_i64, [_i64, _i64, _i64, _i32, _i32]),
    "vbh_stream_copy": (_i32, [_vp, _vp, _i64, _vp]),
    "vbh_stream_read": (_i32, [_vp, _i64, _vp, _i64, _vp]),
    "vbh_stream_read_partial_bytes": (_i64, [_i64]),
    "vbh_tune_override": (_i32, [_i32, _i32, _i32, _i32]),
    "vbh_debug_bounds": (_i32, [ctypes.POINTER(ctypes.c_int64), ctypes.c_char_p, _i64, _i32]),
    "vbh_debug_bounds_slack": (_i32, [_i64]),
}


# entry points _vbhfast binds (every launching one)
FAST_ENTRY_POINTS = (
    "vbh_layer_norm_fwd", "vbh_rms_norm_fwd", "vbh_softmax_fwd", "vbh_softmax_fwd_ws",
    "vbh_softmax_dim_fwd",
    "vbh_logsumexp_fwd", "vbh_logsumexp_fwd_ws", "vbh_cross_entropy_fwd",
    "vbh_cross_entropy_fwd_ws", "vbh_cross_entropy_fwd_noalloc", "vbh_cross_entropy_bwd",
    "vbh_reduce_fwd", "vbh_reduce_fwd_ws", "vbh_stream_copy", "vbh_stream_read",
)


class VbhError(RuntimeError):
    """A nonzero status from libvbhip (argument error < 0, hipError_t > 0)."""

    def __init__(self, fn: str, code: int, message: str):
        super().__init__(f"{fn} failed with status {code}: {message}")
        self.code = code


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None
_fns: dict = {}


def check_provenance(lib_path: Path = None) -> None:
    """Raise ImportError unless the hash recorded next to the library equals
    the hash of the sources in this tree (the library is what they build)."""
    from .build import source_hash

    lib_path = Path(lib_path or LIB_PATH)
    hash_path = lib_path.with_suffix(".srchash")
    if not hash_path.exists():
        raise ImportError(f"{hash_path} is missing, so {lib_path.name} cannot be tied to the "
                          "sources: rebuild with `python -m dslperfgap_amd.build`")
    recorded = hash_path.read_text().strip()
    current = source_hash(PKG_DIR)
    if recorded != current:
        raise ImportError(f"{lib_path.name} was built from other sources than the ones in "
                          f"{PKG_DIR / 'csrc'} and include/ (hash {recorded[:12]} vs "
                          f"{current[:12]}): rebuild with `python -m dslperfgap_amd.build`")


def lib() -> ctypes.CDLL:
    """Load (once) and return the bound library."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise ImportError(
                    f"{LIB_PATH} is missing: build it with `python -m dslperfgap_amd.build` "
                    "(there is no non-HIP fallback)")
            check_provenance(LIB_PATH)
            handle = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            version = handle.vbh_abi_version()
            if version != ABI_VERSION:
                raise ImportError(f"{LIB_PATH} has ABI {version}, expected {ABI_VERSION}")
            try:
                from . import _vbhfast
            except ImportError as e:
                raise ImportError(f"the CPython binding of {LIB_PATH.name} is missing or stale "
                                  f"({e}): build it with `python -m dslperfgap_amd.build`") from e
            if _vbhfast.ABI_VERSION != ABI_VERSION:
                raise ImportError(f"_vbhfast has ABI {_vbhfast.ABI_VERSION}, expected {ABI_VERSION}")
            _vbhfast.bind({name: ctypes.cast(getattr(handle, name), ctypes.c_void_p).value
                           for name in FAST_ENTRY_POINTS})
            _fns.update({name: getattr(handle, name) for name in SIGNATURES})
            # launching entry points through the fast binding
            _fns.update({name: getattr(_vbhfast, name) for name in FAST_ENTRY_POINTS})
            _lib = handle
    return _lib


def last_error() -> str:
    msg = lib().vbh_last_error()
    return msg.decode() if msg else ""


def entry(name: str):
    """The bound function of entry point `name` (loads the library on first use).
    It returns the entry point's status; :func:`call` raises on a nonzero one."""
    if _lib is None:
        lib()
    return _fns[name]


def call(name: str, *args) -> None:
    """Call entry point `name`; raise VbhError on a nonzero status."""
    if _lib is None:
        lib()
    rc = _fns[name](*args)
    if rc != 0:
        raise VbhError(name, rc, last_error())


# vbh_tune_override flag bits (VBH_TUNE_*)
TUNE_PERSIST, TUNE_NO_PERSIST, TUNE_NONTEMPORAL, TUNE_TEMPORAL = 1, 2, 4, 8
TUNE_WRITE_THROUGH, TUNE_NO_WRITE_THROUGH = 16, 32


# caches of host-side plans that depend on the geometry (and so on
# vbh_tune_override); modules that keep one append its lru_cache here
GEOMETRY_CACHES: list = []


def tune_override(op: int, tpr: int = 0, block: int = 0, flags: int = 0) -> None:
    """Force threads-per-row / workgroup size / kernel flags for one op
    (all zero restores the built-in heuristic)."""
    call("vbh_tune_override", op, tpr, block, flags)
    # an overridden geometry turns the row split off (and back on when cleared)
    logsumexp_workspace_bytes.cache_clear()
    softmax_workspace_bytes.cache_clear()
    reduce_workspace_bytes.cache_clear()
    cross_entropy_workspace_bytes.cache_clear()
    for cache in GEOMETRY_CACHES:
        cache.cache_clear()


def debug_bounds(clear: bool = True) -> tuple:
    """(failed checks, "<file>:<line>" of the first failing buffer or "") of the
    bounds-checked debug library (libvbhip_debug.so, selected with VBHIP_LIB);
    waits for the device.  The release library raises VbhError
    (VBH_E_UNSUPPORTED)."""
    n = ctypes.c_int64(0)
    where = ctypes.create_string_buffer(256)
    call("vbh_debug_bounds", ctypes.byref(n), where, len(where), int(clear))
    return n.value, where.value.decode()


def debug_bounds_slack(nbytes: int) -> None:
    """Take `nbytes` off the end of every buffer's allowed extent in the
    bounds-checked library (0 restores)."""
    call("vbh_debug_bounds_slack", int(nbytes))


@functools.lru_cache(maxsize=4096)
def logsumexp_workspace_bytes(rows: int, cols: int, in_dtype: int) -> int:
    """Workspace bytes that split a logsumexp launch (0: no split)."""
    return lib().vbh_logsumexp_workspace_bytes(rows, cols, in_dtype)


@functools.lru_cache(maxsize=4096)
def softmax_workspace_bytes(rows: int, cols: int, in_dtype: int) -> int:
    """Workspace bytes that split a softmax / log_softmax launch (0: no split)."""
    return lib().vbh_softmax_workspace_bytes(rows, cols, in_dtype)


@functools.lru_cache(maxsize=4096)
def cross_entropy_workspace_bytes(n_rows: int, n_cols: int, block_size: int,
                                  logits_dtype: int) -> int:
    """Workspace bytes that split a cross-entropy forward launch (0: no split)."""
    return lib().vbh_cross_entropy_workspace_bytes(n_rows, n_cols, block_size, logits_dtype)


@functools.lru_cache(maxsize=4096)
def reduce_workspace_bytes(outer: int, n: int, inner: int, in_dtype: int, op: int) -> int:
    """Workspace bytes that split a mean / max / argmax launch (0: no split)."""
    return lib().vbh_reduce_workspace_bytes(outer, n, inner, in_dtype, op)
