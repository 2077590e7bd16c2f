"""ctypes binding of libnia_attn.so, the gfx950 attention library.

The library is built in-tree (``build_lib.py``) and loaded from the package
directory.  There is no fallback: if the library is missing, every attention
call raises, so a GPU run can never silently take another path.

``calls()`` is what the per-layer ops call: the CPython fast-call module
``_nia_fast`` bound to this same library (one library instance, one device
state), which converts the ~23 integer arguments of a call in well under a
microsecond where ctypes takes a few; the ctypes library itself where that
module has not been built.  Both take the arguments of nia_attn.h in order and
return the int status.
"""
from __future__ import annotations

import ctypes as C
import os
import threading
from pathlib import Path

LIB_NAME = "libnia_attn.so"
PKG_DIR = Path(os.path.realpath(__file__)).parent

# Mirrors the #defines of include/nia_attn.h.
DTYPE_BF16 = 0
DTYPE_F32 = 1
CAUSAL_NONE = 0
CAUSAL_TOP_LEFT = 1
CAUSAL_BOTTOM_RIGHT = 2
OK = 0
ERR_INVALID_ARGUMENT = 1
ERR_UNSUPPORTED = 2
ERR_WORKSPACE = 3
ERR_LAUNCH = 4
ERR_MISALIGNED = 5
ERR_SCRATCH_LIMIT = 6
DECODE_SCRATCH_BYTES = 40 << 20  # NIA_DECODE_SCRATCH_BYTES

_p = C.c_void_p
_i32 = C.c_int32
_i64 = C.c_int64
_f32 = C.c_float
_sz = C.c_size_t

# name -> (restype, argtypes); the order of arguments is that of nia_attn.h.
SIGNATURES = {
    "nia_abi_version": (_i32, []),
    "nia_error_string": (C.c_char_p, [_i32]),
    "nia_kv_write": (
        _i32,
        [_p, _i64, _i64, _p, _i64, _i64, _p, _p, _p, _i32, _i32, _i32, _i32, _i64, _i32, _p],
    ),
    "nia_paged_decode_workspace_size": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32, _i32]),
    "nia_paged_decode": (
        _i32,
        [_p, _i64, _i64, _p, _i64, _i64, _p, _p, _p, _i32, _i32, _p,
         _i32, _i32, _i32, _i32, _i32, _i64, _f32, _p, _sz, _i32, _p],
    ),
    "nia_paged_decode_noalloc": (
        _i32,
        [_p, _i64, _i64, _p, _i64, _i64, _p, _p, _p, _i32, _i32, _p,
         _i32, _i32, _i32, _i32, _i32, _i64, _f32, _i32, _p],
    ),
    "nia_paged_decode_fp8": (
        _i32,
        [_p, _i64, _i64, _p, _i64, _i64, _p, _p, _p, _p, _p, _i32, _i32, _p,
         _i32, _i32, _i32, _i32, _i32, _i64, _f32, _p, _sz, _p],
    ),
    "nia_prefill": (
        _i32,
        [_p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64,
         _p, _p, _p, _p, _i32, _i32, _i32, _i32, _i32, _f32, _i32, _i32, _p],
    ),
    "nia_prefill_masked": (
        _i32,
        [_p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64,
         _p, _p, _p, _p, _i32, _i32, _i32, _i32, _i32, _f32, _i32, _i32,
         _p, _i64, _i64, _i64, _p],
    ),
    "nia_prefill_paged": (
        _i32,
        [_p, _i64, _i64, _p, _i64, _i64, _p, _p, _p, _i32, _i32, _p, _p, _p,
         _i32, _i32, _i32, _i32, _i32, _i32, _i64, _f32, _i32, _i32, _p],
    ),
    "nia_qk_norm_rope_kv_write": (
        _i32,
        [_p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _p, _p, _f32, _p, _i64, _i32,
         _p, _i32, _i32, _p, _p, _p, _i32, _i32, _i32, _i32, _i32, _i64, _i32, _p],
    ),
    "nia_kv_write_fp8": (
        _i32,
        [_p, _i64, _i64, _p, _i64, _i64, _p, _p, _p, _p, _p, _i32, _i32, _i32, _i32, _i64,
         _i32, _p],
    ),
    "nia_qk_norm_rope_kv_write_fp8": (
        _i32,
        [_p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _p, _p, _f32, _p, _i64, _i32,
         _p, _i32, _i32, _p, _p, _p, _p, _p, _i32, _i32, _i32, _i32, _i32, _i64, _i32, _p],
    ),
    "nia_dequant_gather_fp8": (
        _i32,
        [_p, _p, _p, _p, _p, _i32, _i32, _p, _i32, _i32, _i32, _i32, _i64, _p, _p, _i64, _p],
    ),
    "nia_step_metadata": (
        _i32,
        [_p, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i32,
         _p, _p, _p, _p, _p, _p, _p, _p, _p],
    ),
    "nia_step_metadata_packed": (
        _i32,
        [_p, _i64, _i64, _p, _i64, _i32, _i64, _i32, _i32, _i32,
         _p, _p, _p, _p, _p, _p, _p, _p, _p],
    ),
}

ABI_VERSION = 3

# The entry points _nia_fast wraps: one call per layer and step.
FAST_CALLS = (
    "nia_kv_write",
    "nia_kv_write_fp8",
    "nia_paged_decode",
    "nia_paged_decode_fp8",
    "nia_prefill",
    "nia_prefill_paged",
    "nia_qk_norm_rope_kv_write",
    "nia_qk_norm_rope_kv_write_fp8",
)

_lock = threading.Lock()
_lib: C.CDLL | None = None
_calls = None
_calls_lib: C.CDLL | None = None


class NiaError(RuntimeError):
    """A nonzero status returned by the attention library."""

    def __init__(self, fn: str, status: int, msg: str):
        super().__init__(f"{fn}: {msg} (status {status})")
        self.status = status


def lib_path() -> Path:
    return PKG_DIR / LIB_NAME


def load() -> C.CDLL:
    """Load (once) and return the library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            path = lib_path()
            if not path.exists():
                raise ImportError(
                    f"{path} is missing: build it with `python {PKG_DIR / 'build_lib.py'}` "
                    "(or __graft_entry__.build()); there is no non-HIP attention path"
                )
            lib = C.CDLL(str(path))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            got = lib.nia_abi_version()
            if got != ABI_VERSION:
                raise ImportError(f"{path}: ABI version {got}, expected {ABI_VERSION}")
            _lib = lib
    return _lib


# Argument kind letters of _nia_fast (p pointer, l int64, i int32, f float, z size_t).
_KIND_LETTER = {_p: "p", _i64: "l", _i32: "i", _f32: "f", _sz: "z"}


def fast_kinds(name: str) -> str:
    """The argument kinds _nia_fast must use for ``name``, from ``SIGNATURES``."""
    return "".join(_KIND_LETTER[a] for a in SIGNATURES[name][1])


def fast_module():
    """The _nia_fast extension module, or None where it has not been built or was built
    for other signatures than ``SIGNATURES`` (a stale build: its calls would pass the
    arguments in the wrong layout, so the ctypes binding is used instead)."""
    try:
        from . import _nia_fast
    except ImportError:
        return None
    kinds = getattr(_nia_fast, "kinds", {})
    if any(kinds.get(name) != fast_kinds(name) for name in FAST_CALLS):
        import warnings
        warnings.warn("_nia_fast does not match the library's signatures (rebuild it with "
                      "build_lib.py); the hot calls go through ctypes", RuntimeWarning)
        return None
    return _nia_fast


def calls():
    """The hot entry points (``FAST_CALLS``): _nia_fast bound to the loaded library, or
    the ctypes library where _nia_fast is absent.  Loads the library like ``load()``."""
    global _calls, _calls_lib
    lib = load()
    if _calls is not None and _calls_lib is lib:
        return _calls
    with _lock:
        if _calls is None or _calls_lib is not lib:
            fast = fast_module()
            if fast is not None:
                for name in FAST_CALLS:
                    fast.bind(name, C.cast(getattr(lib, name), C.c_void_p).value)
            _calls, _calls_lib = (fast if fast is not None else lib), lib
    return _calls


def check(fn: str, status: int) -> None:
    if status != OK:
        msg = load().nia_error_string(status).decode()
        raise NiaError(fn, status, msg)
