"""ctypes binding of ``libternel_tq1.so`` (the C ABI declared in include/ternel_tq1.h).

The library is the only compute path: if it is missing, every op raises
:class:`NativeLibraryMissing` -- there is no CPU fallback.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import os

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libternel_tq1.so"


def library_path() -> Path:
    """The engine library, or the build of the same C ABI that
    ``TERNEL_TQ1_LIBRARY`` names when the library is first loaded (the
    phase-profile variant, for bench.py --phase-profile)."""
    return Path(os.environ.get("TERNEL_TQ1_LIBRARY") or LIB_PATH)

TERNEL_TQ1_OK = 0
TERNEL_TQ1_EINVAL = -1
TERNEL_TQ1_EHIP = -2

DTYPE_F16 = 0
DTYPE_BF16 = 1
DTYPE_F32 = 2

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_size = ctypes.c_size_t

# name -> (restype, argtypes); exactly the functions include/ternel_tq1.h declares.
SIGNATURES = {
    "ternel_tq1_last_error": (ctypes.c_char_p, []),
    "ternel_tq1_version": (ctypes.c_char_p, []),
    "ternel_tq1_packed_words": (_i64, [_i64, _i64]),
    "ternel_tq1_validate": (_int, [_p, _i64, _p, _p]),
    "ternel_tq1_decode": (_int, [_p, _i64, _p, _p, _p]),
    "ternel_tq1_from_q2": (_int, [_p, _i64, _p, _p, _p]),
    "ternel_tq1_interleave": (_int, [_p, _i64, _i64, _p, _p]),
    "ternel_tq1_deinterleave": (_int, [_p, _i64, _i64, _p, _p]),
    "ternel_tq1_words_from_tiled": (_int, [_p, _p, _i64, _i64, _i64, _p, _p, _p]),
    "ternel_tq1_tiled_from_words": (_int, [_p, _i64, _i64, _i64, _p, _p, _p]),
    "ternel_tq1_matmul": (_int, [_p, _p, _p, _i64, _i64, _i64, _int, _int, _int, _p, _size, _p]),
    "ternel_tq1_matmul_workspace_bytes": (_size, [_i64, _i64, _i64, _int, _int]),
    "ternel_tq1_matmul_noalloc": (_int, [_p, _p, _p, _i64, _i64, _i64, _int, _int, _int, _p]),
    "ternel_tq1_gemm": (_int, [_p, _p, _p, _i64, _i64, _i64, _int, _int, _int, _p, _size, _p]),
    "ternel_tq1_gemm_workspace_bytes": (_size, [_i64, _i64, _i64, _int, _int]),
    "ternel_tq1_get_rows": (_int, [_p, _i64, _i64, _p, _i64, _p, _int, _p]),
    "ternel_tq1_get_rows_canonical": (_int, [_p, _i64, _i64, _p, _i64, _p, _int, _p]),
    "ternel_tq1_linear_kernel": (_int, [_i64, _i64, _i64, _int]),
    "ternel_tq1_swiglu": (_int, [_p, _p, _p, _i64, _i64, _i64, _int, _p, _size, _p]),
    "ternel_tq1_swiglu_workspace_bytes": (_size, [_i64, _i64, _i64, _int]),
    "ternel_tq1_linear": (_int, [_p, _p, _p, _i64, _i64, _i64, _int, _p, _size, _p]),
    "ternel_tq1_linear_workspace_bytes": (_size, [_i64, _i64, _i64, _int]),
    "ternel_tq1_workspace_error": (_int, [_p, _size, _p, _p]),
    "ternel_tq1_set_spin_limit": (_int, [_int]),
}


class NativeLibraryMissing(RuntimeError):
    """The gfx950 library has not been built; run ``python -m ternel_amd.build``."""


class NativeError(RuntimeError):
    """A HIP call inside the library failed."""


_LIB: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        path = library_path()
        if not path.exists():
            raise NativeLibraryMissing(
                f"{path} is missing; build it with `python -m ternel_amd.build` "
                "(the TQ1 engine has no CPU fallback)"
            )
        handle = ctypes.CDLL(str(path))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _LIB = handle
    return _LIB


def last_error() -> str:
    return lib().ternel_tq1_last_error().decode("utf-8", "replace")


def check(rc: int) -> None:
    """Turn a nonzero status into the reference's exception types."""
    if rc == TERNEL_TQ1_OK:
        return
    message = last_error()
    if rc == TERNEL_TQ1_EINVAL:
        from .format import FormatError

        raise FormatError(message)
    raise NativeError(message or f"ternel_tq1 call failed with status {rc}")
