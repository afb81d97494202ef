"""ctypes binding of ``libhelios_paged.so`` (the C ABI in include/helios_paged.h).

Loading fails loudly: there is no CPU or PyTorch fallback for any operation.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

LIBRARY_PATH = Path(__file__).resolve().with_name("libhelios_paged.so")
HEADER_PATH = Path(__file__).resolve().parent.parent / "include" / "helios_paged.h"

HX_OK = 0
# hx_abi_version() of the library these signatures describe (bumped on any signature change).
ABI_VERSION = 6
HX_E_INVALID_ARG = -1
HX_E_UNSUPPORTED = -2
HX_E_WORKSPACE = -3
HX_E_OVERLAP = -4
HX_E_TOO_LARGE = -5

HX_DTYPE_BF16 = 0
HX_DTYPE_FP16 = 1

HX_WERR_BAD_PAGE = 1
HX_WERR_CLAMPED_LEN = 2
HX_WERR_BAD_CU_SEQ = 4
HX_WERR_GRID = 8
HX_WERR_PLAN_MISMATCH = 16
HX_WERR_BAD_QUERY_ROW = 32

_c_void_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_size = ctypes.c_size_t
_f32 = ctypes.c_float
_p_i32 = ctypes.POINTER(ctypes.c_int32)

# name -> (restype, argtypes); one entry per function declared in the header.
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "hx_strerror": (ctypes.c_char_p, [ctypes.c_int]),
    "hx_abi_version": (ctypes.c_int, []),
    "hx_kv_append": (
        ctypes.c_int,
        [_c_void_p, _c_void_p, _i64,
         _c_void_p, _i64, _i64,
         _c_void_p, _i64, _i64,
         _c_void_p, _i64,
         _i32, _i32, _i32,
         _c_void_p],
    ),
    "hx_kv_copy_pages": (
        ctypes.c_int,
        [ctypes.POINTER(_c_void_p), ctypes.POINTER(_c_void_p), _i32,
         _p_i32, _p_i32, _i32,
         _i32, _i64, _c_void_p],
    ),
    "hx_kv_gather": (
        ctypes.c_int,
        [_c_void_p, _i32, _i32, _i32, _i32, _i32,
         _c_void_p, _i32, _i64, _c_void_p, _c_void_p],
    ),
    "hx_varlen_attn_workspace_bytes": (_size, [_i32, _i32, _i32, _i32, _i32, _i32]),
    "hx_varlen_attn_count_items": (
        ctypes.c_int,
        [_p_i32, _p_i32, _i32, _i32, _i32, _i32, _i32, _p_i32, _p_i32, _p_i32],
    ),
    "hx_varlen_attn_plan": (
        ctypes.c_int,
        [_c_void_p, _c_void_p, _c_void_p, _i32, _i32, _i32, _i32, _i64,
         _i32, _i32, _i32, _i32, _i32, _i32, _i32,
         _c_void_p, _size, _c_void_p],
    ),
    "hx_varlen_attn_run": (
        ctypes.c_int,
        [_c_void_p, _i64, _i64,
         _c_void_p, _c_void_p, _i64, _i64,
         _i32, _i32, _c_void_p, _i32,
         _i32, _i32, _i32, _i32,
         _i32, _i32, _i32,
         _f32, _i32, _i32, _i32,
         _c_void_p, _i64, _i64, _c_void_p,
         _i32, _i32, _i32,
         _c_void_p, _size, _c_void_p],
    ),
    "hx_varlen_attn_run_rows": (
        ctypes.c_int,
        [_c_void_p, _i64, _i64,
         _c_void_p, _i64,
         _c_void_p, _c_void_p, _i64, _i64,
         _i32, _i32, _c_void_p, _i32,
         _i32, _i32, _i32, _i32,
         _i32, _i32, _i32,
         _f32, _i32, _i32, _i32,
         _c_void_p, _i64, _i64, _c_void_p,
         _i32, _i32, _i32,
         _c_void_p, _size, _c_void_p],
    ),
    "hx_varlen_attn_run_merged": (
        ctypes.c_int,
        [_c_void_p, _i64, _i64,
         _c_void_p, _c_void_p, _i64, _i64,
         _i32, _i32, _c_void_p, _i32,
         _i32, _i32, _i32, _i32,
         _i32, _i32, _i32,
         _f32, _i32, _i32, _i32,
         _c_void_p, _i64, _i64, _c_void_p,
         _c_void_p, _i64, _i64, _c_void_p, _i64,
         _c_void_p, _c_void_p, _i32,
         _c_void_p, _c_void_p, _i32,
         _i32, _i32, _i32,
         _c_void_p, _size, _c_void_p],
    ),
    "hx_varlen_attn_run_cascade": (
        ctypes.c_int,
        [_c_void_p, _i64, _i64,
         _c_void_p, _c_void_p, _i64, _i64,
         _i32, _i32, _c_void_p, _i32,
         _i32, _i32, _i32, _i32,
         _i32, _i32, _i32,
         _f32, _i32, _i32, _i32,
         _c_void_p, _i64, _i64, _c_void_p,
         _c_void_p, _i64, _i64, _c_void_p, _i64,
         _i32, _i32, _i32,
         _i32, _c_void_p, _size,
         _c_void_p, _i32, _c_void_p, _i64, _i32, _i32, _i32,
         _c_void_p, _c_void_p, _i32,
         _c_void_p, _c_void_p, _i32,
         _i32, _i32, _i32,
         _c_void_p, _size, _c_void_p],
    ),
    "hx_varlen_attn_append_run": (
        ctypes.c_int,
        [_c_void_p, _i64, _i64,
         _c_void_p, _c_void_p, _i64, _i64,
         _i32, _i32, _c_void_p, _i32,
         _i32, _i32, _i32, _i32,
         _i32, _i32, _i32,
         _f32, _i32, _i32, _i32,
         _c_void_p, _i64, _i64, _c_void_p,
         _c_void_p, _i64, _i64,
         _c_void_p, _i64, _i64,
         _c_void_p, _i64,
         _i32, _i32, _i32,
         _c_void_p, _size, _c_void_p],
    ),
    "hx_varlen_attn": (
        ctypes.c_int,
        [_c_void_p, _i64, _i64,
         _c_void_p, _c_void_p, _i64, _i64,
         _i32, _i32, _c_void_p, _i32,
         _c_void_p, _c_void_p, _c_void_p,
         _i32, _i32, _i32, _i32, _i64,
         _i32, _i32, _i32,
         _f32, _i32, _i32, _i32,
         _c_void_p, _i64, _i64, _c_void_p,
         _c_void_p, _size, _c_void_p],
    ),
    "hx_varlen_attn_error_word_offset": (_size, []),
    "hx_varlen_attn_noalloc": (
        ctypes.c_int,
        [_c_void_p, _i64, _i64,
         _c_void_p, _c_void_p, _i64, _i64,
         _i32, _i32, _c_void_p, _i32,
         _c_void_p, _c_void_p, _c_void_p,
         _i32, _i32, _i32, _i32, _i64,
         _i32, _i32, _i32,
         _f32, _i32, _i32, _i32,
         _c_void_p, _i64, _i64, _c_void_p,
         _c_void_p],
    ),
    "hx_qk_norm_rope_append": (
        ctypes.c_int,
        [_c_void_p, _i64, _i64,
         _c_void_p, _i64, _i64,
         _c_void_p, _i64, _i64,
         _c_void_p, _c_void_p,
         _c_void_p, _c_void_p, _i64,
         _c_void_p, _i64,
         _i32, _i32, _i32,
         _f32, _i32,
         _c_void_p, _i64, _i64,
         _c_void_p, _c_void_p, _i64,
         _c_void_p, _c_void_p],
    ),
    "hx_attn_merge": (
        ctypes.c_int,
        [_c_void_p, _i64, _i64, _c_void_p, _i64,
         _c_void_p, _i64, _i64, _c_void_p, _i64,
         _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i32, _i32, _i32, _c_void_p],
    ),
    "hx_tick_metadata": (
        ctypes.c_int,
        [_c_void_p, _i32, _i32, _i32,
         _c_void_p, _i32, _i32,
         _c_void_p, _c_void_p, _c_void_p,
         _c_void_p, _c_void_p, _c_void_p,
         _c_void_p],
    ),
    "hx_logits_workspace_bytes": (_size, [_i64, _i64, _i32]),
    "hx_final_norm_logits_argmax": (
        ctypes.c_int,
        [_c_void_p, _i64, _i64, _c_void_p,
         _i64, _c_void_p, _f32,
         _c_void_p, _i64,
         _i64, _i32, _i32,
         _c_void_p, _c_void_p,
         _c_void_p, _i64,
         _c_void_p, _size, _c_void_p],
    ),
}

_lib: ctypes.CDLL | None = None


class HeliosLibraryError(RuntimeError):
    """The native library is missing or does not match the header."""


def lib() -> ctypes.CDLL:
    """Load the library once; raise HeliosLibraryError if it was not built."""
    global _lib
    if _lib is None:
        if not LIBRARY_PATH.exists():
            raise HeliosLibraryError(
                f"{LIBRARY_PATH.name} is not built; run `python -m helios_amd.build` "
                "(hipcc, gfx950). helios_amd has no CPU fallback."
            )
        handle = ctypes.CDLL(str(LIBRARY_PATH))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        found = handle.hx_abi_version()
        if found != ABI_VERSION:
            raise HeliosLibraryError(
                f"{LIBRARY_PATH.name} has ABI version {found}, these bindings expect "
                f"{ABI_VERSION}; rebuild it with `python -m helios_amd.build`."
            )
        _lib = handle
    return _lib


def strerror(code: int) -> str:
    return lib().hx_strerror(code).decode()


def check(code: int, what: str) -> None:
    """Map a status code to the reference's exception convention."""
    if code == HX_OK:
        return
    message = f"{what}: {strerror(code)} (status {code})"
    if code < 0:
        raise ValueError(message)
    raise RuntimeError(message)


def header_functions() -> list[str]:
    """Names of the functions declared in include/helios_paged.h."""
    import re

    text = HEADER_PATH.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"\b(hx_[a-z0-9_]+)\s*\(", text)
