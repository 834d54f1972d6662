"""ctypes binding of libtaomate_ltx.so (the C ABI declared in include/taomate_ltx.h).

The library is required: there is no fallback path.  Loading fails with
``NativeLibraryError`` when the shared object is missing, and every entry point
raises ``NativeCallError`` with the library's own message on a non-zero status.
"""
from __future__ import annotations

import ctypes
import os
import pathlib
import threading

LIB_DIR = pathlib.Path(__file__).resolve().parent / "lib"
LIB_NAME = "libtaomate_ltx.so"

F32, BF16, F8E4M3 = 0, 1, 2
MAX_SEGMENTS = 16
MAX_KEYLEN_BATCH = 16  # LTX_MAX_KEYLEN_BATCH
NOALLOC_SCRATCH_BYTES = 24 << 20  # LTX_NOALLOC_SCRATCH_BYTES
ABI_VERSION = 2

_i64 = ctypes.c_int64
_int = ctypes.c_int
_ptr = ctypes.c_void_p
_f32 = ctypes.c_float

# name -> argument types, in the order of include/taomate_ltx.h
SIGNATURES = {
    "ltx_abi_version": [],
    "ltx_last_error": [],
    "ltx_rope_table": [_ptr, _ptr, _int, _ptr, _i64, _int, _i64, _i64, _i64, _i64, _int, _f32, _f32,
                       _f32, _i64, _i64, _i64, _ptr],
    "ltx_rope_table_retime": [_ptr, _ptr, _ptr, _ptr, _int, _ptr, _i64, _i64, _i64, _i64, _i64, _f32, _i64, _i64,
                              _ptr],
    "ltx_qk_rmsnorm_rope": [_int, _i64, _i64, _i64,
                            _ptr, _i64, _i64, _i64, _ptr, _i64, _i64, _ptr, _f32, _ptr, _ptr, _i64,
                            _i64, _i64,
                            _ptr, _i64, _i64, _i64, _ptr, _i64, _i64, _ptr, _f32, _ptr, _ptr, _i64,
                            _i64, _i64,
                            _int, _ptr],
    "ltx_qk_rmsnorm_rope_v": [_int, _i64, _i64, _i64,
                              _ptr, _i64, _i64, _i64, _ptr, _i64, _i64, _ptr, _f32, _ptr, _ptr, _i64,
                              _i64, _i64,
                              _ptr, _i64, _i64, _i64, _ptr, _i64, _i64, _ptr, _f32, _ptr, _ptr, _i64,
                              _i64, _i64, _int,
                              _ptr, _i64, _i64, _i64, _i64, _ptr, _i64, _i64, _i64, _ptr],
    "ltx_kv_append": [_int, _int, _i64, _i64, _i64, _i64, _ptr, _i64, _i64, _i64, _ptr, _i64, _i64,
                      _i64, _i64, _ptr, _i64, _i64, _i64, _ptr],
    "ltx_kv_append_fp8_pair": [_i64, _i64, _i64, _i64, _i64, _ptr, _i64, _i64, _i64, _ptr, _ptr, _ptr, _i64,
                               _i64, _i64, _ptr, _ptr, _i64, _i64, _i64, _i64, _i64, _ptr],
    "ltx_kv_gather": [_i64, _i64, _i64, _i64, _ptr, _i64, _i64, _i64, _ptr, _i64, _i64, _i64, _i64,
                      _ptr, _ptr, _ptr],
    "ltx_flash_attn_fwd": [_ptr, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _ptr, _ptr, _ptr,
                           _i64, _i64, _i64, _i64, _i64, _i64, _i64, _int, _ptr, _ptr, _i64, _i64,
                           _i64, _ptr, _i64, _ptr, _ptr, _i64, _i64, _i64, _ptr, _f32, _ptr, _i64, _ptr],
    "ltx_flash_attn_fwd_noalloc": [_ptr, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _ptr, _ptr, _ptr,
                                   _i64, _i64, _i64, _i64, _i64, _i64, _i64, _int, _ptr, _ptr, _i64, _i64,
                                   _i64, _ptr, _i64, _ptr, _ptr, _i64, _i64, _i64, _ptr, _f32, _ptr],
    "ltx_flash_attn_workspace_size": [_i64, _i64, _i64, _i64, _ptr],
    "ltx_adaln": [_i64, _i64, _i64, _ptr, _i64, _i64, _ptr, _i64, _i64, _ptr, _i64, _i64, _ptr, _i64, _i64,
                  _ptr, _i64, _i64, _ptr, _i64, _i64, _ptr, _i64, _i64, _f32, _ptr],
}


class NativeLibraryError(RuntimeError):
    """The HIP library could not be loaded (not built, wrong ABI)."""


class NativeCallError(RuntimeError):
    """An entry point returned a non-zero ltx_status."""


_lock = threading.Lock()
_lib = None


def lib_path() -> pathlib.Path:
    return pathlib.Path(os.environ.get("TAOMATE_LTX_LIB", LIB_DIR / LIB_NAME))


def load() -> ctypes.CDLL:
    """Load (once) and type the shared library; raise if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = lib_path()
        if not path.exists():
            raise NativeLibraryError(
                f"{path} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
                "or `python -m taomate_amd.build` (hipcc, gfx950)")
        try:
            lib = ctypes.CDLL(str(path))
        except OSError as e:
            raise NativeLibraryError(f"cannot load {path}: {e}") from e
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = ctypes.c_char_p if name == "ltx_last_error" else ctypes.c_int
        ver = lib.ltx_abi_version()
        if ver != ABI_VERSION:
            raise NativeLibraryError(f"{path}: ABI version {ver}, expected {ABI_VERSION}")
        _lib = lib
        return lib


def call(name: str, *args) -> None:
    """Invoke an entry point and raise NativeCallError on failure."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.ltx_last_error().decode(errors="replace")
        raise NativeCallError(f"{name} failed ({rc}): {msg}")


def i64_array(values):
    arr = (ctypes.c_int64 * max(1, len(values)))(*[int(v) for v in values])
    return arr


def ptr_array(values):
    arr = (ctypes.c_void_p * max(1, len(values)))(*[int(v) if v else None for v in values])
    return arr
