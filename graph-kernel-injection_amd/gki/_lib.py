"""ctypes binding of ``libgki_bsa.so`` (the C ABI in ``include/gki_bsa.h``).

The library is loaded lazily, once. If it is missing or fails to load, every
GPU entry point raises ``RuntimeError``: there is no CPU or eager fallback.
ctypes releases the GIL for the duration of each foreign call.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path
from typing import Optional

LIB_PATH = Path(__file__).resolve().parent / "libgki_bsa.so"
# The ABI the SIGNATURES table below binds (gki_abi_version() of a matching
# library). A library built from other sources may export the same names
# with other argument lists, so load() refuses any other version.
ABI_VERSION = 8

_c_int = ctypes.c_int32
_c_i64 = ctypes.c_int64
_c_ptr = ctypes.c_void_p
_c_float = ctypes.c_float

# name -> (restype, argtypes)
SIGNATURES = {
    "gki_abi_version": (ctypes.c_int, []),
    "gki_last_error": (ctypes.c_char_p, []),
    "gki_tile_sizes": (ctypes.c_int, [_c_ptr] * 6),
    "gki_streaming_mask": (ctypes.c_int, [_c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr]),
    "gki_dense_mask": (ctypes.c_int, [_c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_ptr]),
    "gki_tile_mask": (ctypes.c_int, [_c_ptr] + [_c_int] * 11 + [_c_ptr, _c_ptr]),
    "gki_block_list_counts": (ctypes.c_int, [_c_ptr, _c_int, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr,
                                             _c_ptr]),
    "gki_block_list_fill": (ctypes.c_int, [_c_ptr, _c_int, _c_int, _c_ptr, _c_ptr, _c_ptr, _c_ptr,
                                           _c_ptr]),
    "gki_dkdv_items": (ctypes.c_int, [_c_ptr, _c_int, _c_int, _c_int, _c_int, _c_ptr, _c_ptr, _c_ptr,
                                      _c_ptr, _c_ptr]),
    "gki_fwd_order": (ctypes.c_int, [_c_ptr, _c_int, _c_int, _c_ptr]),
    "gki_bsa_fwd": (ctypes.c_int, [_c_ptr] * 5 + [_c_int] * 7 + [_c_ptr, _c_ptr, _c_int, _c_ptr, _c_ptr]
                    + [_c_int] * 4 + [_c_float] + [_c_int] * 3 + [_c_ptr]),
    "gki_bsa_bwd": (ctypes.c_int, [_c_ptr] * 10 + [_c_int] * 7
                    + [_c_ptr, _c_ptr, _c_int, _c_ptr, _c_ptr, _c_int]      # CSR, CSC, n_kt
                    + [_c_ptr, _c_int, _c_ptr, _c_int, _c_int, _c_ptr]      # dK/dV work list
                    + [_c_ptr]                                              # dQ order
                    + [_c_ptr] + [_c_int] * 4 + [_c_float] + [_c_int] * 3 + [_c_ptr]),
    "gki_bsa_decode_workspace_floats": (ctypes.c_int64, [_c_int] * 5),
    "gki_decode_tokens": (ctypes.c_int, [_c_ptr, _c_int, _c_int, _c_int, _c_ptr] + [_c_int] * 7
                          + [_c_ptr, _c_ptr, _c_ptr]),
    "gki_bsa_decode": (ctypes.c_int, [_c_ptr] * 5 + [_c_int] * 7 + [_c_ptr, _c_int, _c_ptr]
                       + [_c_int] * 4 + [_c_float] + [_c_int] * 3 + [_c_ptr, _c_int, _c_ptr]),
    "gki_rolling_stream": (ctypes.c_int, [_c_i64] + [_c_int] * 4 + [_c_ptr] * 3),
    "gki_rolling_append": (ctypes.c_int, [_c_ptr] * 4 + [_c_int] * 6 + [_c_i64, _c_int, _c_ptr]),
    "gki_rolling_decode": (ctypes.c_int, [_c_ptr] * 5 + [_c_int] * 9 + [_c_i64, _c_float, _c_ptr,
                                                                       _c_int, _c_ptr]),
    "gki_rolling_decode_noalloc": (ctypes.c_int, [_c_ptr] * 5 + [_c_int] * 9
                                   + [_c_i64, _c_float, _c_int, _c_ptr]),
    "gki_read_probe_words": (ctypes.c_int64, [_c_int]),
    "gki_read_probe": (ctypes.c_int, [_c_ptr, _c_ptr, _c_int, _c_i64, _c_int, _c_int, _c_int, _c_ptr,
                                      _c_i64, _c_ptr]),
}

_lock = threading.Lock()
_lib: Optional[ctypes.CDLL] = None
_load_error: Optional[str] = None


def load() -> ctypes.CDLL:
    """Return the loaded library or raise ``RuntimeError`` explaining why not."""
    global _lib, _load_error
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if _load_error is None:
            try:
                lib = ctypes.CDLL(str(LIB_PATH))
                lib.gki_abi_version.restype = ctypes.c_int
                lib.gki_abi_version.argtypes = []
                found = int(lib.gki_abi_version())
                if found != ABI_VERSION:
                    _load_error = (f"{LIB_PATH.name} implements C ABI version {found}, this binding "
                                   f"needs version {ABI_VERSION} (a stale build)")
                else:
                    for name, (res, args) in SIGNATURES.items():
                        fn = getattr(lib, name)
                        fn.restype = res
                        fn.argtypes = args
                    _lib = lib
            except (OSError, AttributeError) as exc:
                _load_error = f"{type(exc).__name__}: {exc}"
        if _lib is None:
            raise RuntimeError(
                f"The gfx950 HIP library {LIB_PATH.name} is unavailable ({_load_error}). "
                "Build it with `python graph-kernel-injection_amd/build.py`; this kernel "
                "requires an AMD MI355X (gfx950) GPU and has no CPU fallback."
            )
        return _lib


def available() -> bool:
    try:
        load()
        return True
    except RuntimeError:
        return False


def check(rc: int, what: str) -> None:
    """Raise ``RuntimeError`` with the library's message if ``rc`` is non-zero."""
    if rc != 0:
        msg = load().gki_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (code {rc}): {msg}")


_TILE_SIZES: Optional[dict] = None


def tile_sizes() -> dict:
    """Kernel tile geometry (queried once from the library)."""
    global _TILE_SIZES
    if _TILE_SIZES is None:
        lib = load()
        vals = [ctypes.c_int32() for _ in range(6)]
        lib.gki_tile_sizes(*[ctypes.byref(v) for v in vals])
        keys = ("fwd_tile_m_16", "fwd_tile_m_32", "bwd_tile_m", "tile_n", "decode_tile_m",
                "decode_max_q")
        _TILE_SIZES = {k: int(v.value) for k, v in zip(keys, vals)}
    return _TILE_SIZES
