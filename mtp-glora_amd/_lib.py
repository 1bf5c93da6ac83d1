"""ctypes binding of libmtp_glora_amd.so (the C ABI of include/mtp_glora_amd.h).

The library is loaded from ``lib/`` next to this file. There is no fallback:
if it is missing every operation raises, naming the build command.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

_HERE = Path(__file__).resolve().parent
# MGA_LIBRARY names another build of the same C ABI (e.g. a variant timed
# against the in-tree one); the default is the in-tree build
LIB_PATH = Path(os.environ.get("MGA_LIBRARY") or (_HERE / "lib" / "libmtp_glora_amd.so"))

MGA_OK = 0
MGA_ERR_INVALID = 1
MGA_ERR_CAPACITY = 2
MGA_ERR_HIP = 3
DTYPE_BF16 = 0
DTYPE_F32 = 1
DTYPE_F16 = 2
BWD_DQ = 1
BWD_DKDV = 2
BWD_WS_WORDS_PER_ROW = 3   # MGA_BWD_WS_WORDS_PER_ROW: delta workspace words per (query head, row)

# name -> argtypes; every function returns int (status) unless listed in _RESTYPES
_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_F32 = ctypes.c_float
_F64 = ctypes.c_double
_U64 = ctypes.c_uint64
SIGNATURES = {
    "mga_version": [],
    "mga_last_error": [],
    "mga_kv_append": [_P, _P, _I64, _I64, _I64, _P, _I32, _P, _P, _I64, _I64, _I64, _I64, _I32, _I32, _I32, _P],
    "mga_regular_index": [_P, _I64, _I32, _P, _P, _P],
    "mga_mtp_block_mask": [_P, _I64, _I32, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P],
    "mga_attn_fwd": [_P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64,
                     _P, _P, _P, _P, _P, _P,
                     _I32, _I32, _I32, _I32, _I32, _I32, _I32, _F32, _P],
    "mga_attn_bwd": [_P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64,
                     _P, _P,
                     _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64,
                     _I32, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                     _I32, _I32, _I32, _I32, _I32, _I32, _I32, _F32, _I32, _P],
    "mga_attn_bwd_noalloc": [_P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64,
                             _P,
                             _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64,
                             _I32, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                             _I32, _I32, _I32, _I32, _I32, _I32, _I32, _F32, _I32, _P],
    "mga_qk_norm_rope_fwd": [_P, _I64, _I64, _P, _I64, _I64, _P, _P, _P, _P, _I64, _F32,
                             _I32, _I32, _I32, _I32, _I32, _P, _I64, _I64, _P, _I64, _I64, _P, _P],
    "mga_qk_norm_rope_stage_fwd": [_P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _P, _P, _P, _P, _I64, _F32,
                                   _P, _I32, _I32, _I32, _I32, _I32, _I32, _P, _I64, _I64, _P, _I64, _I64,
                                   _P, _I64, _I64, _P, _P],
    "mga_qk_norm_rope_bwd": [_P, _I64, _I64, _P, _I64, _I64, _P, _P, _P, _P, _I64, _P,
                             _I32, _I32, _I32, _I32, _I32, _P, _I64, _I64, _P, _I64, _I64,
                             _P, _I64, _I64, _P, _I64, _I64, _P],
    "mga_gated_lora_workspace_bytes": [_I32, _I32, _I32, _I32],
    "mga_gated_lora_fwd": [_P, _I64, _P, _I64, _P, _I64, _P, _I64, _P, _F32, _F64, _U64,
                           _I32, _I32, _I32, _I32, _P, _I64, _P, _I64, _P, _I64, _P, _I64, _I32, _P],
    "mga_gated_lora_bwd": [_P, _I64, _P, _I64, _P, _I64, _P, _I64, _P, _I64, _P, _I64, _P, _I64, _P, _F32,
                           _F64, _U64, _I32, _I32, _I32, _I32, _P, _I64, _P, _I64, _P, _I64, _P, _I64, _I32, _P],
    "mga_soft_ce_workspace_floats": [_I32, _I32],
    "mga_soft_ce_fwd": [_P, _I64, _P, _I64, _I32, _I32, _I32, _P, _P, _P, _P],
    "mga_soft_ce_bwd": [_P, _I64, _P, _I64, _I32, _I32, _I32, _P, _P, _P, _I64, _P],
}
_RESTYPES = {"mga_last_error": ctypes.c_char_p, "mga_soft_ce_workspace_floats": ctypes.c_int64,
             "mga_gated_lora_workspace_bytes": ctypes.c_int64}


class MGAError(RuntimeError):
    """Raised when a library call returns a non-zero status."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed (code {code}): {msg}")
        self.code = code


class CapacityError(MGAError):
    pass


_lock = threading.Lock()
_lib = None


def load() -> ctypes.CDLL:
    """Load the library once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build it with `python __graft_entry__.py` "
                    "(or mtp-glora_amd/build.py). There is no CPU fallback.")
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, argtypes in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.argtypes = argtypes
                fn.restype = _RESTYPES.get(name, ctypes.c_int)
            _lib = lib
    return _lib


def call(name: str, *args) -> None:
    fn = getattr(load(), name)
    rc = fn(*args)
    if rc != MGA_OK:
        msg = load().mga_last_error().decode(errors="replace")
        cls = CapacityError if rc == MGA_ERR_CAPACITY else MGAError
        raise cls(name, rc, msg)


def version() -> int:
    return int(load().mga_version())
