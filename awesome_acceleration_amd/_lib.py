"""ctypes binding of libaac_attn.so (the C ABI declared in include/aac_attn.h).

torch is imported before the library is opened so that the library binds
to the HIP runtime torch already loaded (one runtime per process: streams and
device pointers handed over from torch are then valid inside the library).

There is no fallback: if the shared library is missing or lacks a symbol,
``lib()`` raises and every op that needs it fails loudly.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  (must precede loading the HIP library)

from .build import LIB_PATH

_c_int = ctypes.c_int
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_size = ctypes.c_size_t
_p = ctypes.c_void_p

# name -> (restype, argtypes); must mirror include/aac_attn.h exactly.
SIGNATURES: dict[str, tuple] = {
    "aac_abi_version": (_c_int, []),
    "aac_strerror": (ctypes.c_char_p, [_c_int]),
    "aac_kv_store": (_c_int, [_p, _p, _i64, _i64, _p, _p, _i64, _p, _i64, _i32, _i32, _i32, _p]),
    "aac_kv_append_paged": (
        _c_int,
        [_p, _p, _i64, _i64, _p, _p, _i64, _i32, _p, _i32, _p, _i32, _i32, _i32, _i32, _p],
    ),
    "aac_prefill_varlen": (
        _c_int,
        [_p, _p, _p, _i64, _i64, _i64, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _i32,
         _p, _i64, _p, _size, _i32, _p],
    ),
    "aac_prefill_workspace_bytes": (_size, [_i32, _i32, _i32, _i32, _i32, _i32, _i32]),
    "aac_prefill_varlen_store": (
        _c_int,
        [_p, _p, _p, _i64, _i64, _i64, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _i32,
         _p, _i64, _p, _p, _i64, _p, _i64, _i32, _p],
    ),
    "aac_decode_workspace_bytes": (_size, [_i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32]),
    "aac_decode_paged": (
        _c_int,
        [_p, _i64, _p, _p, _i64, _i32, _p, _i32, _p, _i32, _i32, _i32, _i32, _i32, _f32, _p, _i64,
         _p, _size, _i32, _i32, _p],
    ),
    "aac_decode_paged_noalloc": (
        _c_int,
        [_p, _i64, _p, _p, _i64, _i32, _p, _i32, _p, _i32, _i32, _i32, _i32, _i32, _f32, _p, _i64,
         _i32, _i32, _p],
    ),
    "aac_decode_append_paged": (
        _c_int,
        [_p, _i64, _p, _p, _i64, _i64, _p, _p, _i64, _i32, _p, _i32, _p, _i32, _i32, _i32, _i32,
         _i32, _f32, _p, _i64, _p, _size, _i32, _i32, _p],
    ),
    "aac_rmsnorm": (_c_int, [_p, _i64, _p, _p, _p, _p, _i64, _i32, _f32, _i32, _p]),
    "aac_qk_norm_rope_store": (
        _c_int,
        [_p, _i64, _i64, _i32, _i32, _i32, _p, _p, _f32, _p, _p, _i32, _p, _p, _p, _p, _p, _i64,
         _p, _p, _i32, _p, _i32, _i32, _p],
    ),
    "aac_silu_mul": (_c_int, [_p, _p, _i64, _i32, _i32, _p]),
    "aac_gemm_nt": (
        _c_int, [_p, _i64, _p, _i64, _p, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _p]),
    "aac_qkv_norm_rope_store": (
        _c_int,
        [_p, _i64, _p, _i64, _i64, _i32, _i32, _i32, _i32, _p, _p, _f32, _p, _p, _i32, _p, _p, _p,
         _p, _p, _i64, _p, _p, _i32, _p, _i32, _i32, _p]),
    "aac_argmax_rows": (_c_int, [_p, _i64, _i64, _i64, _p, _i32, _p]),
    "aac_kv_export_paged": (
        _c_int, [_p, _i64, _i64, _i32, _i64, _i32, _i32, _i32, _p, _i32, _i32, _p, _i32, _p]),
    "aac_kv_import_paged": (
        _c_int, [_p, _p, _i64, _i64, _i32, _i64, _i32, _i32, _i32, _p, _i32, _i32, _i32, _p]),
}

ABI_VERSION = 2

AAC_DTYPE = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}

_lock = threading.Lock()
_lib = None


def lib_path() -> Path:
    return LIB_PATH


def lib() -> ctypes.CDLL:
    """Open (once) and return the attention library; raise if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build it with `python -m awesome_acceleration_amd.build` "
                    "(no CPU fallback exists for these ops)")
            handle = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)  # AttributeError if the export is missing
                fn.restype = res
                fn.argtypes = args
            v = handle.aac_abi_version()
            if v != ABI_VERSION:
                raise RuntimeError(f"libaac_attn ABI {v} != expected {ABI_VERSION}")
            _lib = handle
    return _lib


def check(rc: int, what: str) -> None:
    """Raise RuntimeError for a non-zero status from the library."""
    if rc != 0:
        msg = lib().aac_strerror(rc).decode()
        raise RuntimeError(f"{what} failed: {msg} (code {rc})")
