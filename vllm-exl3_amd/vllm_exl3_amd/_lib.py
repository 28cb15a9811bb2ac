"""ctypes binding of the C ABI in ``include/exl3_mi355x.h``.

The library ``libexl3_mi355x.so`` sits next to this file (built in-tree by
``make -C vllm-exl3_amd/csrc``).  There is no fallback: if the library is
missing or fails to load, every entry point raises.
"""

from __future__ import annotations

import ctypes
import os
import pathlib
import threading

LIB_PATH = pathlib.Path(__file__).resolve().parent / "libexl3_mi355x.so"

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float
_sz = ctypes.c_size_t

# name -> argtypes (restype is int status unless listed in _RESTYPES)
SIGNATURES: dict[str, list] = {
    "exl3_last_error": [],
    "exl3_abi_version": [],
    "exl3_dequant_trellis": [_p, _i64, _i64, _i64, _i32, _p, _p, _p, _p],
    "exl3_decode_tiles": [_p, _i64, _i64, _i64, _i32, _p, _p],
    "exl3_gemm_workspace_size": [_i64, _i64, _i64],
    "exl3_gemm": [_p, _i32, _i64, _p, _i64, _i64, _i64, _i32, _p, _p, _p, _i32, _p, _i64, _p],
    "exl3_linear": [_p, _i32, _i64, _p, _i64, _i64, _i64, _i32, _p, _p, _p, _i32, _p, _i32, _p, _i64, _p],
    "exl3_gemv_batched_workspace_size": [_i64, _i64, _i64, _i64],
    "exl3_gemv_batched": [_p, _i32, _i64, _i64, _i64, _p, _p, _p, _i64, _p, _i64, _i64, _i32, _p, _i32,
                          _p, _i64, _p],
    "exl3_moe_workspace_size": [_i64, _i64, _i64, _i64, _i64, _i32],
    "exl3_moe_forward": [_p, _i32, _i64, _i64, _i64] + [_p] * 9 + [_i64, _p, _p, _p, _i64, _i64, _i64,
                         _i32, _i32, _i32, _f32, _p, _i32, _p, _i32, _i64, _p, _p, _i32, _p, _i64, _p],
    "exl3_moe_forward_noalloc": [_p, _i32, _i64, _i64, _i64] + [_p] * 9 + [_i64, _p, _p, _p, _i64, _i64,
                                 _i64, _i32, _i32, _i32, _f32, _p, _i32, _p, _i32, _i64, _p, _p, _i32,
                                 _p],
    "exl3_fat_gemm": [_p, _i64, _p, _i64, _i64, _i64, _i32, _p, _p, _p],
    "exl3_fat_gemm_workspace_size": [_i64, _i64, _i32],
    "exl3_fat_gemm_scatter": [_p, _i64, _p, _i64, _i64, _i64, _i32, _p, _p, _p, _p, _i64, _p, _i64,
                              _p],
    "exl3_moe_prefill_workspace_size": [_i64, _i64, _i64, _i64, _i64, _i32],
    "exl3_moe_prefill": [_p, _i32, _i64, _i64, _i64] + [_p] * 9 + [_i64, _p, _p, _p, _i64, _i64, _i64,
                         _i32, _i32, _i32, _f32, _p, _i32, _p, _i32, _i64, _p, _p, _i32, _p, _i64, _p],
    "exl3_kv_page_bytes": [],
    "exl3_kv_pack_pages": [_p, _p, _i32, _i64, _i64, _i64, _i64, _i64, _p, _p, _i64, _i64, _p, _i64,
                           _p],
    "exl3_kv_unpack_pages": [_p, _i64, _i64, _p, _p, _i64, _i64, _i64, _p, _p, _i64, _p],
    "exl3_kv_decode_workspace_size": [_i64, _i64, _i64, _i64, _i64],
    "exl3_kv_decode": [_p, _i32, _i64, _i64, _i64, _i64, _i64, _p, _i64, _p, _i64, _i64, _p, _f32,
                       _p, _i32, _i64, _i64, _i64, _p, _i64, _p],
    "exl3_nvfp4_page_bytes": [_i64],
    "exl3_nvfp4_pack_pages": [_p, _p, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p, _i64, _i64,
                              _p, _i64, _p],
    "exl3_nvfp4_dequant_pages": [_p, _i64, _i64, _p, _p],
    "exl3_nvfp4_stage_pages": [_p, _i64, _i64, _p, _i32, _i64, _p, _i64, _p],
    "exl3_nvfp4_decode_workspace_size": [_i64, _i64, _i64],
    "exl3_nvfp4_sparse_decode": [_p, _i32, _i64, _i64, _i64, _i64, _i64, _p, _i64, _p, _i64, _i64,
                                 _i64, _p, _i64, _i64, _p, _i64, _f32, _p, _i32, _i64, _i64, _i64,
                                 _p, _i64, _p],
    "exl3_ngram_dequant": [_p, _i64, _i64, _i32, _p, _p, _i64, _p, _p],
    "exl3_nvfp4_w1_insert": [_p, _i64, _i64, _p, _p, _p, _p, _i32, _p, _i32, _i64, _p, _i64, _i64,
                             _i64, _i64, _f32, _p, _p, _p, _i64, _p, _i64, _p, _p, _p],
    "exl3_profile_begin": [_i32],
    "exl3_profile_end": [_p, _i32, _p, _p],
    "exl3_fill_hash_u32": [_p, _i64, ctypes.c_uint64, _p],
}
_RESTYPES = {"exl3_last_error": ctypes.c_char_p, "exl3_gemm_workspace_size": _i64,
             "exl3_moe_workspace_size": _i64, "exl3_fat_gemm_workspace_size": _i64,
             "exl3_gemv_batched_workspace_size": _i64,
             "exl3_nvfp4_page_bytes": _i64, "exl3_nvfp4_decode_workspace_size": _i64,
             "exl3_moe_prefill_workspace_size": _i64, "exl3_kv_page_bytes": _i64,
             "exl3_kv_decode_workspace_size": _i64}

_LOCK = threading.Lock()
_LIB: ctypes.CDLL | None = None


class NativeLibraryError(RuntimeError):
    """The HIP library is missing or an entry point reported an error."""


def load() -> ctypes.CDLL:
    """Load and type the library once; raise if it is not built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    with _LOCK:
        if _LIB is not None:
            return _LIB
        if not LIB_PATH.exists():
            raise NativeLibraryError(
                f"{LIB_PATH.name} is not built: run `make -C {LIB_PATH.parent.parent / 'csrc'}` "
                "(or __graft_entry__.build()); there is no CPU fallback"
            )
        lib = ctypes.CDLL(str(LIB_PATH), mode=os.RTLD_LAZY | os.RTLD_LOCAL)
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = _RESTYPES.get(name, ctypes.c_int)
        _LIB = lib
        return lib


def exported_symbols() -> list[str]:
    return list(SIGNATURES)


def last_error() -> str:
    msg = load().exl3_last_error()
    return msg.decode() if msg else ""


def call(name: str, *args) -> None:
    """Invoke an entry point and raise RuntimeError with its message on failure."""
    status = getattr(load(), name)(*args)
    if status != 0:
        raise NativeLibraryError(f"{name}: {last_error()} (status {status})")
