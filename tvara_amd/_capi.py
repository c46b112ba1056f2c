"""ctypes binding of libtvara_capi.so (include/tvara_capi.h).

Library discovery follows the reference's loader (python/tvara/native.py:12-24):
an explicit path, then $TVARA_LIBRARY, then build/{release,debug}/ under the
repository root.  A missing library raises FileNotFoundError: there is no CPU
fallback.
"""

from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


class Handle(C.Structure):
    """tvara_kv_handle: BlockHandle (kv.hpp:35)."""

    _fields_ = [("id", C.c_uint64), ("generation", C.c_uint64)]


_sz = C.c_size_t
_u64 = C.c_uint64
_fp = C.POINTER(C.c_float)
_vp = C.c_void_p

# name -> (restype, argtypes); every export of include/tvara_capi.h
SIGNATURES = {
    # model-level exports (c_api.h:13-24)
    "tvara_model_open": (_vp, [C.c_char_p, _sz, _sz]),
    "tvara_model_close": (None, [_vp]),
    "tvara_model_vocab_size": (_sz, [_vp]),
    "tvara_model_context_size": (_sz, [_vp]),
    "tvara_model_metadata": (C.c_char_p, [_vp]),
    "tvara_sequence_create": (_u64, [_vp]),
    "tvara_sequence_decode": (C.c_int, [_vp, _u64, C.c_uint32, _fp, _sz]),
    "tvara_sequence_drop": (C.c_int, [_vp, _u64]),
    "tvara_sequence_decode_batch": (C.c_int, [_vp, _u64, C.POINTER(C.c_uint32), _sz, _fp, _sz]),
    "tvara_sequence_prefill": (C.c_int, [_vp, _u64, C.POINTER(C.c_uint32), _sz, _fp, _sz]),
    "tvara_sequence_truncate": (C.c_int, [_vp, _u64, _sz]),
    "tvara_sequences_decode": (C.c_int, [_vp, C.POINTER(_u64), C.POINTER(C.c_uint32), _sz, _fp, _sz]),
    "tvara_model_cache": (_vp, [_vp]),
    "tvara_radix_create": (_vp, [_vp, C.c_char_p]),
    "tvara_radix_destroy": (None, [_vp]),
    "tvara_radix_insert": (C.c_int, [_vp, C.POINTER(C.c_int32), _sz, C.POINTER(_u64)]),
    "tvara_radix_lookup": (C.c_int, [_vp, C.POINTER(C.c_int32), _sz, C.POINTER(_u64), C.POINTER(_sz)]),
    "tvara_radix_attach": (C.c_int, [_vp, _u64, _u64]),
    "tvara_radix_reuse": (C.c_int, [_vp, C.POINTER(C.c_int32), _sz, C.c_int, C.POINTER(_u64), C.POINTER(_sz)]),
    "tvara_radix_pin": (C.c_int, [_vp, _u64]),
    "tvara_radix_unpin": (C.c_int, [_vp, _u64]),
    "tvara_radix_touch": (C.c_int, [_vp, _u64]),
    "tvara_radix_eviction_candidate": (C.c_int, [_vp, C.POINTER(_u64)]),
    "tvara_radix_evict_one": (C.c_int, [_vp, C.POINTER(C.c_int)]),
    "tvara_radix_reset": (C.c_int, [_vp]),
    "tvara_radix_size": (C.c_int, [_vp, C.POINTER(_sz)]),
    "tvara_radix_node": (C.c_int, [_vp, _u64, C.POINTER(_u64), C.POINTER(C.c_int32), _sz, C.POINTER(_sz),
                                   C.POINTER(_sz), C.POINTER(_u64), C.POINTER(_sz), C.POINTER(_sz), C.POINTER(_sz)]),
    "tvara_radix_external_references": (C.c_int, [_vp, C.POINTER(_sz), _sz]),
    "tvara_last_error": (C.c_char_p, []),
    "tvara_last_status": (C.c_int, []),
    "tvara_kv_cache_create": (_vp, [_sz, _sz, _sz, _sz, _sz, C.c_int]),
    "tvara_kv_cache_destroy": (None, [_vp]),
    "tvara_kv_block_bytes": (_sz, [_vp]),
    "tvara_kv_set_stream": (C.c_int, [_vp, _vp]),
    "tvara_kv_synchronize": (C.c_int, [_vp]),
    "tvara_kv_pool_allocate": (C.c_int, [_vp, C.POINTER(Handle)]),
    "tvara_kv_pool_retain": (C.c_int, [_vp, Handle]),
    "tvara_kv_pool_release": (C.c_int, [_vp, Handle]),
    "tvara_kv_pool_references": (C.c_int, [_vp, Handle, C.POINTER(_sz)]),
    "tvara_kv_pool_references_by_id": (C.c_int, [_vp, _sz, C.POINTER(_sz)]),
    "tvara_kv_pool_available": (_sz, [_vp]),
    "tvara_kv_pool_audit": (C.c_int, [_vp]),
    "tvara_kv_pool_state": (C.c_int, [_vp, C.POINTER(_sz), C.POINTER(_u64), C.POINTER(_sz), C.POINTER(_sz)]),
    "tvara_kv_block_read": (C.c_int, [_vp, Handle, _vp, _sz]),
    "tvara_kv_block_write": (C.c_int, [_vp, Handle, _sz, _vp, _sz]),
    "tvara_kv_block_checksums": (C.c_int, [_vp, C.POINTER(Handle), _sz, C.POINTER(_u64)]),
    "tvara_kv_sequence_create": (_u64, [_vp]),
    "tvara_kv_sequence": (C.c_int, [_vp, _u64, C.POINTER(_sz), C.POINTER(Handle), _sz, C.POINTER(_sz)]),
    "tvara_kv_sequence_ids": (C.c_int, [_vp, C.POINTER(_u64), _sz, C.POINTER(_sz)]),
    "tvara_kv_physical_block": (C.c_int, [_vp, _u64, _sz, C.POINTER(Handle)]),
    "tvara_kv_append": (C.c_int, [_vp, _u64, _fp, _fp]),
    "tvara_kv_append_batch": (C.c_int, [_vp, C.POINTER(_u64), _sz, _fp, _fp, C.c_int, C.POINTER(_sz)]),
    "tvara_kv_append_tokens": (C.c_int, [_vp, _u64, _fp, _fp, _sz, C.c_int, C.POINTER(_sz)]),
    "tvara_kv_read": (C.c_int, [_vp, _u64, _sz, _sz, C.c_int, _fp]),
    "tvara_kv_read_all": (C.c_int, [_vp, _u64, _sz, C.c_int, _fp, _sz]),
    "tvara_kv_drop": (C.c_int, [_vp, _u64]),
    "tvara_kv_fork": (_u64, [_vp, _u64]),
    "tvara_kv_truncate": (C.c_int, [_vp, _u64, _sz]),
    "tvara_kv_truncate_batch": (C.c_int, [_vp, C.POINTER(_u64), C.POINTER(_sz), _sz, C.POINTER(_sz)]),
    "tvara_kv_audit": (C.c_int, [_vp, C.POINTER(_sz), _sz]),
    "tvara_kv_import_sequence": (_u64, [_vp, C.POINTER(Handle), _sz, _sz, _sz]),
    "tvara_attn_decode": (C.c_int, [_vp, C.POINTER(_u64), _sz, _sz, _sz, _sz, _fp, _fp, _fp, C.POINTER(_sz), _fp,
                                    C.c_int]),
    "tvara_attn_prefill": (C.c_int, [_vp, C.POINTER(_u64), _sz, _sz, _sz, _sz, C.POINTER(_sz), C.POINTER(_sz), _fp,
                                     _fp, C.c_int, C.c_int]),
    "tvara_attn_decode_noalloc": (C.c_int, [_vp, C.POINTER(_u64), _sz, _sz, _sz, _sz, _vp, _vp, _vp,
                                            C.POINTER(_sz), _vp]),
    "tvara_attn_decode_noalloc_limit": (_sz, []),
    "tvara_attn_plan_create": (_vp, [_vp, C.POINTER(_u64), _sz, _sz, _sz, C.POINTER(_sz), C.c_int]),
    "tvara_attn_plan_decode": (C.c_int, [_vp, _sz, _vp, _vp, _vp, _vp, _vp]),
    "tvara_attn_plan_check": (C.c_int, [_vp]),
    "tvara_attn_plan_info": (C.c_int, [_vp, C.POINTER(_sz), C.POINTER(_sz), C.POINTER(_sz)]),
    "tvara_attn_plan_destroy": (None, [_vp]),
    "tvara_prefill_plan_create": (_vp, [_vp, C.POINTER(_u64), _sz, _sz, _sz, C.POINTER(_sz), C.POINTER(_sz), C.c_int]),
    "tvara_prefill_plan_launch": (C.c_int, [_vp, _sz, _vp, _vp, _vp]),
    "tvara_prefill_plan_check": (C.c_int, [_vp]),
    "tvara_prefill_plan_destroy": (None, [_vp]),
    "tvara_profile_enable": (C.c_int, [C.c_int]),
    "tvara_profile_read": (C.c_int, [C.c_char_p, C.POINTER(C.c_double), C.POINTER(_sz)]),
    "tvara_profile_reset": (C.c_int, []),
}

OK, ERROR, INVALID, EXHAUSTED, LOGIC = 0, -1, -2, -3, -4
KV_F32, KV_Q8_0 = 0, 1
ATTN_F32, ATTN_BF16, ATTN_F32X3 = 0, 1, 2


class NativeError(RuntimeError):
    """A failure reported by libtvara_capi (std::runtime_error or HIP)."""


class InvalidArgument(NativeError, ValueError):
    """std::invalid_argument in the reference."""


class CacheExhausted(NativeError):
    """tvara::CacheExhausted (kv.hpp:34)."""


class LogicError(NativeError):
    """std::logic_error: a violated audit invariant (kv.hpp:61-64, 138-146)."""


_ERRORS = {INVALID: InvalidArgument, EXHAUSTED: CacheExhausted, LOGIC: LogicError}


def find_library(explicit=None) -> Path:
    if explicit:
        return Path(explicit).resolve()
    if os.environ.get("TVARA_LIBRARY"):
        return Path(os.environ["TVARA_LIBRARY"]).resolve()
    for mode in ("release", "debug"):
        candidate = ROOT / "build" / mode / "libtvara_capi.so"
        if candidate.exists():
            return candidate
    raise FileNotFoundError("Build libtvara_capi (python -m tvara_amd.build) or set TVARA_LIBRARY")


_lib = None


def lib(explicit=None):
    global _lib
    if _lib is None or explicit:
        handle = C.CDLL(str(find_library(explicit)))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        if explicit:
            return handle
        _lib = handle
    return _lib


MODEL_EXPORTS = ("tvara_last_error", "tvara_model_open", "tvara_model_close", "tvara_model_vocab_size",
                 "tvara_model_context_size", "tvara_model_metadata", "tvara_sequence_create", "tvara_sequence_decode",
                 "tvara_sequence_drop", "tvara_sequence_decode_batch", "tvara_sequence_truncate")


def model_lib(explicit=None):
    """A library with the 11 model-level exports bound (this one by default, or
    any build of that ABI given by path)."""
    if not explicit:
        return lib()
    handle = C.CDLL(str(Path(explicit).resolve()))
    for name in MODEL_EXPORTS:
        fn = getattr(handle, name)
        fn.restype, fn.argtypes = SIGNATURES[name]
    return handle


def bind_subset(path):
    """Any build that exports part of this ABI (the CPU test harness of the
    ledger and prefix-cache exports): binds the names it has."""
    handle = C.CDLL(str(Path(path).resolve()))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(handle, name, None)
        if fn is not None:
            fn.restype = restype
            fn.argtypes = argtypes
    return handle


def last_error(library=None) -> str:
    msg = (library or lib()).tvara_last_error()
    return msg.decode("utf-8", errors="replace") if msg else "native operation failed"


def check(rc: int, library=None) -> None:
    if rc != OK:
        raise _ERRORS.get(rc, NativeError)(last_error(library))


def raise_last(library=None):
    """Raise for a failed NULL- or 0-returning call."""
    library = library or lib()
    raise _ERRORS.get(library.tvara_last_status(), NativeError)(last_error(library))
