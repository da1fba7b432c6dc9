"""ctypes binding of ``libqsa_hip.so`` (the C ABI declared in include/qsa_hip.h).

The library is built in-tree by ``qsa_vllm_amd.build``. Loading fails loudly
when it is missing: there is no CPU or eager fallback for any entry point.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

_LIB_PATH = Path(__file__).resolve().parent / "libqsa_hip.so"
_lock = threading.Lock()
_lib = None

QSA_OK = 0
QSA_ERR_WORKSPACE = -4
SPARSE_ATTENTION_SCRATCH_BYTES = 32 << 20  # QSA_SPARSE_ATTENTION_SCRATCH_BYTES
ABI_VERSION = 3

c_i32 = ctypes.c_int
c_i64 = ctypes.c_int64
c_size = ctypes.c_size_t
c_ptr = ctypes.c_void_p

# name -> (restype, argtypes); mirrors include/qsa_hip.h exactly.
SIGNATURES = {
    "qsa_last_error": (ctypes.c_char_p, []),
    "qsa_abi_version": (c_i32, []),
    "qsa_topk_workspace_bytes": (c_size, [c_i32, c_i32, c_i32]),
    "qsa_topk": (c_i32, [c_ptr, c_i64, c_i32, c_i32, c_ptr, c_ptr, c_i64, c_i32,
                         c_ptr, c_size, c_ptr]),
    "qsa_topk_expand": (c_i32, [c_ptr, c_i64, c_i32, c_i32,
                                c_ptr, c_ptr,
                                c_ptr, c_i32,
                                c_ptr,
                                c_ptr, c_i64, c_i32,
                                c_ptr, c_i64, c_i64,
                                c_i32, c_ptr, c_i32, c_i32,
                                c_i32, c_i32,
                                c_ptr, c_size, c_ptr]),
    "qsa_indexer_prepare": (c_i32, [c_ptr, c_i64, c_i32,
                                    c_ptr, c_i64,
                                    c_ptr, c_ptr,
                                    c_ptr, c_i32, ctypes.c_float,
                                    c_ptr,
                                    c_ptr, c_i64,
                                    c_i64, c_i32, c_i32,
                                    c_ptr, c_ptr,
                                    c_i64, c_ptr,
                                    c_ptr, c_i32,
                                    c_ptr, c_i64,
                                    c_i64, c_i32, c_i32,
                                    c_ptr, c_ptr, c_i32,
                                    c_ptr, c_i64,
                                    c_i64,
                                    c_ptr, c_i64,
                                    c_i64,
                                    c_ptr, c_i64,
                                    c_i64, c_i64,
                                    c_ptr, c_i64,
                                    c_i64,
                                    c_i64,
                                    c_ptr, c_i32, c_i32,
                                    c_i32, c_i32, c_i32,
                                    c_i32, c_i32, c_i32,
                                    c_ptr]),
    "qsa_indexer_norm_rope": (c_i32, [c_ptr, c_i64, c_i64,
                                      c_i32, c_i32, c_i32, c_ptr,
                                      c_ptr, c_i64,
                                      c_ptr, c_i32, ctypes.c_float, c_i32,
                                      c_ptr, c_ptr]),
    "qsa_store_cache_rows": (c_i32, [c_ptr, c_i64, c_i64,
                                     c_i32, c_i32, c_i32,
                                     c_ptr, c_ptr, c_i64,
                                     c_i32, c_ptr]),
    "qsa_compress_groups": (c_i32, [c_ptr, c_i64,
                                    c_ptr, c_i64,
                                    c_i64, c_ptr,
                                    c_i64, c_i64, c_i32,
                                    c_i32, c_ptr,
                                    c_i64, c_i64,
                                    c_i64, c_ptr,
                                    c_i64, c_ptr,
                                    c_ptr, c_i32,
                                    c_ptr, c_ptr,
                                    c_i32, c_i32, c_i32, c_ptr,
                                    c_i64, c_ptr,
                                    c_i64, c_i64,
                                    c_ptr]),
    "qsa_expand_block_indices": (c_i32, [c_ptr, c_i64,
                                         c_i64, c_i32, c_i32, c_i32,
                                         c_ptr, c_ptr,
                                         c_i32, c_ptr,
                                         c_ptr, c_i64, c_i32,
                                         c_ptr, c_i64,
                                         c_i64, c_i32, c_ptr,
                                         c_i32, c_i32, c_i32, c_i32,
                                         c_ptr]),
    "qsa_indexer_decode": (c_i32, [c_ptr, c_i64, c_i64,
                                   c_i32, c_i32, c_i32, c_ptr,
                                   c_i64, c_i64,
                                   c_i32, c_i32, c_ptr,
                                   c_i64, c_i32,
                                   c_ptr, c_i32, c_ptr,
                                   c_i64, c_i32, c_ptr]),
    "qsa_indexer_prefill": (c_i32, [c_ptr, c_i64, c_i64,
                                    c_i32, c_i32, c_ptr,
                                    c_i64, c_i64,
                                    c_i32, c_i32, c_ptr,
                                    c_i64, c_i32, c_i32,
                                    c_ptr, c_ptr,
                                    c_i32, c_i32, c_i32,
                                    c_ptr, c_i64, c_i32,
                                    c_ptr]),
    "qsa_indexer_prefill_span_rows": (c_i32, [c_i32, c_i64]),
    "qsa_sparse_attention_splits": (c_i32, [c_i32, c_i32, c_i32, c_i32, c_i32, c_i32]),
    "qsa_sparse_attention_workspace_bytes": (c_size, [c_i32, c_i32, c_i32, c_i32]),
    "qsa_sparse_attention": (c_i32, [c_ptr, c_i64, c_i64, c_i32, c_i32, c_i32,
                                     c_ptr, c_i64, c_i64, c_i64,
                                     c_ptr, c_i64, c_i64, c_i64,
                                     c_i32, c_i32, c_i32,
                                     c_ptr, c_i64, c_i32,
                                     c_ptr, c_i64, c_i32, c_i32,
                                     c_ptr, c_ptr,
                                     c_ptr, c_i64, c_i64,
                                     c_ptr, c_i64, c_i64, c_i64,
                                     c_i32, c_i32,
                                     c_ptr, c_size, c_ptr]),
    "qsa_decode_select_attention_fuses": (c_i32, [c_i32, c_i32, c_i32, c_i32, c_i32, c_i32,
                                                  c_i32]),
    "qsa_decode_select_attention_workspace_bytes": (c_size, [c_i32, c_i32, c_i32, c_i32, c_i32,
                                                             c_i32, c_i32]),
    "qsa_decode_select_attention": (c_i32, [c_ptr, c_i64, c_i32, c_i32, c_ptr, c_ptr,
                                            c_ptr, c_i32, c_ptr, c_ptr, c_i64, c_i32, c_i32,
                                            c_ptr, c_i64, c_i32, c_ptr,
                                            c_ptr, c_i64, c_i64, c_i32, c_i32,
                                            c_ptr, c_i64, c_i64, c_i64,
                                            c_ptr, c_i64, c_i64, c_i64,
                                            c_i32, c_i32, c_i32,
                                            c_ptr, c_i64, c_i64,
                                            c_ptr, c_i64, c_i64, c_i64,
                                            c_i32, c_ptr, c_size, c_ptr]),
    "qsa_sparse_attention_noalloc": (c_i32, [c_ptr, c_i64, c_i64, c_i32, c_i32, c_i32,
                                             c_ptr, c_i64, c_i64, c_i64,
                                             c_ptr, c_i64, c_i64, c_i64,
                                             c_i32, c_i32, c_i32,
                                             c_ptr, c_i64, c_i32,
                                             c_ptr, c_i64, c_i32, c_i32,
                                             c_ptr, c_ptr,
                                             c_ptr, c_i64, c_i64,
                                             c_ptr, c_i64, c_i64, c_i64,
                                             c_i32, c_i32, c_ptr]),
    "qsa_sparse_attention_merge": (c_i32, [c_ptr, c_ptr, c_i32, c_i32, c_i32, c_i32,
                                           c_ptr, c_i64, c_i64,
                                           c_ptr, c_i64, c_i64, c_i64,
                                           c_ptr]),
    "qsa_gated_norm": (c_i32, [c_ptr, c_i64, c_ptr, c_i64, c_ptr, c_i64,
                               c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_i64,
                               c_i32, c_i32, c_i32, ctypes.c_float, c_ptr, c_size, c_ptr]),
    "qsa_gated_norm_workspace_bytes": (c_size, [c_i32, c_i32]),
    "qsa_silu_mul": (c_i32, [c_ptr, c_i64, c_ptr, c_i64, c_i32, c_i32, c_ptr]),
    "qsa_gdn_prep": (c_i32, [c_ptr, c_i64, c_ptr, c_i64, c_ptr, c_ptr, c_i32,
                             c_ptr, c_ptr, c_ptr, c_i32, c_ptr, c_ptr,
                             c_i32, c_i32, c_i32, c_i32, c_i32,
                             c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr]),
    "qsa_gdn_conv_state": (c_i32, [c_ptr, c_i64, c_i32, c_ptr, c_i32, c_ptr, c_ptr, c_i32,
                                   c_i32, c_i32, c_i32, c_i32, c_ptr]),
    "qsa_gdn_recurrence": (c_i32, [c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_i32, c_ptr, c_i32,
                                   c_ptr, c_ptr, c_i32, c_i32, c_i32, c_i32, c_i32, c_ptr,
                                   c_ptr]),
    "qsa_gdn_gated_norm": (c_i32, [c_ptr, c_ptr, c_i64, c_ptr, ctypes.c_float, c_i32, c_i32,
                                   c_i32, c_i32, c_ptr, c_ptr]),
}


class QSAError(RuntimeError):
    """A C-ABI entry point returned a non-zero status."""


def library_path() -> Path:
    return _LIB_PATH


def load() -> ctypes.CDLL:
    """Load ``libqsa_hip.so`` once; raise if it is missing or has the wrong ABI."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not _LIB_PATH.exists():
            raise QSAError(
                f"{_LIB_PATH} is missing: build it with `python -m qsa_vllm_amd.build` "
                "(the QSA path has no fallback without its HIP library)")
        lib = ctypes.CDLL(os.fspath(_LIB_PATH))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        if lib.qsa_abi_version() != ABI_VERSION:
            raise QSAError(f"{_LIB_PATH} has ABI {lib.qsa_abi_version()}, expected {ABI_VERSION}")
        _lib = lib
        return lib


def check(status: int, what: str) -> None:
    if status != QSA_OK:
        msg = load().qsa_last_error().decode("utf-8", "replace")
        raise QSAError(f"{what} failed with status {status}: {msg}")


def call(name: str, *args) -> int:
    """Call entry point ``name`` and raise QSAError on a non-zero status."""
    fn = getattr(load(), name)
    status = fn(*args)
    check(status, name)
    return status
