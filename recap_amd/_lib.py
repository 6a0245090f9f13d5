"""ctypes binding of librecap_hip.so (the C ABI declared in include/recap_hip.h).

The library is loaded on first use and never replaced by a fallback: if it is missing or
stale, every entry point raises.  Build it with ``python -m recap_amd.build_lib``.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "librecap_hip.so"
ABI_VERSION = 8

RECAP_OK, RECAP_EINVAL, RECAP_EUNSUPPORTED, RECAP_EHIP = 0, 1, 2, 3
RECAP_F16, RECAP_BF16 = 1, 2
CLOSURE_ROT, CLOSURE_CVK, CLOSURE_SCATTER = 1, 2, 4
CAPTURE_NOALLOC_MAX_PAIRS = 1 << 19  # RECAP_CAPTURE_NOALLOC_MAX_PAIRS
PAGER_TIMING = 1  # RECAP_PAGER_TIMING

_P, _I64, _I, _F = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float
_STRIDES = [_I64, _I64, _I64]

# name -> (restype, argtypes), exactly the prototypes of include/recap_hip.h
SIGNATURES: dict[str, tuple] = {
    "recap_abi_version": (_I, []),
    "recap_last_error": (ctypes.c_char_p, []),
    "recap_hilbert_permutation": (_I, [_I64, _I64, _I64, _P]),
    "recap_pool_blocks": (_I, [_P, _I, _I64, _I64, _I64, *_STRIDES, _P, _I64, _I64, _P, _P]),
    "recap_kv_pack": (_I, [_P, _P, _I, _I64, _I64, _I64, *_STRIDES, *_STRIDES, _P, _I64, _I64,
                           _P, _P, _P, _P, _P]),
    "recap_block_scores": (_I, [_P, _P, _I64, _I64, _I64, _F, _P, _P]),
    "recap_pool_select_workspace_size": (_I64, [_I64, _I64, _I64]),
    "recap_pool_select": (_I, [_P, _I, _I64, _I64, _I64, *_STRIDES, _P, _I64, _I64, _P, _F,
                               ctypes.c_double, _P, _I64, _P, _P, _P]),
    "recap_topk_blocks": (_I, [_P, _I64, _I64, _I64, _I, _P, _P]),
    "recap_kernel_block_mask": (_I, [_P, _I64, _I64, _I64, _P, _P]),
    "recap_mask_overlap": (_I, [_P, _P, _I64, _P, _P]),
    "recap_closure_groups": (_I64, [_I64, _I64]),
    "recap_closure_stats": (_I, [_P, _P, _P, _I, _P, _P, _I64, _I64, _I64, _I64, _I64, _I, _P,
                                 _P, _P, _P]),
    "recap_partial_reduce": (_I, [_P, _I64, _I64, _I64, _F, _P, _P]),
    "recap_symmetric_eigen": (_I, [_P, _I64, _I64, _P, _P, _P]),
    "recap_coarse_tables": (_I, [_P, _P, _P, _I, _I64, _I64, _I64, _I64, _P, _P, _P, _P]),
    "recap_basis_tables": (_I, [_P, _P, _I, _I64, _I64, _P, _P, _P, _P, _P]),
    "recap_coarse_w_width": (_I64, [_I, _I64, _I64]),
    "recap_coarse_tail": (_I, [_P, _I, _I64, _I64, _I64, *_STRIDES, _P, _P, _P, _P, _P, _P, _P,
                               _I64, _I64, _F, _F, _I64, _P, _P, _P, _P, _P]),
    "recap_drift_center": (_I, [_P, _I64, _I64, _P, _P]),
    "recap_block_sparse_attn": (_I, [_P, _I, _I64, _I64, _I64, *_STRIDES, _P, _P, _P, _P, _I64,
                                     _F, _P, _P, _P]),
    "recap_dense_attn": (_I, [_P, _I, _I64, _I64, _I64, *_STRIDES, _P, _P, _P, _I64, _F, _P,
                              *_STRIDES, _P, _P]),
    "recap_dense_head_attn": (_I, [_P, _I, _I64, _I64, _I64, *_STRIDES, _P, _P, _P, _P, _I64, _F,
                                   _P, *_STRIDES, _P, _P, _P, _P, _P]),
    "recap_sparse_merge_attn": (_I, [_P, _I, _I64, _I64, _I64, *_STRIDES, _P, _P, _P, _P, _I64,
                                     _I64, _F, _P, _P, _P, _P, _P, _P, _F, _P, *_STRIDES, _P, _P]),
    "recap_attn_queue_words": (_I64, []),
    "recap_capture_partials": (_I64, [_I64, _I64, _I64]),
    "recap_refresh_capture": (_I, [_P, _I, _I64, _I64, _I64, *_STRIDES, _P, _P, _P, _P, _P, _P,
                                   _I64, _I64, _P, _P, _P, _P, _P, _P, _P]),
    "recap_refresh_capture_noalloc": (_I, [_P, _I, _I64, _I64, _I64, *_STRIDES, _P, _P, _P,
                                           _P, _P, _P, _I64, _I64, _P, _P, _P, _P, _P, _P]),
    "recap_pager_create": (_I, [_I64, ctypes.c_int32, _P, ctypes.c_int32, ctypes.c_int32,
                                _P]),
    "recap_pager_destroy": (_I, [_P]),
    "recap_pager_bind": (_I, [_P, ctypes.c_int32, _P]),
    "recap_pager_reserve": (_I, [_P, _I64]),
    "recap_pager_stage_in": (_I, [_P, _I64, ctypes.c_int32, _P]),
    "recap_pager_prefetch": (_I, [_P, _I64, ctypes.c_int32]),
    "recap_pager_stage_out": (_I, [_P, _I64, ctypes.c_int32, _P]),
    "recap_pager_acquire": (_I, [_P, ctypes.c_int32, _P]),
    "recap_pager_release": (_I, [_P, ctypes.c_int32, _P]),
    "recap_pager_finish": (_I, [_P]),
    "recap_pager_stored": (_I, [_P, _I64]),
    "recap_pager_host_bytes": (_I64, [_P]),
    "recap_pager_counts": (_I, [_P, _P]),
    "recap_pager_copy_time": (_I, [_P, _P, _P]),
    "recap_pager_resize": (_I, [_P, _P, ctypes.c_int32]),
    "recap_bank_copy_async": (_I, [_P, _P, _I64, _P]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class RecapLibraryError(RuntimeError):
    """The native library is missing, stale or failed a HIP call."""


def load() -> ctypes.CDLL:
    """Load and bind the library once; raise if it is absent or of another ABI."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RecapLibraryError(
                f"{LIB_PATH} is missing: build it with `python -m recap_amd.build_lib` "
                "(hipcc --offload-arch=gfx950); there is no fallback implementation")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        version = lib.recap_abi_version()
        if version != ABI_VERSION:
            raise RecapLibraryError(f"librecap_hip.so ABI {version} != expected {ABI_VERSION}")
        _lib = lib
        return lib


def call(name: str, *args) -> int:
    """Call an entry point and map a non-zero status to a Python exception."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != RECAP_OK:
        message = lib.recap_last_error().decode(errors="replace")
        if rc == RECAP_EINVAL:
            raise ValueError(f"{name}: {message}")
        raise RecapLibraryError(f"{name} failed ({rc}): {message}")
    return rc
