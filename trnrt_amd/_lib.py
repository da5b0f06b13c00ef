"""ctypes binding of libdsa_gfx950.so (the C ABI declared in include/dsa_gfx950.h).

The library is loaded once, on first use, from the package directory. There is no fallback: if the library is not
built the first call raises RuntimeError, the reference's behaviour when its kernel backend is missing
(trnrt/kernels/dsa_index.py:258-259).

torch is imported before the library is opened. torch ships its own HIP runtime under the soname libamdhip64.so.7,
the soname the library links against: with torch loaded first the library binds to that runtime, while a library
opened first would pull in ROCm's copy and the later torch import a second one, two HIP runtimes in one process
(which crashes on the GPU).
"""

from __future__ import annotations

import ctypes
from ctypes import c_float, c_int, c_size_t, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libdsa_gfx950.so"

DSA_OK = 0
DSA_EINVAL = -1
DSA_EUNSUPPORTED = -2
DSA_EWORKSPACE = -3
DSA_ELAUNCH = -4
DSA_ESCRATCH = -5
NOALLOC_SCRATCH_BYTES = 32 << 20

DSA_WS_TOPK = 1
DSA_WS_ATTENTION = 2
DSA_WS_LAYER = 3

ABI_VERSION = 10

P = c_void_p
# Every entry point of include/dsa_gfx950.h with its ctypes signature (restype, argtypes).
SIGNATURES: dict[str, tuple] = {
    "dsa_abi_version": (c_int, []),
    "dsa_strerror": (ctypes.c_char_p, [c_int]),
    "dsa_indexer_decode": (c_int, [P, P, P, P, P, P, P, P, c_int, c_int, c_int, c_int, c_int, c_int, c_int, P]),
    "dsa_indexer_decode_bf16": (c_int, [P, P, P, P, P, P, P, c_int, c_int, c_int, c_int, c_int, c_int, c_int, P]),
    "dsa_indexer_prefill": (c_int, [P, P, P, P, P, P, c_int, c_int, c_int, c_int, c_int, c_float, P]),
    "dsa_pool_slots": (c_int, [P, P, P, P, P, c_int, P, P, c_int, c_int, c_int, c_int, c_int, c_int, P]),
    "dsa_pool_keys_write": (c_int, [P, c_int, P, c_int, P, P, P, c_int, c_int, P, P, c_int, c_int, c_int,
                                    ctypes.c_longlong, P]),
    "dsa_cache_write": (c_int, [P, c_int, P, P, P, c_int, c_int, ctypes.c_longlong, c_int, c_float, P]),
    "dsa_indexer_prefill_fp8": (c_int, [P, P, P, P, P, P, P, c_int, c_int, c_int, c_int, c_int, c_float, P]),
    "dsa_topk": (c_int, [P, P, P, P, P, c_size_t, c_int, c_int, c_int, c_int, c_int, P]),
    "dsa_topk_supported": (c_int, [c_int, c_int, c_int]),
    "dsa_workspace_clear": (c_int, [P, c_size_t, P]),
    "dsa_topk_mask": (c_int, [P, P, P, P, c_int, c_int, c_int, c_int, c_int, P]),
    "dsa_sparse_mla_decode": (
        c_int,
        [P, P, P, P, P, P, P, P, P, P, P, P, c_size_t, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int,
         c_float, c_int, P],
    ),
    "dsa_sparse_mla_slots_n": (
        c_int,
        [P, P, P, P, P, P, P, P, P, P, c_size_t, c_int, c_int, c_int, c_int, ctypes.c_longlong, c_float, c_int, P],
    ),
    "dsa_token_rows": (c_int, [P, P, P, P, P, c_int, c_int, c_int, c_int, c_int, P]),
    "dsa_compact_mask": (c_int, [P, c_int, c_int, c_int, P, P, P]),
    "dsa_value_order": (c_int, [P, P, P, c_int, c_int, P, P, P]),
    "dsa_slots_compact_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    "dsa_sparse_mla_slots_compact": (
        c_int,
        [P, P, P, P, P, P, P, P, P, c_size_t, c_int, c_int, c_int, c_int, c_int, ctypes.c_longlong, c_float, c_int,
         P],
    ),
    "dsa_decode_layer": (
        c_int,
        [P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, c_size_t, c_int, c_int, c_int, c_int, c_int, c_int, c_int,
         c_int, c_int, c_float, c_int, P],
    ),
    "dsa_decode_layer_chain": (
        c_int,
        [P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, c_size_t, c_int, c_int, c_int, c_int, c_int, c_int, c_int,
         c_int, c_int, c_float, c_int, P],
    ),
    "dsa_decode_layer_noalloc": (
        c_int,
        [P, P, P, P, P, P, P, P, P, P, P, P, P, P, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int,
         c_float, c_int, P],
    ),
    "dsa_pooled_decode_layer": (
        c_int,
        [P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, c_size_t, c_int, c_int, c_int, c_int, c_int, c_int, c_int,
         c_int, c_int, c_float, c_int, P],
    ),
    "dsa_pooled_decode_layer_chain": (
        c_int,
        [P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, c_size_t, c_int, c_int, c_int, c_int, c_int, c_int, c_int,
         c_int, c_int, c_float, c_int, P],
    ),
    "dsa_pooled_decode_step": (
        c_int,
        [P, c_int, P, c_int, P, P] + [P] * 15 + [c_size_t, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int,
                                                  c_int, c_float, c_int, P],
    ),
    "dsa_pooled_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int, c_int]),
    "dsa_sparse_mla_pooled": (
        c_int,
        [P, P, P, P, P, P, P, P, P, P, P, P, c_size_t, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_int,
         c_float, c_int, P],
    ),
    "dsa_sparse_mla_pooled_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    "dsa_prefill_select": (
        c_int,
        [P, P, P, P, P, P, P, P, P, P, P, c_size_t, c_int, c_int, c_int, c_int, c_int, c_int, c_float, c_int, P],
    ),
    "dsa_prefill_select_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int, c_int]),
    "dsa_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int, c_int]),
    "dsa_default_splits": (c_int, [c_int, c_int, c_int]),
    "dsa_layer_status": (c_int, [P, P, P, c_int, P]),
    "dsa_timing_begin": (c_int, [P, c_int]),
    "dsa_timing_end": (c_int, []),
    "dsa_timing_kernel_name": (ctypes.c_char_p, [c_int]),
}

_lib = None


def lib() -> ctypes.CDLL:
    """The loaded library (RuntimeError if it is not built or its ABI version differs)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH.name} is not built: run `python -m trnrt_amd.build` (needs hipcc, gfx950)")
        import torch  # noqa: F401  (its HIP runtime first: one runtime per process)

        h = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            f = getattr(h, name)
            f.restype = res
            f.argtypes = args
        if h.dsa_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH.name}: ABI version {h.dsa_abi_version()}, expected {ABI_VERSION}")
        _lib = h
    return _lib


def check(status: int, what: str) -> None:
    """Raises the reference's exception kind for a non-zero status (ValueError for bad arguments,
    NotImplementedError for unsupported shapes, RuntimeError for launch failures)."""
    if status == DSA_OK:
        return
    msg = f"{what}: {lib().dsa_strerror(status).decode()}"
    if status in (DSA_EINVAL, DSA_EWORKSPACE, DSA_ESCRATCH):
        raise ValueError(msg)
    if status == DSA_EUNSUPPORTED:
        raise NotImplementedError(msg)
    raise RuntimeError(msg)


def layer_status(workspace_ptr: int | None, stream_ptr: int, clear: bool = False) -> tuple[int, int]:
    """(barrier waits that gave up, rows selected in the two-exchange form) counted in a decode workspace since its
    last clear (workspace_ptr None: the allocation-free entry point's scratch on the current device). Synchronises
    the stream."""
    gave_up, two = ctypes.c_int32(0), ctypes.c_int32(0)
    check(lib().dsa_layer_status(workspace_ptr, ctypes.byref(gave_up), ctypes.byref(two), int(clear), stream_ptr),
          "dsa_layer_status")
    return int(gave_up.value), int(two.value)


def workspace_bytes(kind: int, B: int, H: int, keep: int, max_len: int, splits: int = 0) -> int:
    return int(lib().dsa_workspace_bytes(kind, B, H, keep, max_len, splits))
