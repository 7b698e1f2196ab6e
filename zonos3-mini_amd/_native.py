"""ctypes binding of ``libzonos3_gdn.so`` (the C ABI declared in ``include/zonos3_gdn.h``).

The library is loaded after ``torch`` so that it binds to the HIP runtime torch already loaded (both carry
the soname ``libamdhip64.so.7``); device pointers and streams then come straight from torch tensors.
There is no fallback: a missing or unloadable library raises ``RuntimeError``.
"""

from __future__ import annotations

import ctypes
from ctypes import POINTER, c_char_p, c_float, c_int, c_int32, c_long, c_size_t, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libzonos3_gdn.so"

# dtype codes (enum zgdn_dtype)
F32, BF16 = 0, 1
# status codes (enum zgdn_status)
OK, EINVAL, EHIP, EUNSUPPORTED = 0, 1, 2, 3
# bits of the chunked path's device status word (zgdn_chunk_status)
STATUS_WAIT_GAVE_UP = 1
ABI_VERSION = 2  # zgdn_abi_version() of the library these signatures describe

_P = c_void_p
_I32P = POINTER(c_int32)

# name -> (restype, argtypes); one entry per function of include/zonos3_gdn.h
SIGNATURES: dict[str, tuple] = {
    "zgdn_last_error": (c_char_p, []),
    "zgdn_abi_version": (c_int, []),
    "zgdn_recurrent_fwd": (
        c_int,
        [_P, _P, _P, c_int, _P, _P, c_int, _P, _P, c_int, _P, _P, _P, c_int, _P, c_int,
         c_int, c_int, c_int, c_int, c_int, c_int, c_float, _P],
    ),
    "zgdn_chunk_workspace_size": (c_size_t, [c_int, c_int]),
    "zgdn_chunk_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    "zgdn_gemm_nt": (c_int, [_P, c_long, _P, _P, c_long, c_int, c_int, c_int, c_int, _P]),
    "zgdn_in_proj_conv": (c_int, [_P, c_long, _P, _P, c_long, c_int, c_int, c_int, _P, c_int, _P, _P, c_int, _P]),
    "zgdn_chunk_set_launch_form": (c_int, [c_int]),
    "zgdn_chunk_get_launch_form": (c_int, []),
    "zgdn_chunk_status": (c_int, [POINTER(c_int), c_int]),
    "zgdn_chunk_status_async": (c_int, [_P, _P]),
    "zgdn_chunk_overlap_queues": (c_int, [c_int, c_int]),
    "zgdn_chunk_set_wait_limit": (c_int, [c_int, c_int]),
    "zgdn_chunk_segment_workspace_size": (c_size_t, [c_int, c_int, c_int]),
    "zgdn_chunk_fwd": (
        c_int,
        [_P, _P, _P, c_int, _P, _P, c_int, _P, _P, c_int, _P, _P, _P, _P, _P, c_int, c_int,
         c_int, c_int, c_int, c_int, c_int, c_int, c_long, c_long, c_long, c_long, c_int, c_float, _P, c_size_t,
         _P],
    ),
    "zgdn_chunk_noalloc_max_bytes": (c_size_t, []),
    "zgdn_chunk_fwd_noalloc": (
        c_int,
        [_P, _P, _P, c_int, _P, _P, c_int, _P, _P, c_int, _P, _P, _P, _P, _P, c_int, c_int,
         c_int, c_int, c_int, c_int, c_int, c_int, c_long, c_long, c_long, c_long, c_int, c_float, _P],
    ),
    "zgdn_fused_decode_step": (
        c_int,
        [_P, _P, _P, _P, c_int, _P, _P, _P, _P, _P, _P, _P,
         c_int, c_int, c_int, c_int, c_int, c_int, c_float, c_float, c_int, _P],
    ),
    "zgdn_serving_decode_step": (
        c_int,
        [_P, c_long, _P, c_int, c_int, _P, c_int, c_int, c_int, c_int, c_int, c_int, c_int,
         _P, _P, _P, _P, _P, _P, _P, c_int, _P, _P, _P, _P, c_float, c_float, c_int, _P],
    ),
    "zgdn_attnres_route": (
        c_int,
        [POINTER(c_void_p), c_int, c_int, c_int, c_long, c_int, _P, c_float, _P, _P],
    ),
    "zgdn_causal_conv1d_fwd": (
        c_int,
        [_P, _P, _P, c_int, _P, _P, c_int, _P, _P, _P, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_long,
         _P],
    ),
    "zgdn_l2norm_fwd": (c_int, [_P, c_int, _P, c_int, _P, c_int, c_int, c_int, c_long, c_float, _P]),
    "zgdn_sigmoid_fwd": (c_int, [_P, c_int, _P, c_int, c_size_t, c_float, _P]),
    "zgdn_gated_rmsnorm_fwd": (c_int, [_P, _P, _P, c_int, _P, _P, c_int, c_int, c_int, c_long, c_float, _P]),
    "zgdn_accent_workspace_size": (c_size_t, [c_int, c_int, c_int, c_int]),
    "zgdn_accent_shift": (
        c_int,
        [_P, c_long, _P, _P, _P, c_long, _P, c_long, _P, c_long, c_int, c_int, c_int, c_int, c_int, _P, c_size_t, _P],
    ),
}

_lib: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """The loaded library (raises RuntimeError when it is not built or cannot be loaded)."""
    global _lib
    if _lib is None:
        import torch  # noqa: F401  -- load torch's HIP runtime first

        if not LIB_PATH.exists():
            raise RuntimeError(
                f"gated-DeltaNet HIP library not built ({LIB_PATH} missing); run `python zonos3-mini_amd/build.py`"
            )
        try:
            handle = ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_GLOBAL)
        except OSError as exc:
            raise RuntimeError(f"cannot load {LIB_PATH}: {exc}") from exc
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        if handle.zgdn_abi_version() != ABI_VERSION:
            raise RuntimeError("libzonos3_gdn.so ABI version mismatch; rebuild it")
        _lib = handle
    return _lib


def call(name: str, *args) -> None:
    """Call entry point ``name``; a non-zero status raises RuntimeError with the library's message."""
    status = getattr(lib(), name)(*args)
    if status != OK:
        msg = lib().zgdn_last_error().decode(errors="replace")
        raise RuntimeError(msg or f"{name} failed with status {status}")
