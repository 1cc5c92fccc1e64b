"""ctypes binding of libmt_flce.so (declarations: include/mt_flce.h).

There is no fallback: if the library is missing or does not match the header
version, every entry point raises.  Nothing here touches the GPU at import.
"""
from __future__ import annotations

import ctypes
from ctypes import c_float, c_int, c_int64, c_size_t, c_void_p, c_char_p, POINTER
from pathlib import Path

import os

# MT_FLCE_LIB: another build of the same library (the sanitized host-only
# build of the CPU tests); unset in production.
LIB_PATH = Path(os.environ.get("MT_FLCE_LIB") or Path(__file__).resolve().parent / "libmt_flce.so")
ABI_VERSION = 7

MT_DTYPE_F32 = 0
MT_DTYPE_BF16 = 1

MT_OK = 0
STATUS_NAMES = {
    1: "MT_ERR_INVALID_ARGUMENT",
    2: "MT_ERR_WORKSPACE_TOO_SMALL",
    3: "MT_ERR_UNSUPPORTED",
    4: "MT_ERR_HIP",
}

# name -> (restype, argtypes); mirrors include/mt_flce.h
SIGNATURES = {
    "mt_flce_abi_version": (c_int, []),
    "mt_flce_last_error": (c_char_p, []),
    "mt_flce_prepare": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_int, c_void_p, c_void_p,
                                c_void_p, c_void_p]),
    "mt_flce_forward_workspace_bytes": (c_size_t, [c_int64, c_int64, c_int64, c_int64, c_int]),
    "mt_flce_forward": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64, c_int64,
                                c_int, c_float, c_void_p, c_void_p, c_int64, c_void_p, c_void_p,
                                c_void_p, c_size_t, c_void_p]),
    "mt_flce_forward_keep": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64,
                                     c_int64, c_int, c_float, c_void_p, c_void_p, c_int64,
                                     c_void_p, c_void_p, c_void_p, c_size_t, c_void_p, c_int64,
                                     c_size_t, c_void_p, c_void_p]),
    "mt_flce_noalloc_scratch_bytes": (c_size_t, []),
    "mt_flce_max_buffer_bytes": (ctypes.c_uint64, []),
    "mt_flce_forward_noalloc": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64,
                                        c_int64, c_int, c_float, c_void_p, c_void_p, c_int64,
                                        c_void_p, c_void_p, c_void_p]),
    "mt_flce_backward_plan": (c_int, [c_int64, c_int64, c_int64, c_int64, c_int, c_size_t,
                                      POINTER(c_int64), POINTER(c_int64), POINTER(c_size_t)]),
    "mt_flce_backward_narrow_plan": (c_int, [c_int64, c_int64, c_int64, c_int64, c_int, c_size_t,
                                            POINTER(c_int64), POINTER(c_int64),
                                            POINTER(c_size_t)]),
    "mt_flce_backward": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64, c_int64,
                                 c_int, c_float, c_void_p, c_void_p, c_int64, c_void_p, c_void_p,
                                 c_int64, c_void_p, c_int64, c_void_p, c_int64, c_int, c_int64,
                                 c_int64, c_void_p, c_size_t, c_void_p]),
    "mt_flce_fused_plan": (c_int, [c_int64, c_int64, c_int64, c_int64, c_int, c_size_t, c_int,
                                   POINTER(c_int64), POINTER(c_size_t), POINTER(c_int)]),
    "mt_flce_fused": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64, c_int64,
                              c_int, c_float, c_void_p, c_void_p, c_int64, c_void_p, c_int64,
                              c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_int64, c_int,
                              c_int64, c_void_p, c_size_t, c_void_p]),
    "mt_flce_backward_tiles": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64,
                                       c_int64, c_int, c_float, c_void_p, c_void_p, c_int64,
                                       c_void_p, c_void_p, c_int64, c_void_p, c_int64, c_void_p,
                                       c_size_t, c_void_p, c_size_t, c_int, c_int64, c_int64,
                                       c_void_p, c_size_t, c_void_p]),
    "mt_flce_backward_narrow": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64,
                                        c_int64, c_int, c_float, c_void_p, c_void_p, c_int64,
                                        c_void_p, c_void_p, c_int64, c_void_p, c_int64, c_void_p,
                                        c_size_t, c_void_p, c_size_t, c_int64, c_int64, c_void_p,
                                        c_size_t, c_void_p, c_void_p]),
    "mt_flce_narrow_scratch_bytes": (c_size_t, [c_int64, c_int64, c_int64]),
    "mt_flce_dw_tiles_layout": (c_int, [c_int64, c_int64, POINTER(c_size_t), POINTER(c_int64),
                                        POINTER(c_size_t)]),
    "mt_flce_fused_tiles": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64,
                                    c_int64, c_int, c_float, c_void_p, c_void_p, c_int64,
                                    c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_int64,
                                    c_void_p, c_size_t, c_void_p, c_size_t, c_int, c_int64,
                                    c_void_p, c_size_t, c_void_p]),
    "mt_flce_narrow_tiles": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p, c_size_t, c_int64,
                                     c_int64, c_void_p]),
    "mt_segment_sum": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_int, c_void_p, c_int64,
                               c_void_p, c_void_p, c_void_p, c_void_p]),
    "mt_flce_scale_grads": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int, c_void_p,
                                    c_int64, c_int64, c_void_p, c_int64, c_int, c_void_p]),
    "mt_flce_profile_enable": (c_int, [c_int]),
    "mt_flce_profile_report": (c_int, [c_char_p, c_size_t, POINTER(c_size_t)]),
    "mt_flce_probe_mfma": (c_int, [c_int, c_int64, ctypes.c_int32, c_void_p, c_void_p, c_void_p]),
    "mt_ce_forward": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_int, c_void_p, c_int64,
                              c_void_p, c_void_p, c_void_p]),
    "mt_ce_backward": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_int, c_void_p, c_int64,
                               c_void_p, c_void_p, c_int64, c_void_p, c_int64, c_void_p]),
}

_lib = None


class FlceError(RuntimeError):
    """A non-zero status from libmt_flce.so."""


def load() -> ctypes.CDLL:
    """Load (once) and type the library; raise if it is missing or mismatched."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise FlceError(
            f"{LIB_PATH} is not built: the fused linear-CE path has no fallback. "
            "Build it with `python -m mini_trainer_amd.build` (hipcc, gfx950)."
        )
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    v = lib.mt_flce_abi_version()
    if v != ABI_VERSION:
        raise FlceError(f"{LIB_PATH} ABI version {v} != expected {ABI_VERSION}")
    _lib = lib
    return lib


def check(status: int, what: str) -> None:
    if status != MT_OK:
        msg = load().mt_flce_last_error().decode(errors="replace")
        raise FlceError(f"{what}: {STATUS_NAMES.get(status, status)}: {msg}")


def exported_symbols() -> list[str]:
    return list(SIGNATURES)
