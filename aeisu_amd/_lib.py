"""ctypes binding of ``libaeisu_amd.so`` (declared in include/aeisu_amd.h).

torch is imported first so that the library's ``libamdhip64.so.7`` dependency
resolves to the HIP runtime torch already loaded: one HIP runtime per process,
so torch device pointers and streams are valid in the library.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import torch  # noqa: F401  (must precede the CDLL load, see module docstring)

LIB_PATH = Path(__file__).resolve().parent / "libaeisu_amd.so"

AEISU_OK = 0
AEISU_ERR_INVALID_ARGUMENT = -1
AEISU_ERR_ARTIFACT = -2
AEISU_ERR_HIP = -3
AEISU_ERR_STATE = -4
AEISU_ERR_NONFINITE = -5
PRECISION = {"fp16": 1, "mixed": 2, "int8": 3, "mixed-fp8mma": 4, "fp32": 5}
LAYOUT_F16, LAYOUT_F32 = 0, 1
FLAG_KEEP_INTERMEDIATES, FLAG_STAGE_TIMING, FLAG_NO_PAD, FLAG_UNFUSED, FLAG_BODY_TILE24 = 1, 2, 4, 8, 16
FLAG_BODY_NO_EXCHANGE, FLAG_BODY_EXCHANGE_FALLBACK = 32, 64
BUF_SKIP, BUF_LOW0, BUF_WORK, BUF_META = 0, 1, 6, 7
STAGES = ("project", "compress", "bottleneck", "expand", "refine_tail", "head", "total")

_P, _I, _U, _S = ctypes.c_void_p, ctypes.c_int, ctypes.c_uint, ctypes.c_size_t
SIGNATURES = {
    "aeisu_create_from_file": (_I, [ctypes.c_char_p, _I, ctypes.POINTER(_P)]),
    "aeisu_create_from_memory": (_I, [_P, _S, _I, ctypes.POINTER(_P)]),
    "aeisu_create_sibling": (_I, [_P, ctypes.POINTER(_P)]),
    "aeisu_shares_weights": (_I, [_P, _P]),
    "aeisu_configure": (_I, [_P, _I, _I, _I, _I, _I, _I, _U]),
    "aeisu_upscale_noalloc": (_I, [_P, _I, _I, _I, _I, _I, _P, _P, _P]),
    "aeisu_startup_report": (_S, [_P, ctypes.c_char_p, _S]),
    "aeisu_upscale_async": (_I, [_P, _P, _P, _P]),
    "aeisu_upscale": (_I, [_P, _P, _P, _P]),
    "aeisu_upscale_graph": (_I, [_P, _P, _P, _P]),
    "aeisu_controller_async": (_I, [_P, _P, _P, _P]),
    "aeisu_head_async": (_I, [_P, _P, _P, _P, _P]),
    "aeisu_check_finite": (_I, [_P, _P]),
    "aeisu_copy_intermediate": (_I, [_P, _I, _P, _S, _P]),
    "aeisu_intermediate_bytes": (_S, [_P, _I]),
    "aeisu_geometry": (_I, [_P, ctypes.POINTER(_I)]),
    "aeisu_stage_timings": (_I, [_P, ctypes.POINTER(ctypes.c_float), ctypes.POINTER(_I)]),
    "aeisu_reset_timings": (_I, [_P]),
    "aeisu_persistent_bytes": (_S, [_P]),
    "aeisu_artifact_checksum": (_I, [_P, ctypes.c_char_p]),
    "aeisu_destroy": (None, [_P]),
    "aeisu_last_error": (ctypes.c_char_p, []),
    "aeisu_version": (ctypes.c_char_p, []),
}

_lib = None


def lib() -> ctypes.CDLL:
    """Load the native library; raises if it has not been built (there is no fallback path)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH.name} is not built; run `python -m aeisu_amd.build` "
                               "(the HIP path has no CPU fallback)")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
    return _lib


class AeisuError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code


def check(rc: int) -> None:
    if rc != AEISU_OK:
        msg = lib().aeisu_last_error().decode(errors="replace")
        if rc == AEISU_ERR_NONFINITE:
            raise FloatingPointError(msg or "Non-finite model reconstruction")
        if rc == AEISU_ERR_INVALID_ARGUMENT:
            raise ValueError(msg)
        raise AeisuError(rc, msg)
