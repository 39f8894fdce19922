"""ctypes binding of the C ABI declared in ``include/pulsarlm_amd.h``.

Loads the in-tree ``libpulsarlm_amd.so``; raises if it has not been built.
There is no fallback: every op in this package runs the HIP library.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libpulsarlm_amd.so"

PLM_OK, PLM_ERR_INVALID, PLM_ERR_HIP, PLM_ERR_WORKSPACE = 0, 1, 2, 3
PLM_BF16, PLM_FP16, PLM_FP32 = 0, 1, 2
PLM_INT4, PLM_FP8 = 0, 1

# name -> (restype, argtypes). Pointers are c_void_p; int64 sizes; enums as c_int.
_P, _I64, _INT, _SZ = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_size_t
SIGNATURES = {
    "plm_last_error": (ctypes.c_char_p, []),
    "plm_version": (ctypes.c_char_p, []),
    "plm_weight_bytes": (_I64, [_INT, _I64, _I64]),
    "plm_scale_bytes": (_I64, [_I64, _I64, _I64, _I64, _INT]),
    "plm_repack_int4": (_INT, [_P, _P, _INT, _I64, _I64, _I64, _I64, _P, _P, _P]),
    "plm_repack_fp8": (_INT, [_P, _P, _INT, _I64, _I64, _I64, _I64, _P, _P, _P]),
    "plm_convert_marlin": (_INT, [_INT, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _P]),
    "plm_dequant": (_INT, [_INT, _P, _P, _INT, _I64, _I64, _I64, _I64, _P, _INT, _P]),
    "plm_gemm_workspace_bytes": (_I64, [_INT, _I64, _I64, _I64]),
    "plm_gemm": (_INT, [_INT, _P, _INT, _P, _P, _INT, _I64, _I64, _I64, _I64, _I64, _P, _P, _SZ, _P]),
    "plm_gemm_noalloc": (_INT, [_INT, _P, _INT, _P, _P, _INT, _I64, _I64, _I64, _I64, _I64, _P, _P]),
    "plm_quantize_rows_e4m3": (_INT, [_P, _INT, _I64, _I64, _P, _P, _P]),
    "plm_gemm_w8a8_workspace_bytes": (_I64, [_I64, _I64, _I64]),
    "plm_gemm_w8a8": (_INT, [_P, _INT, _P, _P, _INT, _I64, _I64, _I64, _I64, _I64, _P, _P, _SZ, _P]),
    "plm_grouped_gemm": (_INT, [_INT, _P, _INT, _P, _P, _INT, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P, _SZ,
                                _P]),
    "plm_grouped_gemm_workspace_bytes": (_I64, [_I64, _I64]),
    "plm_moe_workspace_bytes": (_I64, [_I64, _I64, _I64, _I64, _I64]),
    "plm_gemm_int4_plain_workspace_bytes": (_I64, [_I64, _I64, _I64, _I64]),
    "plm_gemm_int4_plain": (_INT, [_P, _INT, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _SZ, _P]),
    "plm_route_top_k": (_INT, [_P, _INT, _I64, _I64, _I64, _I64, _P, _P, _P, _P]),
    "plm_silu_mul": (_INT, [_P, _INT, _I64, _I64, _P, _P]),
    "plm_moe": (_INT, [_P, _INT, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _INT, _I64, _P, _P, _P, _SZ,
                       _P]),
}

_lib = None


class PlmError(RuntimeError):
    pass


def load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is not built; run `python -m pulsarlm_amd.build` (hipcc, gfx950) first")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def reload_tuning() -> None:
    """Make the library re-read its PLM_* measurement knobs from the environment (it parses
    them once per process otherwise). An internal hook for tests, not part of the C ABI."""
    fn = load().plm_internal_reload_tuning
    fn.restype, fn.argtypes = None, []
    fn()


def check(rc: int) -> None:
    if rc != PLM_OK:
        msg = load().plm_last_error().decode()
        raise PlmError(msg or f"pulsarlm_amd call failed with status {rc}")


def exported_symbols() -> list[str]:
    return list(SIGNATURES)
