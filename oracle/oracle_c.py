"""ctypes loader of the C restatement of the int4 dequant (oracle/dequant.c, built into
oracle/_c/liboracle_c.so by oracle/build_c.py). Test infrastructure only."""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "_c" / "liboracle_c.so"
_lib = None

_SCALE_DTYPES = {np.dtype(np.float16): 0, np.dtype(np.float32): 2}


def _load():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built: run python oracle/build_c.py")
        lib = ctypes.CDLL(str(LIB_PATH))
        lib.oracle_dequant_int4.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int64,
                                            ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int,
                                            ctypes.c_void_p, ctypes.c_int]
        lib.oracle_dequant_int4.restype = ctypes.c_int
        _lib = lib
    return _lib


def dequant_int4(packed, scale, block_n: int, group_size: int, dtype: str = "bf16", threads: int = 0,
                 scale_is_bf16: bool = False) -> np.ndarray:
    """Same rule and result as oracle.dequant_int4 (float32 [N, K] holding dtype-rounded
    values); scale is fp16, fp32, or (scale_is_bf16) bf16 bits stored as uint16."""
    p = np.ascontiguousarray(packed, dtype=np.int32)
    s = np.ascontiguousarray(scale)
    sd = 1 if scale_is_bf16 else _SCALE_DTYPES[s.dtype]
    n, kw = p.shape
    out = np.empty((n, kw * 8), np.float32)
    rc = _load().oracle_dequant_int4(p.ctypes.data, s.ctypes.data, sd, n, kw * 8, block_n, group_size,
                                     1 if dtype == "bf16" else 0, out.ctypes.data, threads)
    if rc != 0:
        raise ValueError("oracle_dequant_int4: bad shape or group size")
    return out
