"""The C ABI (include/pulsarlm_amd.h) on the CPU: the library loads, exports
every declared symbol, sizes agree with the layout, and argument errors are
reported with the op's name before any device work (no GPU needed)."""

import ctypes
import re
from pathlib import Path

import pytest

from pulsarlm_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "pulsarlm_amd.h"


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const char\*|int64_t|int)\s+(plm_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_symbols()
    assert len(names) >= 14
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(_lib.exported_symbols())


def test_version_and_error_are_strings():
    lib = _lib.load()
    assert b"gfx950" in lib.plm_version()
    assert isinstance(lib.plm_last_error(), bytes)


def test_sizes():
    lib = _lib.load()
    assert lib.plm_weight_bytes(_lib.PLM_INT4, 4096, 4096) == 4096 * 4096 // 2
    assert lib.plm_weight_bytes(_lib.PLM_FP8, 4096, 4096) == 4096 * 4096
    assert lib.plm_weight_bytes(_lib.PLM_INT4, 200, 144) == 13 * 2 * 1024
    assert lib.plm_scale_bytes(4096, 4096, 1, 128, _lib.PLM_FP16) == 4096 * 32 * 2
    assert lib.plm_scale_bytes(4096, 4096, 128, 128, _lib.PLM_FP32) == 256 * 32 * 4
    assert lib.plm_scale_bytes(200, 144, 1, 16, _lib.PLM_FP32) == 13 * 16 * 16 * 4
    assert lib.plm_scale_bytes(200, 144, 1, 24, _lib.PLM_FP32) == -1
    assert lib.plm_gemm_workspace_bytes(_lib.PLM_INT4, 0, 4096, 4096) == 0


@pytest.mark.parametrize("args,msg", [
    ((_lib.PLM_INT4, 16, 4096, 4096, 1, 24), b"gemm_int4_marlin: group_size must be a positive multiple of 16"),
    ((_lib.PLM_FP8, 16, 4096, 4000, 1, 128), b"gemm_fp8_marlin: K must be a multiple of group_size"),
    ((_lib.PLM_INT4, 16, 4096, 4096, 0, 128), b"gemm_int4_marlin: block_n must be positive"),
])
def test_gemm_argument_errors(args, msg):
    lib = _lib.load()
    fmt, m, n, k, bn, g = args
    dummy = ctypes.c_void_p(16)
    rc = lib.plm_gemm(fmt, dummy, _lib.PLM_BF16, dummy, dummy, _lib.PLM_FP16, m, n, k, bn, g, dummy, None, 0, None)
    assert rc == _lib.PLM_ERR_INVALID
    assert lib.plm_last_error() == msg


def test_gemm_rejects_fp32_x_and_unaligned_x():
    lib = _lib.load()
    d = ctypes.c_void_p(256)
    rc = lib.plm_gemm(_lib.PLM_INT4, d, _lib.PLM_FP32, d, d, _lib.PLM_FP16, 4, 64, 128, 1, 128, d, None, 0, None)
    assert rc == _lib.PLM_ERR_INVALID and lib.plm_last_error() == b"gemm_int4_marlin: x must be fp16 or bf16"
    rc = lib.plm_gemm(_lib.PLM_INT4, ctypes.c_void_p(258), _lib.PLM_BF16, d, d, _lib.PLM_FP16, 4, 64, 128, 1, 128, d,
                      None, 0, None)
    assert rc == _lib.PLM_ERR_INVALID and b"16-byte aligned" in lib.plm_last_error()


def test_empty_gemm_is_ok_without_device_work():
    lib = _lib.load()
    rc = lib.plm_gemm(_lib.PLM_INT4, None, _lib.PLM_BF16, None, None, _lib.PLM_FP16, 0, 64, 128, 1, 128, None, None, 0,
                      None)
    assert rc == _lib.PLM_OK


def test_repack_argument_errors():
    lib = _lib.load()
    d = ctypes.c_void_p(256)
    rc = lib.plm_repack_int4(d, d, _lib.PLM_FP16, 64, 100, 1, 16, d, d, None)
    assert rc == _lib.PLM_ERR_INVALID
    assert lib.plm_last_error() == b"repack_int4_marlin: K must be a multiple of group_size"
    rc = lib.plm_repack_fp8(d, d, 7, 64, 128, 1, 16, d, d, None)
    assert lib.plm_last_error() == b"repack_fp8_marlin: scale dtype must be bf16, fp16 or fp32"
