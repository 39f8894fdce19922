"""The C++ host layer (pulsarlm_amd/_host.so) on the CPU: it loads, exposes the
reference's operator names, and rejects bad arguments with the reference's
"<op>: ..." messages before any device work."""

import pytest
import torch

from pulsarlm_amd import _host

REFERENCE_OPS = ["repack_int4_marlin_cuda", "repack_fp8_marlin_cuda", "gemm_int4_marlin_cuda", "gemm_fp8_marlin_cuda"]


def test_reference_operator_names():
    for name in REFERENCE_OPS:
        assert callable(getattr(_host, name))
    assert hasattr(_host, "linear") and hasattr(_host.linear, "int4") and hasattr(_host.linear, "fp8")


def test_cpu_tensors_are_rejected():
    with pytest.raises(RuntimeError, match="gemm_int4_marlin: all inputs must be CUDA tensors"):
        _host.gemm_int4_marlin_cuda(torch.zeros(2, 128), torch.zeros(8, dtype=torch.int32), torch.zeros(1), 64, 1, 128)
    with pytest.raises(RuntimeError, match="repack_int4_marlin: weight_packed must be int32"):
        _host.repack_int4_marlin_cuda(torch.zeros(4, 4), torch.zeros(4, 1), 1, 32)
    with pytest.raises(RuntimeError, match="repack_fp8_marlin: weight must be float8_e4m3fn"):
        _host.repack_fp8_marlin_cuda(torch.zeros(4, 4), torch.zeros(4, 1), 1, 16)


def test_dense_linear_runs_on_cpu():
    w = torch.randn(8, 16)
    x = torch.randn(3, 2, 16)
    y = _host.linear.dense(w).apply(x)
    assert torch.allclose(y, x @ w.T)
