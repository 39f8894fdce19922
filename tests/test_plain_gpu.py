"""Parity of the non-repacked int4 GEMM (plm_gemm_int4_plain; gemm_int4_cuda and
gemm_int4_split_cuda of pulsarlm-core/inc/pulsarlm/kernels/ops.hpp:272-297) with the CPU
oracle: W = round(fp32(q * scale)) (int4_gemm.cu:136-138). The reference has no test of
its own for these ops; the checks follow test_marlin.cpp's: identity-GEMM exactness and
the dequantize-then-matmul tolerance (elementwise 2e-2 + 2e-2 |ref|, rel-L2 <= 5e-3), plus
split invariance."""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from pulsarlm_amd import _host, ops
from tests._util import TDT, assert_close, to_dev, to_np, x_case

pytestmark = pytest.mark.gpu


def _case(n, k, g, seed):
    rng = np.random.default_rng(seed)
    q = rng.integers(-8, 8, size=(n, k))
    s = (rng.random((n, k // g)) * 0.1 + 0.01).astype(np.float32)
    return O.pack_int4(q), s


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
@pytest.mark.parametrize("n,k,g", [(200, 144, 16), (72, 256, 128), (33, 1040, 16)])
def test_identity_gemm_exact(dtype, n, k, g):
    packed, s = _case(n, k, g, seed=n)
    ref = O.dequant_int4_plain(packed, s, g, dtype)
    eye = torch.eye(k, dtype=TDT[dtype], device="cuda")
    w, sc = to_dev(packed), to_dev(s)
    assert np.array_equal(to_np(ops.gemm_int4_cuda(eye, w, sc, g)), ref.T)
    for r0, rows in [(0, 16), (k - 16, 16), (37, 1), (70, 5)]:
        y = ops.gemm_int4_cuda(eye[r0:r0 + rows].contiguous(), w, sc, g)
        assert np.array_equal(to_np(y), ref.T[r0:r0 + rows]), (r0, rows)


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
@pytest.mark.parametrize("m", [1, 5, 16, 64, 100, 300])
@pytest.mark.parametrize("n,k,g", [(200, 144, 16), (520, 1024, 128), (4096, 4096, 128)])
def test_gemm_matches_oracle(dtype, m, n, k, g):
    packed, s = _case(n, k, g, seed=m + n)
    x = x_case(m, k, dtype, seed=m)
    y = ops.gemm_int4_cuda(to_dev(x, TDT[dtype]), to_dev(packed), to_dev(s), g)
    assert y.shape == (m, n) and y.dtype == TDT[dtype]
    assert_close(y, O.gemm_ref(x, O.dequant_int4_plain(packed, s, g, dtype), None), f"m={m}")


def test_split_invariance_and_determinism():
    n, k, g, m = 300, 2048, 128, 24
    packed, s = _case(n, k, g, seed=1)
    x = to_dev(x_case(m, k, "bf16", seed=2), torch.bfloat16)
    ref = O.gemm_ref(to_np(x), O.dequant_int4_plain(packed, s, g), None)
    w, sc = to_dev(packed), to_dev(s)
    for splits in (1, 2, 3, 7, 16, 40):  # 40 > the 16 K tiles: empty splits contribute zero
        y = ops.gemm_int4_split_cuda(x, w, sc, g, splits)
        assert_close(y, ref, f"splits={splits}")
        assert torch.equal(y, ops.gemm_int4_split_cuda(x, w, sc, g, splits))


def test_host_layer_and_errors():
    n, k, g, m = 200, 144, 16, 7
    packed, s = _case(n, k, g, seed=3)
    x = to_dev(x_case(m, k, "bf16", seed=3), torch.bfloat16)
    w, sc = to_dev(packed), to_dev(s)
    assert torch.equal(_host.gemm_int4_cuda(x, w, sc, g), ops.gemm_int4_cuda(x, w, sc, g))
    assert torch.equal(_host.gemm_int4_split_cuda(x, w, sc, g, 3), ops.gemm_int4_split_cuda(x, w, sc, g, 3))
    with pytest.raises(RuntimeError, match="gemm_int4"):
        _host.gemm_int4_split_cuda(x, w, sc, g, 0)
    with pytest.raises(RuntimeError, match="gemm_int4"):
        _host.gemm_int4_cuda(x, w, sc, 32)  # scale shape does not match the group size
    assert _host.gemm_int4_cuda(x[:0], w, sc, g).shape == (0, n)
