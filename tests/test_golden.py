"""Committed golden fixtures (tests/golden/make_golden.py): the oracle must still
reproduce them (CPU), and the HIP path must match them (GPU)."""

import os

import numpy as np
import pytest
import torch

from oracle import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return dict(np.load(os.path.join(GOLDEN, name), allow_pickle=False))


def test_oracle_reproduces_marlin_fixture():
    f = load("marlin_n200_k144_g16.npz")
    w4 = O.dequant_int4(f["packed"], f["scale_int4"], 1, 16)
    w8 = O.dequant_fp8(f["codes"], f["scale_fp8"], 128, 16)
    assert np.array_equal(O.bf16_bits(w4), f["dequant_int4_bf16"])
    assert np.array_equal(O.bf16_bits(w8), f["dequant_fp8_bf16"])
    assert np.array_equal(O.plm_layout_int4(f["packed"]), f["plm_int4"])
    assert np.array_equal(O.marlin_encode_int4(f["packed"]), f["marlin_int4"])
    assert np.allclose(O.gemm_ref(f["x"], w4, None), f["y_int4"], rtol=1e-6, atol=1e-6)


def test_oracle_reproduces_config1_fixture():
    f = load("config1_m16_k4096_n64.npz")
    w = O.dequant_int4(f["packed"], f["scale"], 1, 128)
    assert np.allclose(O.gemm_ref(f["x"], w, None), f["y"], rtol=1e-6, atol=1e-6)


@pytest.mark.gpu
def test_gpu_matches_golden():
    from pulsarlm_amd import ops

    f = load("marlin_n200_k144_g16.npz")
    dev = "cuda"
    w, s = ops.repack_int4_marlin_cuda(torch.from_numpy(f["packed"]).to(dev), torch.from_numpy(f["scale_int4"]).to(dev),
                                       1, 16)
    assert np.array_equal(w.cpu().numpy().view(np.uint32), f["plm_int4"])
    deq = ops.dequant_marlin_cuda("int4", w, s, 200, 144, 1, 16)
    assert np.array_equal(deq.view(torch.int16).cpu().numpy().view(np.uint16), f["dequant_int4_bf16"])
    x = torch.from_numpy(f["x"]).to(dev).to(torch.bfloat16)
    ok, st = O.check_close(ops.gemm_int4_marlin_cuda(x, w, s, 200, 1, 16).float().cpu().numpy(), f["y_int4"])
    assert ok, st
    w8, s8 = ops.repack_fp8_marlin_cuda(torch.from_numpy(f["codes"]).to(dev).view(torch.float8_e4m3fn),
                                        torch.from_numpy(f["scale_fp8"]).to(dev), 128, 16)
    ok, st = O.check_close(ops.gemm_fp8_marlin_cuda(x, w8, s8, 200, 128, 16).float().cpu().numpy(), f["y_fp8"])
    assert ok, st
    c = load("config1_m16_k4096_n64.npz")
    wc, sc = ops.repack_int4_marlin_cuda(torch.from_numpy(c["packed"]).to(dev), torch.from_numpy(c["scale"]).to(dev),
                                         1, 128)
    y = ops.gemm_int4_marlin_cuda(torch.from_numpy(c["x"]).to(dev).to(torch.bfloat16), wc, sc, 64, 1, 128)
    ok, st = O.check_close(y.float().cpu().numpy(), c["y"])
    assert ok, st
