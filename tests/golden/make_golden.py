"""Writes the committed golden fixtures (tests/golden/*.npz) from the CPU oracle.

The reference commits no golden vectors for this path (its tests draw unseeded
random tensors on the device, pulsarlm-core/tests/kernels/test_marlin.cpp), so
these fixtures are seeded inputs with the oracle's expected outputs at the
reference test's shape (n=200, k=144, g=16) and a slice of benchmark config 1.
They pin the oracle and the GPU path against regressions.

    python tests/golden/make_golden.py
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as O  # noqa: E402


def marlin_shape():
    rng = np.random.default_rng(20250101)
    n, k, g, m = 200, 144, 16, 16
    q = rng.integers(-8, 8, size=(n, k))
    packed = O.pack_int4(q)
    scale_int4 = (rng.random((n, k // g)) * 0.1 + 0.01).astype(np.float32)
    codes = rng.integers(0, 256, (n, k), dtype=np.uint8)
    codes[(codes == 0x7F) | (codes == 0xFF)] = 0
    scale_fp8 = (rng.random((-(-n // 128), k // g)) * 0.1 + 0.01).astype(np.float32)
    x = O.bf16_round(rng.standard_normal((m, k)).astype(np.float32))
    w4 = O.dequant_int4(packed, scale_int4, 1, g)
    w8 = O.dequant_fp8(codes, scale_fp8, 128, g)
    np.savez_compressed(
        os.path.join(HERE, "marlin_n200_k144_g16.npz"),
        packed=packed, scale_int4=scale_int4, codes=codes, scale_fp8=scale_fp8, x=x,
        dequant_int4_bf16=O.bf16_bits(w4), dequant_fp8_bf16=O.bf16_bits(w8),
        y_int4=O.gemm_ref(x, w4, None), y_fp8=O.gemm_ref(x, w8, None),
        plm_int4=O.plm_layout_int4(packed), marlin_int4=O.marlin_encode_int4(packed))


def config1_slice():
    x, packed, scale = O.make_w4a16(16, 4096, 4096, 128, seed=1)
    cols = slice(0, 64)  # first 64 output columns of config 1
    w = O.dequant_int4(packed[cols], scale[cols], 1, 128)
    np.savez_compressed(os.path.join(HERE, "config1_m16_k4096_n64.npz"), x=x, packed=packed[cols],
                        scale=scale[cols], y=O.gemm_ref(x, w, None))


if __name__ == "__main__":
    marlin_shape()
    config1_slice()
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))
