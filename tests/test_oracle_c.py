"""The oracle's C restatement of the int4 dequant (oracle/dequant.c, the host baseline's
dequant) against the numpy oracle and the committed golden fixture, bit for bit. CPU only."""

import os

import numpy as np
import pytest

from oracle import build_c
from oracle import oracle as O
from oracle import oracle_c as C

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module", autouse=True)
def _built():
    build_c.build()  # gcc, well under a second


def test_matches_golden_fixture():
    g = np.load(os.path.join(GOLDEN, "marlin_n200_k144_g16.npz"))
    got = C.dequant_int4(g["packed"], g["scale_int4"], 1, 16, "bf16")
    assert np.array_equal(O.bf16_bits(got), g["dequant_int4_bf16"])


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
@pytest.mark.parametrize("sdt", [np.float16, np.float32, "bf16"])
@pytest.mark.parametrize("block_n,g", [(1, 16), (1, 128), (128, 32), (3, 48)])
@pytest.mark.parametrize("threads", [1, 4])
def test_matches_numpy_oracle(dtype, sdt, block_n, g, threads):
    rng = np.random.default_rng(block_n * 1000 + g)
    n, k = 131, 384
    packed = rng.integers(-2**31, 2**31, size=(n, k // 8), dtype=np.int64).astype(np.int32)
    # Scale exponents from fp16-subnormal territory to near its overflow, so that both the
    # scale rounding and the product rounding hit subnormal, normal and overflowing cases.
    mag = np.abs(rng.standard_normal((-(-n // block_n), k // g))) * np.exp2(rng.integers(-24, 14, (-(-n // block_n), k // g)))
    if sdt == "bf16":
        scale = O.bf16_round(mag.astype(np.float32))
        raw = (scale.view(np.uint32) >> 16).astype(np.uint16)
        got = C.dequant_int4(packed, raw, block_n, g, dtype, threads=threads, scale_is_bf16=True)
    else:
        scale = mag.astype(sdt)
        got = C.dequant_int4(packed, scale, block_n, g, dtype, threads=threads)
    with np.errstate(over="ignore"):
        ref = O.dequant_int4(packed, scale, block_n, g, dtype)
    assert np.array_equal(got, ref, equal_nan=True)


def test_rejects_bad_shapes():
    with pytest.raises(ValueError):
        C.dequant_int4(np.zeros((4, 2), np.int32), np.ones((4, 3), np.float16), 1, 5)
