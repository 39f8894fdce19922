"""Shared helpers for the parity tests: seeded inputs (numpy, from the oracle's
generators) moved to the GPU, and the oracle comparisons."""

from __future__ import annotations

import numpy as np
import torch

from oracle import oracle as O

TDT = {"bf16": torch.bfloat16, "fp16": torch.float16}


def to_dev(a: np.ndarray, dtype=None, device="cuda") -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.to(device)


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def int4_case(n, k, g, block_n=1, seed=0, scale_dtype=np.float16, scale_kind="baseline"):
    """q uniform [-8, 7] packed LSB-first, scales per the benchmark spec (|N(0,.02)|+1e-3) or the
    reference test's rand*0.1+0.01 (test_marlin.cpp:23-25)."""
    rng = np.random.default_rng(seed)
    q = rng.integers(-8, 8, size=(n, k))
    rows = -(-n // block_n)
    if scale_kind == "baseline":
        s = np.abs(rng.standard_normal((rows, k // g)) * 0.02) + 1e-3
    else:
        s = rng.random((rows, k // g)) * 0.1 + 0.01
    return O.pack_int4(q), s.astype(scale_dtype)


def fp8_case(n, k, g, block_n=1, seed=0, scale_dtype=np.float32):
    """Every e4m3 code except the NaNs (test_marlin.cpp:32-36), scales rand*0.1+0.01."""
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 256, (n, k), dtype=np.uint8)
    codes[(codes == 0x7F) | (codes == 0xFF)] = 0
    rows = -(-n // block_n)
    s = (rng.random((rows, k // g)) * 0.1 + 0.01).astype(scale_dtype)
    return codes, s


def scale_tensor(s: np.ndarray) -> torch.Tensor:
    if s.dtype == np.float16:
        return to_dev(s)
    if s.dtype == np.float32:
        return to_dev(s)
    raise ValueError(s.dtype)


def x_case(m, k, dtype="bf16", seed=0):
    rng = np.random.default_rng(1000 + seed)
    x = rng.standard_normal((m, k)).astype(np.float32)
    return O.round_to(x, dtype)


def assert_close(y: torch.Tensor, ref: np.ndarray, what=""):
    ok, st = O.check_close(to_np(y), ref)
    assert ok, f"{what}: {st}"
    return st
