"""plm_gemm_noalloc (no workspace, no allocation: a fixed device scratch array) against
plm_gemm with a workspace, through the C ABI: bit for bit, on two calls in a row, the
second with a smaller input, for shapes that split K on the decode kernel and on the MFMA
kernel; and a call needing more scratch than the fixed array is refused."""

import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as O
from pulsarlm_amd import _lib, ops
from tests._util import to_dev

pytestmark = pytest.mark.gpu


def _weights(n, k, seed):
    rng = np.random.default_rng(seed)
    packed = rng.integers(-(2**31), 2**31, size=(n, k // 8), dtype=np.int64).astype(np.int32)
    s = (np.abs(rng.standard_normal((n, k // 128))) * 0.02 + 1e-3).astype(np.float16)
    return ops.repack_int4_marlin_cuda(to_dev(packed), to_dev(s), 1, 128)


def _call(fn, x, w, sc, n, k, y, *tail):
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    rc = getattr(lib, fn)(_lib.PLM_INT4, x.data_ptr(), _lib.PLM_BF16, w.data_ptr(), sc.data_ptr(), _lib.PLM_FP16,
                          x.shape[0], n, k, 1, 128, y.data_ptr(), *tail, stream)
    return rc


def _with_workspace(x, w, sc, n, k):
    lib = _lib.load()
    need = lib.plm_gemm_workspace_bytes(_lib.PLM_INT4, x.shape[0], n, k)
    ws = torch.zeros(max(need, 1), dtype=torch.uint8, device="cuda")
    y = torch.empty((x.shape[0], n), dtype=torch.bfloat16, device="cuda")
    _lib.check(_call("plm_gemm", x, w, sc, n, k, y, ws.data_ptr(), ws.numel()))
    return y


@pytest.mark.parametrize("case", [
    # (n, k, first M, second M): decode kernel with a K split across workgroups
    (4096, 12288, 16, 5),
    # MFMA kernel with a K split (fewer work tiles than CUs)
    (4096, 4096, 256, 100),
])
def test_noalloc_matches_workspace_entry_point(case):
    n, k, m1, m2 = case
    lib = _lib.load()
    assert 0 < lib.plm_gemm_workspace_bytes(_lib.PLM_INT4, m1, n, k) <= (32 << 20)
    print(f"noalloc case {case}", flush=True)
    w, sc = _weights(n, k, seed=n + k)
    for m, seed in ((m1, 1), (m2, 2)):
        x = to_dev(O.bf16_round(np.random.default_rng(seed).standard_normal((m, k)).astype(np.float32)),
                   torch.bfloat16)
        y = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device="cuda")
        _lib.check(_call("plm_gemm_noalloc", x, w, sc, n, k, y))
        ref = _with_workspace(x, w, sc, n, k)
        torch.cuda.synchronize()
        assert torch.equal(y, ref), f"M={m}"


def test_noalloc_rejects_calls_beyond_its_scratch():
    lib = _lib.load()
    n, k, m = 4096, 12288, 1024
    assert lib.plm_gemm_workspace_bytes(_lib.PLM_INT4, m, n, k) > (32 << 20)
    w, sc = _weights(n, k, seed=3)
    x = torch.zeros((m, k), dtype=torch.bfloat16, device="cuda")
    y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    assert _call("plm_gemm_noalloc", x, w, sc, n, k, y) == _lib.PLM_ERR_INVALID
    assert b"gemm_int4_marlin: " in lib.plm_last_error() and b"fixed" in lib.plm_last_error()
