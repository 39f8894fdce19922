"""plm_gemm_noalloc (no workspace, no allocation: a fixed device scratch array) against
plm_gemm with a workspace, through the C ABI: bit for bit, on two calls in a row, the
second with a smaller input, for int4 and fp8 shapes that split K on the decode kernel and
on the MFMA kernel; its first call on the device made inside a HIP graph capture (fresh
process) and the graph replayed; and a call needing more scratch than the fixed array is
refused."""

import os
import subprocess
import sys
import textwrap

import numpy as np
import pytest
import torch

from oracle import oracle as O
from pulsarlm_amd import _lib, ops
from tests._util import fp8_case, to_dev

pytestmark = pytest.mark.gpu


def _weights(n, k, seed):
    rng = np.random.default_rng(seed)
    packed = rng.integers(-(2**31), 2**31, size=(n, k // 8), dtype=np.int64).astype(np.int32)
    s = (np.abs(rng.standard_normal((n, k // 128))) * 0.02 + 1e-3).astype(np.float16)
    return ops.repack_int4_marlin_cuda(to_dev(packed), to_dev(s), 1, 128)


def _fp8_weights(n, k, seed):
    codes, s = fp8_case(n, k, 128, 128, seed=seed)
    return ops.repack_fp8_marlin_cuda(to_dev(codes).view(torch.float8_e4m3fn), to_dev(s), 128, 128)


# format -> (C enum, scale dtype enum, block_n)
_FMT = {"int4": (_lib.PLM_INT4, _lib.PLM_FP16, 1), "fp8": (_lib.PLM_FP8, _lib.PLM_FP32, 128)}


def _call(fn, x, w, sc, n, k, y, *tail, fmt="int4"):
    lib = _lib.load()
    f, sdt, bn = _FMT[fmt]
    stream = torch.cuda.current_stream().cuda_stream
    rc = getattr(lib, fn)(f, x.data_ptr(), _lib.PLM_BF16, w.data_ptr(), sc.data_ptr(), sdt,
                          x.shape[0], n, k, bn, 128, y.data_ptr(), *tail, stream)
    return rc


def _with_workspace(x, w, sc, n, k, fmt="int4"):
    lib = _lib.load()
    need = lib.plm_gemm_workspace_bytes(_FMT[fmt][0], x.shape[0], n, k)
    ws = torch.zeros(max(need, 1), dtype=torch.uint8, device="cuda")
    y = torch.empty((x.shape[0], n), dtype=torch.bfloat16, device="cuda")
    _lib.check(_call("plm_gemm", x, w, sc, n, k, y, ws.data_ptr(), ws.numel(), fmt=fmt))
    return y


@pytest.mark.parametrize("case", [
    # (format, n, k, first M, second M): decode kernel with a K split across workgroups
    ("int4", 4096, 12288, 16, 5),
    # MFMA kernel with a K split (fewer work tiles than CUs)
    ("int4", 4096, 4096, 256, 100),
    # fp8 weights, 128 x 128 block scales: decode kernel with a K split, then the MFMA kernel
    ("fp8", 5120, 17408, 16, 7),
    ("fp8", 2048, 4096, 256, 64),
])
def test_noalloc_matches_workspace_entry_point(case):
    fmt, n, k, m1, m2 = case
    lib = _lib.load()
    assert 0 < lib.plm_gemm_workspace_bytes(_FMT[fmt][0], m1, n, k) <= (32 << 20)
    print(f"noalloc case {case}", flush=True)
    w, sc = (_weights if fmt == "int4" else _fp8_weights)(n, k, seed=n + k)
    for m, seed in ((m1, 1), (m2, 2)):
        x = to_dev(O.bf16_round(np.random.default_rng(seed).standard_normal((m, k)).astype(np.float32)),
                   torch.bfloat16)
        y = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device="cuda")
        _lib.check(_call("plm_gemm_noalloc", x, w, sc, n, k, y, fmt=fmt))
        ref = _with_workspace(x, w, sc, n, k, fmt=fmt)
        torch.cuda.synchronize()
        assert torch.equal(y, ref), f"M={m}"


# Run in a fresh process so that the first plm_gemm_noalloc call on the device (the scratch
# set-up: symbol lookup and counter clear) happens inside the capture.
_CAPTURE_SCRIPT = textwrap.dedent("""
    import sys
    import numpy as np
    import torch
    sys.path.insert(0, {root!r})
    from tests import test_zz_no_alloc as T
    from pulsarlm_amd import _lib
    torch.cuda.init()
    n, k = 4096, 12288
    w, sc = T._weights(n, k, seed=11)
    xs = [torch.randn(m, k, device="cuda").to(torch.bfloat16) for m in (16, 3)]
    ys = [torch.full((x.shape[0], n), float("nan"), dtype=torch.bfloat16, device="cuda") for x in xs]
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for x, y in zip(xs, ys):
                _lib.check(T._call("plm_gemm_noalloc", x, w, sc, n, k, y))
    torch.cuda.synchronize()
    refs = [T._with_workspace(x, w, sc, n, k) for x in xs]
    torch.cuda.synchronize()
    for rep in range(3):
        for y in ys:
            y.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for i, (y, r) in enumerate(zip(ys, refs)):
            assert torch.equal(y, r), f"replay {{rep}} call {{i}}"
        # eager work between replays, on the same scratch
        y2 = torch.empty_like(ys[0])
        _lib.check(T._call("plm_gemm_noalloc", xs[0], w, sc, n, k, y2))
        torch.cuda.synchronize()
        assert torch.equal(y2, refs[0]), f"eager after replay {{rep}}"
    print("CAPTURE_OK", flush=True)
""")


def test_noalloc_first_call_inside_graph_capture():
    lib = _lib.load()
    assert lib.plm_gemm_workspace_bytes(_lib.PLM_INT4, 16, 4096, 12288) > 0  # the decode kernel splits K
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    print("noalloc first call under capture (subprocess)", flush=True)
    res = subprocess.run([sys.executable, "-c", _CAPTURE_SCRIPT.format(root=root)], capture_output=True, text=True,
                         timeout=110, cwd=root)
    assert res.returncode == 0 and "CAPTURE_OK" in res.stdout, res.stdout[-2000:] + res.stderr[-3000:]


def test_noalloc_rejects_calls_beyond_its_scratch():
    lib = _lib.load()
    n, k, m = 4096, 12288, 1024
    assert lib.plm_gemm_workspace_bytes(_lib.PLM_INT4, m, n, k) > (32 << 20)
    w, sc = _weights(n, k, seed=3)
    x = torch.zeros((m, k), dtype=torch.bfloat16, device="cuda")
    y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    assert _call("plm_gemm_noalloc", x, w, sc, n, k, y) == _lib.PLM_ERR_INVALID
    assert b"gemm_int4_marlin: " in lib.plm_last_error() and b"fixed" in lib.plm_last_error()
