"""Parity of the HIP W4A16 / W8A16 path with the CPU oracle, through the C ABI.

Mirrors pulsarlm-core/tests/kernels/test_marlin.cpp (shape n=200, k=144, g=16;
identity-GEMM exactness; dequantize-then-matmul tolerance) and extends it to the
benchmark configs. Tolerance for every GEMM: elementwise |y - ref| <= 2e-2 +
2e-2 |ref| (the reference's allclose, test_marlin.cpp:95,113) and rel-L2 <= 5e-3
against the float64-accumulated dequantize-then-matmul of the reference's
dequantized weights."""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from pulsarlm_amd import ops
from tests._util import TDT, assert_close, fp8_case, int4_case, scale_tensor, to_dev, to_np, x_case

pytestmark = pytest.mark.gpu

N, K, G = 200, 144, 16  # test_marlin.cpp:15-17


def _repack_int4(packed, scale, block_n, g):
    return ops.repack_int4_marlin_cuda(to_dev(packed), scale_tensor(scale), block_n, g)


def _repack_fp8(codes, scale, block_n, g):
    w = to_dev(codes).view(torch.float8_e4m3fn)
    return ops.repack_fp8_marlin_cuda(w, scale_tensor(scale), block_n, g)


# ------------------------------------------------------------------ repack / dequant


@pytest.mark.parametrize("block_n", [1, 128])
@pytest.mark.parametrize("sdt", [np.float16, np.float32])
def test_repack_int4_bit_exact(block_n, sdt):
    packed, s = int4_case(N, K, G, block_n, seed=1, scale_dtype=sdt, scale_kind="test")
    w, sc = _repack_int4(packed, s, block_n, G)
    torch.cuda.synchronize()
    assert np.array_equal(w.cpu().numpy().view(np.uint32), O.plm_layout_int4(packed))
    assert np.array_equal(sc.cpu().numpy(), O.plm_layout_scale(s, N, K, block_n, G))


@pytest.mark.parametrize("block_n", [1, 128])
def test_repack_fp8_bit_exact(block_n):
    codes, s = fp8_case(N, K, G, block_n, seed=2)
    w, sc = _repack_fp8(codes, s, block_n, G)
    assert np.array_equal(w.cpu().numpy().view(np.uint8), O.plm_layout_fp8(codes))
    assert np.array_equal(sc.cpu().numpy(), O.plm_layout_scale(s, N, K, block_n, G))


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
@pytest.mark.parametrize("block_n", [1, 128])
@pytest.mark.parametrize("fmt", ["int4", "fp8"])
def test_dequant_bit_exact(fmt, dtype, block_n):
    if fmt == "int4":
        packed, s = int4_case(N, K, G, block_n, seed=3, scale_dtype=np.float32, scale_kind="test")
        w, sc = _repack_int4(packed, s, block_n, G)
        ref = O.dequant_int4(packed, s, block_n, G, dtype)
    else:
        codes, s = fp8_case(N, K, G, block_n, seed=3)
        w, sc = _repack_fp8(codes, s, block_n, G)
        ref = O.dequant_fp8(codes, s, block_n, G, dtype)
    got = ops.dequant_marlin_cuda(fmt, w, sc, N, K, block_n, G, TDT[dtype])
    assert np.array_equal(to_np(got), ref)


# ------------------------------------------------------------------ identity GEMM (exactness)


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
@pytest.mark.parametrize("block_n", [1, 128])
@pytest.mark.parametrize("fmt", ["int4", "fp8"])
@pytest.mark.parametrize("g", [16, 48, 32, 128])
def test_identity_gemm_exact(fmt, dtype, block_n, g):
    """test_marlin.cpp:54-78: y = I_k @ dequant(W)^T must equal dequant(W)^T exactly,
    through the MFMA path (M = K) and the decode path (16-row and 1-row slices)."""
    n, k = N, 144 if g in (16, 48) else 256
    if fmt == "int4":
        packed, s = int4_case(n, k, g, block_n, seed=4, scale_dtype=np.float32, scale_kind="test")
        w, sc = _repack_int4(packed, s, block_n, g)
        ref = O.dequant_int4(packed, s, block_n, g, dtype)
        gemm = ops.gemm_int4_marlin_cuda
    else:
        codes, s = fp8_case(n, k, g, block_n, seed=4)
        w, sc = _repack_fp8(codes, s, block_n, g)
        ref = O.dequant_fp8(codes, s, block_n, g, dtype)
        gemm = ops.gemm_fp8_marlin_cuda
    eye = torch.eye(k, dtype=TDT[dtype], device="cuda")
    y = gemm(eye, w, sc, n, block_n, g)
    assert np.array_equal(to_np(y), ref.T), "MFMA path"
    for r0, rows in [(0, 16), (k - 16, 16), (37, 1), (70, 5)]:
        y = gemm(eye[r0:r0 + rows].contiguous(), w, sc, n, block_n, g)
        assert np.array_equal(to_np(y), ref.T[r0:r0 + rows]), f"decode path rows {r0}+{rows}"


# ------------------------------------------------------------------ dequantize-then-matmul tolerance


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
@pytest.mark.parametrize("m", [1, 5, 16, 17, 100, 300])
def test_int4_gemm_reference_shape(m, dtype):
    """test_marlin.cpp:98-114 (block_n = 1)."""
    packed, s = int4_case(N, K, G, 1, seed=5, scale_dtype=np.float32, scale_kind="test")
    w, sc = _repack_int4(packed, s, 1, G)
    x = x_case(m, K, dtype, seed=m)
    y = ops.gemm_int4_marlin_cuda(to_dev(x, TDT[dtype]), w, sc, N, 1, G)
    assert y.shape == (m, N) and y.dtype == TDT[dtype]
    assert_close(y, O.gemm_ref(x, O.dequant_int4(packed, s, 1, G, dtype), None), f"m={m}")


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
@pytest.mark.parametrize("m", [1, 16, 100])
def test_fp8_gemm_reference_shape(m, dtype):
    """test_marlin.cpp:80-96 (block_n = 128)."""
    codes, s = fp8_case(N, K, G, 128, seed=6)
    w, sc = _repack_fp8(codes, s, 128, G)
    x = x_case(m, K, dtype, seed=m)
    y = ops.gemm_fp8_marlin_cuda(to_dev(x, TDT[dtype]), w, sc, N, 128, G)
    assert_close(y, O.gemm_ref(x, O.dequant_fp8(codes, s, 128, G, dtype), None), f"m={m}")


@pytest.mark.parametrize("m", [1, 4, 16, 64, 256])
@pytest.mark.parametrize("g", [32, 64, 128, 256])
def test_int4_gemm_group_sizes(m, g):
    n, k = 520, 1024
    packed, s = int4_case(n, k, g, 1, seed=g)
    w, sc = _repack_int4(packed, s, 1, g)
    x = x_case(m, k, "bf16", seed=m + g)
    y = ops.gemm_int4_marlin_cuda(to_dev(x, torch.bfloat16), w, sc, n, 1, g)
    assert_close(y, O.gemm_ref(x, O.dequant_int4(packed, s, 1, g), None), f"m={m} g={g}")


@pytest.mark.parametrize("m", [1, 17, 40, 300])
@pytest.mark.parametrize("n,k", [(8, 16), (40, 32), (24, 48), (200, 16)])
def test_int4_gemm_below_one_k_tile(m, n, k):
    """K below one 128-wide tile (16-wide groups, the reference test's group size) and N below
    or not a multiple of a 16-column strip, on the decode kernels (M <= 32) and the MFMA
    kernel (M > 32): the partial K tile and the partial strip read as zero."""
    g = 16
    packed, s = int4_case(n, k, g, 1, seed=n + k)
    w, sc = _repack_int4(packed, s, 1, g)
    x = x_case(m, k, "bf16", seed=m + k)
    y = ops.gemm_int4_marlin_cuda(to_dev(x, torch.bfloat16), w, sc, n, 1, g)
    assert_close(y, O.gemm_ref(x, O.dequant_int4(packed, s, 1, g), None), f"m={m} n={n} k={k}")


@pytest.mark.parametrize("m", [1, 3, 4, 8, 13, 16])
@pytest.mark.parametrize("case", ["fp16s-bf16x", "fp32s-bf16x", "bf16s-fp16x", "fp32s-strip", "g256"])
def test_decode_kernel_variants(m, case):
    """The M <= 16 decode kernels across scale layouts, activation dtypes and a ragged strip
    count (N = 8200: 513 strips, so strip groups of 2, 3 or more end in a partial group)."""
    n, k, g, block_n, dtype = 8200, 512, 128, 1, "bf16"
    sdt = np.float16
    if case == "fp32s-bf16x":
        sdt = np.float32
    elif case == "bf16s-fp16x":
        dtype, sdt = "fp16", np.float32
    elif case == "fp32s-strip":
        block_n, sdt = 128, np.float32
    elif case == "g256":
        g = 256
    packed, s = int4_case(n, k, g, block_n, seed=m + 7)
    s = s.astype(sdt)
    if case == "bf16s-fp16x":  # bf16-stored scales
        s = O.round_to(s.astype(np.float32), "bf16")
        s_dev = to_dev(s).to(torch.bfloat16)
    else:
        s_dev = scale_tensor(s)
    w, sc = ops.repack_int4_marlin_cuda(to_dev(packed), s_dev, block_n, g)
    x = x_case(m, k, dtype, seed=m)
    y = ops.gemm_int4_marlin_cuda(to_dev(x, TDT[dtype]), w, sc, n, block_n, g)
    assert_close(y, O.gemm_ref(x, O.dequant_int4(packed, s, block_n, g, dtype), None), f"{case} m={m}")


def test_config1_m16_k4096_n4096():
    """benchmark config 1: M=16, K=N=4096, int4 g128 symmetric, fp16 scales |N(0,.02)|+1e-3."""
    x, packed, s = O.make_w4a16(16, 4096, 4096, 128, seed=1)
    w, sc = ops.repack_int4_marlin_cuda(to_dev(packed), to_dev(s), 1, 128)
    y = ops.gemm_int4_marlin_cuda(to_dev(x, torch.bfloat16), w, sc, 4096, 1, 128)
    st = assert_close(y, O.gemm_ref(x, O.dequant_int4(packed, s, 1, 128), None), "config1")
    print("config1", st)


@pytest.mark.parametrize("shape", [(4096, 6144), (4096, 4096), (4096, 24576), (12288, 4096)])
@pytest.mark.parametrize("m", [1, 4, 16, 256])
def test_qwen3_8b_shapes(shape, m):
    k, n = shape
    x, packed, s = O.make_w4a16(m, n, k, 128, seed=k + n + m)
    w, sc = ops.repack_int4_marlin_cuda(to_dev(packed), to_dev(s), 1, 128)
    y = ops.gemm_int4_marlin_cuda(to_dev(x, torch.bfloat16), w, sc, n, 1, 128)
    assert_close(y, O.gemm_ref(x, O.dequant_int4(packed, s, 1, 128), None), f"{shape} m={m}")


def test_deterministic_across_calls():
    x, packed, s = O.make_w4a16(16, 4096, 12288, 128, seed=9)
    w, sc = ops.repack_int4_marlin_cuda(to_dev(packed), to_dev(s), 1, 128)
    xd = to_dev(x, torch.bfloat16)
    a = ops.gemm_int4_marlin_cuda(xd, w, sc, 4096, 1, 128)
    b = ops.gemm_int4_marlin_cuda(xd, w, sc, 4096, 1, 128)
    assert torch.equal(a, b)
    x2 = to_dev(O.make_w4a16(300, 64, 12288, 128, seed=9)[0], torch.bfloat16)
    a = ops.gemm_int4_marlin_cuda(x2, w, sc, 4096, 1, 128)
    b = ops.gemm_int4_marlin_cuda(x2, w, sc, 4096, 1, 128)
    assert torch.equal(a, b)


@pytest.mark.parametrize("case", [
    ("int4", 16, 12288, 4096),  # decode kernel with a K split across workgroups
    ("int4", 256, 4096, 4096),  # MFMA kernel with a K split (fewer tiles than CUs)
    ("int4", 4096, 4096, 6144),  # MFMA kernel: whole rounds, then the tail as 128-row halves
    ("fp8", 2048, 5120, 34816),  # fp8 W8A16 tall tiles: whole rounds, then the K-split tail launch
    ("fp8", 16, 5120, 7168),  # fp8 W8A16 decode: two strips on 8 wavefronts, K split in two
    ("w8a8", 16, 5120, 5120),  # per-token quantizer, then the W8A8 decode kernel
    ("w8a8", 2, 5120, 5120),  # the W8A8 decode kernel with the quantizer fused in
])
def test_gemm_graph_replays_match_eager(case):
    """plm_gemm captured into a graph: the split-K arrival counters are reset by the last
    workgroup of every call, so each replay (with eager calls between them) must equal the
    eager result bit for bit."""
    fmt, m, k, n = case
    print(f"graph replay case {case}", flush=True)
    rng = np.random.default_rng(61)
    xd = torch.from_numpy(rng.standard_normal((m, k), dtype=np.float32)).to("cuda").to(torch.bfloat16)
    if fmt == "int4":
        packed = rng.integers(-(2**31), 2**31, size=(n, k // 8), dtype=np.int64).astype(np.int32)
        s = (np.abs(rng.standard_normal((n, k // 128))) * 0.02 + 1e-3).astype(np.float16)
        w, sc = ops.repack_int4_marlin_cuda(to_dev(packed), to_dev(s), 1, 128)
        run = lambda: ops.gemm_int4_marlin_cuda(xd, w, sc, n, 1, 128)  # noqa: E731
    elif fmt == "fp8":
        codes, s = fp8_case(n, k, 128, 128, seed=63)
        w, sc = _repack_fp8(codes, s, 128, 128)
        run = lambda: ops.gemm_fp8_marlin_cuda(xd, w, sc, n, 128, 128)  # noqa: E731
    else:
        codes, s = fp8_case(n, k, 128, 128, seed=62)
        w, sc = _repack_fp8(codes, s, 128, 128)
        run = lambda: ops.gemm_fp8_w8a8_cuda(xd, w, sc, n, 128, 128)  # noqa: E731
    eager = run()
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        run()  # the stream's workspace is allocated (zeroed) outside the capture
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            out = run()
    for i in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"{case}: replay {i} differs from the eager result"
        again = run()
        torch.cuda.synchronize()
        assert torch.equal(again, eager), f"{case}: eager call after replay {i} differs"


# ------------------------------------------------------------------ Marlin-layout ingest, edge cases


@pytest.mark.parametrize("fmt", ["int4", "fp8"])
def test_convert_marlin_matches_repack(fmt):
    bn = 1 if fmt == "int4" else 128
    if fmt == "int4":
        packed, s = int4_case(N, K, G, bn, seed=7, scale_dtype=np.float32, scale_kind="test")
        words = O.marlin_encode_int4(packed)
        w_ref, s_ref = _repack_int4(packed, s, bn, G)
    else:
        codes, s = fp8_case(N, K, G, bn, seed=7)
        words = O.marlin_encode_fp8(codes)
        w_ref, s_ref = _repack_fp8(codes, s, bn, G)
    w, sc = ops.convert_marlin_cuda(fmt, to_dev(words), to_dev(O.marlin_scale(s)), N, K, bn, G)
    assert torch.equal(w, w_ref)
    assert torch.equal(sc, s_ref)


def test_empty_m_and_n():
    packed, s = int4_case(N, K, G, 1, seed=8, scale_dtype=np.float32)
    w, sc = _repack_int4(packed, s, 1, G)
    y = ops.gemm_int4_marlin_cuda(torch.empty((0, K), dtype=torch.bfloat16, device="cuda"), w, sc, N, 1, G)
    assert y.shape == (0, N)


def test_errors_name_the_op():
    packed, s = int4_case(N, K, G, 1, seed=8, scale_dtype=np.float32)
    w, sc = _repack_int4(packed, s, 1, G)
    x = torch.zeros((4, K), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError, match="gemm_int4_marlin: .*wrong size"):
        ops.gemm_int4_marlin_cuda(x, w[:-1], sc, N, 1, G)
    with pytest.raises(RuntimeError, match="gemm_int4_marlin: x must be fp16 or bf16"):
        ops.gemm_int4_marlin_cuda(x.float(), w, sc, N, 1, G)
    with pytest.raises(RuntimeError, match="repack_int4_marlin: group_size"):
        ops.repack_int4_marlin_cuda(to_dev(packed), scale_tensor(s), 1, 24)


# ------------------------------------------------------------------ full sizes (benchmark configs 2 and 3)
#
# At full size the CPU oracle is too slow, so the weights come from plm_dequant (bit-exact,
# pinned above against the oracle) and the reference product is torch's fp32 matmul of the
# rounded operands on the GPU, to the same tolerance as every other GEMM here.


def _full_case(m, k, n, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    q = torch.randint(-8, 8, (n, k), generator=g, dtype=torch.int32)
    nib = (q & 0xF).view(n, k // 8, 8)
    packed = torch.zeros((n, k // 8), dtype=torch.int64)
    for i in range(8):
        packed |= nib[:, :, i].to(torch.int64) << (4 * i)
    packed = packed.to(torch.uint32).view(torch.int32)
    s = (torch.randn((n, k // 128), generator=g) * 0.02).abs_().add_(1e-3).half()
    x = torch.randn((m, k), generator=g).bfloat16()
    return x.cuda(), packed.cuda(), s.cuda()


def _check_full(y, x, wd):
    torch.backends.cuda.matmul.allow_tf32 = False
    ref = x.float() @ wd.float().T
    err = (y.float() - ref).abs()
    assert bool((err <= 2e-2 + 2e-2 * ref.abs()).all()), f"max err {err.max().item():.4g}"
    rel = (torch.linalg.vector_norm(y.float() - ref) / torch.linalg.vector_norm(ref)).item()
    assert rel <= 5e-3, rel
    # Row checksums: sum_n y[m, n] against x[m] . sum_n W[n, :] (fp64), a property that does
    # not depend on how the kernel tiles or splits K. Each bf16 output carries at most half an
    # ulp (2^-9 relative) of rounding, so a row sum may move by sum |y| * 2^-9; 2^-8 leaves room
    # for the fp32 accumulation.
    cs = x.double() @ wd.double().sum(0)
    bound = y.double().abs().sum(1) * 2.0**-8 + 1e-3
    assert bool(((y.double().sum(1) - cs).abs() <= bound).all())
    return rel


@pytest.mark.parametrize("shape", [(4096, 6144), (4096, 4096), (4096, 24576), (12288, 4096)])
@pytest.mark.parametrize("m", [16, 1024, 4096])
def test_full_size_against_gpu_fp32(shape, m):
    """Configs 2 and 3 at full size, every row: M=16 on the decode kernels, M=1024 and
    M=4096 on the MFMA kernel (gate_up at M=1024 and qkv at M=4096 end with the 128-row
    halves launch)."""
    k, n = shape
    x, packed, s = _full_case(m, k, n, seed=k ^ n ^ m)
    w, sc = ops.repack_int4_marlin_cuda(packed, s, 1, 128)
    wd = ops.dequant_marlin_cuda("int4", w, sc, n, k, 1, 128)
    y = ops.gemm_int4_marlin_cuda(x, w, sc, n, 1, 128)
    print(shape, m, "rel-L2", _check_full(y, x, wd))


@pytest.mark.parametrize("n", [1024, 1000, 1004])
@pytest.mark.parametrize("y_shift", [0, 1])
def test_mfma_epilogue_store_forms(n, y_shift, tuning_env):
    """The tall shape stores its output 16 bytes at a time when N % 8 == 0 and y is 16-byte
    aligned, and element by element otherwise (y need only be 2-byte aligned; N = 1004 and a
    y one element past an aligned address take the fallback). Both forms must give the
    aligned call's result on the same shape bit for bit, and every row must match the fp32
    reference."""
    m, k = 512, 512  # 8 tall tiles, K not split (the split-K kernels keep the 2-byte stores)
    tuning_env("PLM_MFMA", "X")
    x, packed, s = _full_case(m, k, n, seed=n + y_shift)
    w, sc = ops.repack_int4_marlin_cuda(packed, s, 1, 128)
    wd = ops.dequant_marlin_cuda("int4", w, sc, n, k, 1, 128)
    buf = torch.full((m * n + 16,), float("nan"), dtype=torch.bfloat16, device=x.device)
    y = buf[y_shift:y_shift + m * n].view(m, n)
    ops.gemm_int4_marlin_cuda(x, w, sc, n, 1, 128, out=y)
    torch.cuda.synchronize()
    _check_full(y, x, wd)
    assert bool(buf[:y_shift].isnan().all()) and bool(buf[y_shift + m * n:].isnan().all()), "wrote outside y"
    ref = ops.gemm_int4_marlin_cuda(x, w, sc, n, 1, 128)  # a fresh, aligned y
    assert torch.equal(y, ref)


def test_decode_and_mfma_kernels_agree():
    """M=16 and M=32 run the decode kernels (one and two 16-row blocks), M=33 the MFMA
    kernel; their common rows must agree to the GEMM tolerance (each is checked against the
    oracle elsewhere)."""
    k, n = 12288, 4096
    x, packed, s = _full_case(33, k, n, seed=5)
    w, sc = ops.repack_int4_marlin_cuda(packed, s, 1, 128)
    a = ops.gemm_int4_marlin_cuda(x[:16].contiguous(), w, sc, n, 1, 128)
    b = ops.gemm_int4_marlin_cuda(x[:32].contiguous(), w, sc, n, 1, 128)
    c = ops.gemm_int4_marlin_cuda(x, w, sc, n, 1, 128)
    assert torch.allclose(a.float(), c[:16].float(), atol=2e-2, rtol=2e-2)
    assert torch.allclose(b.float(), c[:32].float(), atol=2e-2, rtol=2e-2)


@pytest.mark.parametrize("m", [17, 20, 24, 28, 31, 32])
@pytest.mark.parametrize("shape", [(4096, 6144), (4096, 4096), (4096, 24576), (12288, 4096)])
def test_two_row_block_decode(shape, m):
    """17 to 32 rows: the decode kernels with two 16-row MFMA blocks per dequantized weight
    fragment (gate_up above 24 rows goes to the MFMA kernel), rows past M of the second
    block never stored."""
    k, n = shape
    x, packed, s = O.make_w4a16(m, n, k, 128, seed=k + n + m)
    w, sc = ops.repack_int4_marlin_cuda(to_dev(packed), to_dev(s), 1, 128)
    y = ops.gemm_int4_marlin_cuda(to_dev(x, torch.bfloat16), w, sc, n, 1, 128)
    assert_close(y, O.gemm_ref(x, O.dequant_int4(packed, s, 1, 128), None), f"{shape} m={m}")


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
@pytest.mark.parametrize("case", ["fp16s", "fp32s-strip", "g256", "g64", "k-tail"])
def test_two_row_block_decode_variants(case, dtype):
    """Two row blocks across scale layouts, groups below and above one K tile, fp16 x, a
    ragged strip count (N = 8200) and a partial last K tile (K = 400, 16-wide groups)."""
    m, n, k, g, block_n, sdt = 23, 8200, 512, 128, 1, np.float16
    if case == "fp32s-strip":
        block_n, sdt = 128, np.float32
    elif case == "g256":
        g = 256
    elif case == "g64":
        g = 64
    elif case == "k-tail":
        m, n, k, g = 29, 300, 400, 16
    packed, s = int4_case(n, k, g, block_n, seed=len(case))
    s = s.astype(sdt)
    w, sc = ops.repack_int4_marlin_cuda(to_dev(packed), scale_tensor(s), block_n, g)
    x = x_case(m, k, dtype, seed=m)
    y = ops.gemm_int4_marlin_cuda(to_dev(x, TDT[dtype]), w, sc, n, block_n, g)
    assert_close(y, O.gemm_ref(x, O.dequant_int4(packed, s, block_n, g, dtype), None), f"{case} {dtype}")


@pytest.mark.parametrize("m", [1, 4, 7, 16, 17, 32])
@pytest.mark.parametrize("n,k,g", [(16, 128, 128), (48, 128, 128), (40, 256, 256), (1000, 384, 128)])
def test_decode_small_k_and_narrow_n(m, n, k, g):
    """Decode kernels where most wavefronts of a workgroup own no K tile (K of 1-3 tiles),
    a single strip (N = 16) and a 256-wide scale group spanning two tiles."""
    packed, s = int4_case(n, k, g, 1, seed=n + k + m)
    w, sc = ops.repack_int4_marlin_cuda(to_dev(packed), scale_tensor(s), 1, g)
    x = x_case(m, k, "bf16", seed=m)
    y = ops.gemm_int4_marlin_cuda(to_dev(x, torch.bfloat16), w, sc, n, 1, g)
    assert_close(y, O.gemm_ref(x, O.dequant_int4(packed, s, 1, g), None), f"m={m} n={n} k={k}")


@pytest.mark.parametrize("m", [1, 2, 4])
@pytest.mark.parametrize("n,k,g,dtype", [(4096, 12288, 128, "bf16"), (520, 10240, 128, "bf16"),
                                         (264, 16384, 256, "fp16"), (100, 12288, 128, "fp16")])
def test_decode_long_k(m, n, k, g, dtype):
    """M <= 4 at long K (80-128 K tiles, more than the round-robin kernel's one load batch
    holds): the split-K decode kernel, with 128- and 256-wide groups, fp16 x and ragged N."""
    packed, s = int4_case(n, k, g, 1, seed=n + k + m)
    w, sc = ops.repack_int4_marlin_cuda(to_dev(packed), scale_tensor(s), 1, g)
    x = x_case(m, k, dtype, seed=m + 3)
    y = ops.gemm_int4_marlin_cuda(to_dev(x, TDT[dtype]), w, sc, n, 1, g)
    assert_close(y, O.gemm_ref(x, O.dequant_int4(packed, s, 1, g, dtype), None), f"m={m} n={n} k={k} g={g}")


# ------------------------------------------------------------------ int4 scale domain


def _edge_scales(n, groups, seed):
    """bf16-exact scales in [2^119, 2^120): the largest the int4 kernels accept."""
    j = np.random.default_rng(seed).integers(0, 128, size=(n, groups))
    return (np.ldexp(1.0 + j / 128.0, 119)).astype(np.float32)


@pytest.mark.parametrize("m", [1, 16, 256])
@pytest.mark.parametrize("sdt", ["fp32", "bf16"])
def test_int4_scale_domain_edge_exact(m, sdt):
    """Scales just below 2^120 (where (128 + q + 8) s still fits fp32) go through the decode
    (M = 1, 16) and MFMA (M = 256) kernels exactly: the identity rows of x pick out
    round(q round(s)) bit for bit, as test_marlin.cpp:54-78 does for ordinary scales."""
    n, k, g = 64, 256, 128
    print(f"scale edge m={m} scale={sdt}", flush=True)
    packed, _ = int4_case(n, k, g, 1, seed=m)
    s = _edge_scales(n, k // g, seed=m)
    st = to_dev(s) if sdt == "fp32" else to_dev(s, torch.bfloat16)
    w, sc = ops.repack_int4_marlin_cuda(to_dev(packed), st, 1, g)
    cols = np.random.default_rng(m + 1).permutation(k)[:m]
    x = np.zeros((m, k), np.float32)
    x[np.arange(m), cols] = 1.0
    y = ops.gemm_int4_marlin_cuda(to_dev(x, torch.bfloat16), w, sc, n, 1, g)
    ref = O.dequant_int4(packed, s, 1, g, "bf16")[:, cols].T
    got = to_np(y)
    assert np.isfinite(got).all()
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("sdt", ["fp32", "bf16"])
def test_int4_scales_beyond_the_domain_are_rejected(sdt):
    """A scale whose bf16 rounding reaches 2^120 is refused at repack time with the op's
    name (the kernels would overflow (128 + q + 8) s), and so is one that rounds up to it;
    one bf16 step below passes (previous test)."""
    n, k, g = 32, 256, 128
    packed, _ = int4_case(n, k, g, 1, seed=7)
    for big in (2.0**120, np.float32(2.0**120 * (1 - 2.0**-10))):  # the second rounds up to 2^120 in bf16
        s = np.full((n, k // g), 0.02, np.float32)
        s[5, 1] = -big
        st = to_dev(s) if sdt == "fp32" else to_dev(s, torch.bfloat16)
        with pytest.raises(Exception, match=r"repack_int4_marlin: int4 scales must be below 2\^120"):
            ops.repack_int4_marlin_cuda(to_dev(packed), st, 1, g)


def test_int4_scale_check_from_several_threads():
    """The repack's scale check uses one flag per device. Repacks from two host threads, each
    on its own stream, one thread with an out-of-domain scale and one with valid scales, must
    each get their own verdict: the valid weights repack to the same bits as alone, and every
    out-of-domain repack is refused."""
    import threading

    n, k, g = 64, 512, 128
    packed, _ = int4_case(n, k, g, 1, seed=9)
    good = np.full((n, k // g), 0.03, np.float32)
    bad = good.copy()
    bad[7, 2] = 2.0**121
    pk = to_dev(packed)
    ref_w, ref_s = ops.repack_int4_marlin_cuda(pk, to_dev(good), 1, g)
    torch.cuda.synchronize()
    results = {"good": [], "bad": []}

    def worker(kind, scales):
        stream = torch.cuda.Stream()
        st = to_dev(scales)
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            for _ in range(20):
                try:
                    w, sc = ops.repack_int4_marlin_cuda(pk, st, 1, g)
                    stream.synchronize()
                    results[kind].append(torch.equal(w, ref_w) and torch.equal(sc, ref_s))
                except Exception as e:  # noqa: BLE001 - the refusal is the expected outcome for "bad"
                    results[kind].append("below 2^120" in str(e) and "refused")

    threads = [threading.Thread(target=worker, args=("good", good)), threading.Thread(target=worker, args=("bad", bad))]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert results["good"] == [True] * 20, results["good"]
    assert results["bad"] == ["refused"] * 20, results["bad"]


@pytest.mark.parametrize("m,k,n", [(1, 4096, 6144), (4, 4096, 24576), (1, 12288, 512), (3, 12288, 512)])
def test_int4_scales_across_ranges_exact(m, k, n):
    """Scales mostly ordinary, with scattered groups below 2^-17 or at 2^16 and above, and one
    strip entirely at 2^-18, through the decode kernels (round-robin at K = 4096, split-K at
    K = 12288): identity rows of x must pick out round(q round(s)) bit for bit in every
    column."""
    g = 128
    print(f"scale ranges m={m} k={k} n={n}", flush=True)
    rng = np.random.default_rng(k + n + m)
    packed, s = int4_case(n, k, g, 1, seed=m + 3, scale_dtype=np.float32)
    groups = s.shape[1]
    pick = rng.random(s.shape) < 0.01
    s[pick] = rng.choice(np.array([3.0e-6, 1.5e-7, 7.0e4, -1.2e5, 2.0**-17, 2.0**16], np.float32), pick.sum())
    s[0, :] = 2.0**-18  # one strip entirely on the bf16 form
    w, sc = ops.repack_int4_marlin_cuda(to_dev(packed), to_dev(s), 1, g)
    cols = rng.permutation(k)[:m]
    x = np.zeros((m, k), np.float32)
    x[np.arange(m), cols] = 1.0
    y = ops.gemm_int4_marlin_cuda(to_dev(x, torch.bfloat16), w, sc, n, 1, g)
    ref = O.dequant_int4(packed, s, 1, g, "bf16")[:, cols].T
    assert np.array_equal(to_np(y), ref)
    assert groups == k // g
