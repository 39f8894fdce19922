"""pulsarlm-core/tests/kernels/test_marlin.cpp restated against the C++ host layer
(pulsarlm_amd/_host.so -> C ABI -> HIP): same shape (n=200, k=144, g=16), same
generators (seeded here), same exactness and allclose(2e-2, 2e-2) checks. Plus the
linear operator (linear.hpp) with the int4 alternative, on a 3-D input."""

import numpy as np
import pytest
import torch

from pulsarlm_amd import _host

pytestmark = pytest.mark.gpu

N, K, G = 200, 144, 16  # test_marlin.cpp:15-17


def cuda(dtype):
    return dict(device="cuda", dtype=dtype)


def random_scale(block_n, gen):  # test_marlin.cpp:23-25
    return torch.rand(((N + block_n - 1) // block_n, K // G), generator=gen, **cuda(torch.float)) * 0.1 + 0.01


def expanded_scale(scale, block_n):  # test_marlin.cpp:27-29
    return scale.repeat_interleave(block_n, 0)[:N].repeat_interleave(G, 1)


def random_fp8(gen):  # test_marlin.cpp:32-36
    b = torch.randint(0, 256, (N, K), generator=gen, **cuda(torch.uint8))
    b[(b == 0x7F) | (b == 0xFF)] = 0
    return b.view(torch.float8_e4m3fn)


def random_int4(gen):  # test_marlin.cpp:38-40
    return torch.randint(-8, 8, (N, K), generator=gen, **cuda(torch.int32))


def packed_int4(values):  # test_marlin.cpp:42-46
    shifts = torch.arange(0, 32, 4, dtype=torch.long)
    nib = values.cpu().bitwise_and(0xF).to(torch.long).view(N, K // 8, 8)
    return nib.bitwise_left_shift(shifts).sum(-1).to(torch.int32).cuda()


def dequantized(weight, scale, block_n, dtype):  # test_marlin.cpp:48-50
    return weight.to(dtype) * expanded_scale(scale, block_n).to(dtype)


def gen(seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return g


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("block_n", [1, 128])
def test_fp8_dequantizes_every_e4m3_code_exactly(dtype, block_n):  # test_marlin.cpp:54-65
    g = gen(1)
    weight = random_fp8(g)
    scale = random_scale(block_n, g)
    wm, sm = _host.repack_fp8_marlin_cuda(weight, scale, block_n, G)
    identity = torch.eye(K, **cuda(dtype))
    y = _host.gemm_fp8_marlin_cuda(identity, wm, sm, N, block_n, G)
    assert torch.equal(y, dequantized(weight, scale, block_n, dtype).t())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("block_n", [1, 128])
def test_int4_dequantizes_every_int4_value_exactly(dtype, block_n):  # test_marlin.cpp:67-78
    g = gen(2)
    values = random_int4(g)
    scale = random_scale(block_n, g)
    wm, sm = _host.repack_int4_marlin_cuda(packed_int4(values), scale, block_n, G)
    identity = torch.eye(K, **cuda(dtype))
    y = _host.gemm_int4_marlin_cuda(identity, wm, sm, N, block_n, G)
    assert torch.equal(y, dequantized(values, scale, block_n, dtype).t())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m", [1, 16, 100])
def test_fp8_matches_dequantize_then_matmul(dtype, m):  # test_marlin.cpp:80-96
    g = gen(3 + m)
    block_n = 128
    weight = random_fp8(g)
    scale = random_scale(block_n, g)
    wm, sm = _host.repack_fp8_marlin_cuda(weight, scale, block_n, G)
    x = torch.randn((m, K), generator=g, **cuda(dtype))
    y = _host.gemm_fp8_marlin_cuda(x, wm, sm, N, block_n, G)
    ref = x.float() @ dequantized(weight, scale, block_n, dtype).float().t()
    assert torch.allclose(y.float(), ref, 2e-2, 2e-2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m", [1, 16, 100])
def test_int4_matches_dequantize_then_matmul(dtype, m):  # test_marlin.cpp:98-114
    g = gen(4 + m)
    block_n = 1
    values = random_int4(g)
    scale = random_scale(block_n, g)
    wm, sm = _host.repack_int4_marlin_cuda(packed_int4(values), scale, block_n, G)
    x = torch.randn((m, K), generator=g, **cuda(dtype))
    y = _host.gemm_int4_marlin_cuda(x, wm, sm, N, block_n, G)
    ref = x.float() @ dequantized(values, scale, block_n, dtype).float().t()
    assert torch.allclose(y.float(), ref, 2e-2, 2e-2)


def test_empty_rows_return_empty_output():  # marlin.cu:573-576
    g = gen(5)
    wm, sm = _host.repack_int4_marlin_cuda(packed_int4(random_int4(g)), random_scale(1, g), 1, G)
    y = _host.gemm_int4_marlin_cuda(torch.empty((0, K), **cuda(torch.bfloat16)), wm, sm, N, 1, G)
    assert y.shape == (0, N)


@pytest.mark.parametrize("kind", ["int4", "fp8"])
def test_linear_quantized_matches_dense(kind):
    g = gen(6)
    if kind == "int4":
        values = random_int4(g)
        scale = random_scale(1, g)
        lin = _host.linear.int4(packed_int4(values), scale, 1, G)
        dense = dequantized(values, scale, 1, torch.bfloat16)
    else:
        weight = random_fp8(g)
        scale = random_scale(128, g)
        lin = _host.linear.fp8(weight, scale, 128, G)
        dense = dequantized(weight, scale, 128, torch.bfloat16)
    x = torch.randn((3, 5, K), generator=g, **cuda(torch.bfloat16))
    y = lin.apply(x)
    assert y.shape == (3, 5, N)
    ref = _host.linear.dense(dense).apply(x)
    assert torch.allclose(y.float(), ref.float(), 2e-2, 2e-2)


def _quantize_int4(w, group):
    """Symmetric int4 per (row, group): scale = amax / 7 stored as fp16, q = clamp(round(w / s))."""
    n, k = w.shape
    blocks = w.float().view(n, k // group, group)
    scale = (blocks.abs().amax(-1) / 7).clamp_min(1e-8).to(torch.float16)
    q = torch.clamp(torch.round(blocks / scale.float()[..., None]), -8, 7).to(torch.int32).view(n, k)
    nib = q.bitwise_and(0xF).to(torch.long).view(n, k // 8, 8)
    packed = nib.bitwise_left_shift(torch.arange(0, 32, 4, device=w.device)).sum(-1).to(torch.int32)
    dense = q.to(torch.bfloat16) * scale.repeat_interleave(group, 1).to(torch.bfloat16)
    return packed, scale, dense


def _quantize_fp8(w, block):
    """The test_qwen3_5.cpp:301-311 block quantizer: scale = max(amax, 1e-12) / 448 per
    block x block tile, codes = e4m3(w / scale)."""
    n, k = w.shape
    t = w.float().view(n // block, block, k // block, block)
    scale = (t.abs().amax(dim=(1, 3)).clamp_min(1e-12) / 448).contiguous()
    codes = (t / scale[:, None, :, None]).view(n, k).to(torch.float8_e4m3fn)
    full = scale.repeat_interleave(block, 0).repeat_interleave(block, 1)
    dense = codes.to(torch.bfloat16) * full.to(torch.bfloat16)
    return codes, scale, dense


@pytest.mark.parametrize("kind", ["int4", "fp8_32", "fp8_128"])
@pytest.mark.parametrize("m", [1, 16, 24, 64])
def test_mlp_block_quantized_matches_dense(kind, m):
    """A Qwen3-style MLP block (gate_up, silu·mul, down) through linear::int4 / linear::fp8
    and silu_mul_cuda, against the same block on the dequantized weights in fp32: the
    model-level comparison of test_qwen3_5.cpp:691-696 (fp8 in 32 x 32 blocks there), with its
    bound, max |y - ref| / max |ref| < 5e-2. M = 1 and 16 run the decode kernels, 24 the
    two-row-block decode kernels, 64 the MFMA kernel."""
    hidden, inter = 512, 1024
    g = gen(40 + m)
    w_gu = (torch.randn((2 * inter, hidden), generator=g, **cuda(torch.float)) * 0.02).to(torch.bfloat16)
    w_dn = (torch.randn((hidden, inter), generator=g, **cuda(torch.float)) * 0.02).to(torch.bfloat16)
    x = torch.randn((m, hidden), generator=g, **cuda(torch.bfloat16))
    if kind == "int4":
        p_gu, s_gu, d_gu = _quantize_int4(w_gu, 128)
        p_dn, s_dn, d_dn = _quantize_int4(w_dn, 128)
        lin_gu, lin_dn = _host.linear.int4(p_gu, s_gu, 1, 128), _host.linear.int4(p_dn, s_dn, 1, 128)
    else:
        b = 32 if kind == "fp8_32" else 128
        c_gu, s_gu, d_gu = _quantize_fp8(w_gu, b)
        c_dn, s_dn, d_dn = _quantize_fp8(w_dn, b)
        lin_gu, lin_dn = _host.linear.fp8(c_gu, s_gu, b, b), _host.linear.fp8(c_dn, s_dn, b, b)
    y = lin_dn.apply(_host.silu_mul_cuda(lin_gu.apply(x)))
    h = x.float() @ d_gu.float().T
    ref = (torch.nn.functional.silu(h[:, :inter]) * h[:, inter:]) @ d_dn.float().T
    err = ((y.float() - ref).abs().max() / ref.abs().max()).item()
    assert err < 5e-2, f"{kind} m={m}: max relative error {err:.3g}"


# ------------------------------------------------- router and activation (test_fused_ops.cpp)


@pytest.mark.parametrize("dtype", [torch.float, torch.bfloat16])
@pytest.mark.parametrize("experts", [16, 512])
def test_route_top_k_picks_the_most_probable_experts(dtype, experts):
    """test_fused_ops.cpp:83-100 through the C++ route_top_k_cuda."""
    gen = torch.Generator(device="cuda").manual_seed(experts)
    k = 10
    logits = torch.randn(64, experts + 1, generator=gen, **cuda(dtype)).narrow(1, 0, experts)
    weights, chosen = _host.route_top_k_cuda(logits, k)
    probabilities = torch.softmax(logits, -1, dtype=torch.float)
    top = torch.topk(probabilities, k, -1).values
    assert chosen.dtype == torch.long
    assert torch.allclose(probabilities.gather(1, chosen), top, 1e-6, 0.0)
    assert torch.allclose(weights, top / top.sum(-1, True), 1e-6, 1e-6)


@pytest.mark.parametrize("dtype", [torch.float, torch.bfloat16])
def test_silu_mul_multiplies_silu_of_gate_by_up(dtype):
    """test_fused_ops.cpp:102-111 through the C++ silu_mul_cuda."""
    gen = torch.Generator(device="cuda").manual_seed(5)
    x = torch.randn(64, 2 * 256, generator=gen, **cuda(dtype))
    got = _host.silu_mul_cuda(x)
    expected = torch.nn.functional.silu(x.narrow(1, 0, 256)) * x.narrow(1, 256, 256)
    tol = 1e-5 if dtype == torch.float else 1e-2
    assert torch.allclose(got.float(), expected.float(), tol, tol)


# ------------------------------------------------- fp8 checkpoint ingest (weight_scale_inv)


def _block_checkpoint(n, k, seed):
    """A block-quantized fp8 checkpoint linear: the test_qwen3_5.cpp:301-311 quantizer on
    bf16 N(0, 0.02) weights, 128 x 128 blocks (weight, weight_scale_inv fp32)."""
    from oracle import oracle as O
    rng = np.random.default_rng(seed)
    w = O.round_to((rng.standard_normal((n, k)) * 0.02).astype(np.float32), "bf16")
    codes, scale_inv = O.fp8_block_quantize(w, 128, 128)
    weight = torch.from_numpy(codes).cuda().view(torch.float8_e4m3fn)
    return weight, torch.from_numpy(scale_inv).cuda(), O.dequant_fp8(codes, scale_inv, 128, 128, "bf16")


@pytest.mark.parametrize("n", [640, 5120 + 64])
def test_fp8_checkpoint_linear(n):
    """linear::fp8(weight, weight_scale_inv, 128, 128) as qwen3_5.cpp:52-63 builds it."""
    k = 1024
    weight, scale_inv, dense = _block_checkpoint(n, k, seed=n)
    lin = _host.linear.fp8(weight, scale_inv, 128, 128)
    x = torch.randn((2, 9, k), generator=gen(7), **cuda(torch.bfloat16))
    ref = x.float() @ torch.from_numpy(dense).cuda().t()
    assert torch.allclose(lin.apply(x).float(), ref, 2e-2, 2e-2)


def test_fp8_checkpoint_permuted_rows():
    """need_permuted_linear (qwen3_5.cpp:65-83): rows reordered across scale blocks
    (an interleave within 128-row heads) after expanding the scales to one per row."""
    n, k, head = 512, 768, 128
    weight, scale_inv, dense = _block_checkpoint(n, k, seed=3)
    within = torch.cat([torch.arange(0, head, 2), torch.arange(1, head, 2)])
    order = torch.cat([h * head + within for h in range(n // head)])
    order = order.view(-1, head).flip(0).reshape(-1)  # heads reversed too: rows cross blocks
    lin = _host.linear.fp8_rows(weight, scale_inv, 128, 128, order)
    for m in (1, 16, 200):
        x = torch.randn((m, k), generator=gen(m), **cuda(torch.bfloat16))
        ref = x.float() @ torch.from_numpy(dense).cuda()[order.cuda()].t()
        assert torch.allclose(lin.apply(x).float(), ref, 2e-2, 2e-2), m
