"""Parity of the MoE router (plm_route_top_k) and activation (plm_silu_mul) with the CPU
oracle, through the C ABI, mirroring pulsarlm-core/tests/kernels/test_fused_ops.cpp:83-111
(route_top_k: the chosen experts' probabilities equal the top-k probabilities to 1e-6 and
the weights equal them divided by their sum to 1e-6; silu_mul: allclose at 1e-5 for fp32
and 1e-2 for 16-bit dtypes), plus the router feeding the int4 MoE block on the device."""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from pulsarlm_amd import _lib, ops
from tests._util import int4_case, to_dev, to_np

pytestmark = pytest.mark.gpu

TDTYPE = {"fp32": torch.float32, "bf16": torch.bfloat16, "fp16": torch.float16}


@pytest.mark.parametrize("dtype", ["fp32", "bf16", "fp16"])
@pytest.mark.parametrize("experts,k", [(16, 10), (512, 10), (128, 8), (4096, 64), (1, 1)])
def test_route_top_k_matches_oracle(dtype, experts, k):
    gen = torch.Generator().manual_seed(experts + k)
    # Rows one element apart more than the experts, as the reference test narrows them.
    logits = torch.randn(300, experts + 1, generator=gen).to(TDTYPE[dtype]).cuda().narrow(1, 0, experts)
    weights, chosen = ops.route_top_k_cuda(logits, k)
    assert chosen.dtype == torch.int64 and weights.dtype == torch.float32
    w_ref, _, p_ref = O.route_top_k_ref(logits.float().cpu().numpy(), k)
    p = torch.from_numpy(p_ref)
    top = torch.topk(p, k, -1).values
    got_p = p.gather(1, chosen.cpu())
    assert torch.allclose(got_p, top, rtol=1e-6, atol=0.0)
    assert torch.allclose(weights.cpu(), top / top.sum(-1, keepdim=True), rtol=1e-6, atol=1e-6)
    assert torch.allclose(weights.cpu(), torch.from_numpy(w_ref), rtol=1e-6, atol=1e-6)
    assert all(len(set(r)) == k for r in chosen.cpu().tolist())  # distinct experts per token


def test_route_top_k_ties_and_int32_output():
    logits = torch.tensor([[1.0, 3.0, 3.0, 2.0, 3.0], [0.0] * 5], device="cuda")
    weights, chosen = ops.route_top_k_cuda(logits, 5)
    assert chosen.cpu().tolist() == [[1, 2, 4, 3, 0], [0, 1, 2, 3, 4]]
    w32, c32 = ops.route_top_k_cuda(logits, 3, experts_i32=True)
    assert c32.dtype == torch.int32 and c32.cpu().tolist() == [[1, 2, 4], [0, 1, 2]]
    assert torch.allclose(w32.cpu(), torch.full((2, 3), 1 / 3), atol=1e-7)


def test_route_top_k_errors_and_empty():
    with pytest.raises(RuntimeError, match="route_top_k"):
        ops.route_top_k_cuda(torch.randn(4, 8, device="cuda"), 9)
    with pytest.raises(RuntimeError, match="route_top_k"):
        ops.route_top_k_cuda(torch.randn(4, 5000, device="cuda"), 2)
    w, c = ops.route_top_k_cuda(torch.randn(0, 8, device="cuda"), 2)
    assert w.shape == (0, 2) and c.shape == (0, 2)


@pytest.mark.parametrize("dtype", ["fp32", "bf16", "fp16"])
@pytest.mark.parametrize("tokens,n", [(64, 768), (7, 13), (1, 8), (3000, 96)])
def test_silu_mul_matches_oracle(dtype, tokens, n):
    rng = np.random.default_rng(tokens + n)
    x = (rng.standard_normal((tokens, 2 * n)) * 3).astype(np.float32)
    xd = to_dev(x, TDTYPE[dtype])
    y = ops.silu_mul_cuda(xd)
    ref = O.silu_mul_ref(xd.float().cpu().numpy(), dtype)
    tol = 1e-5 if dtype == "fp32" else 1e-2
    assert np.allclose(to_np(y), ref, rtol=tol, atol=tol)
    if dtype == "fp32":  # exp and the division may differ from numpy's in the last bits
        assert np.allclose(to_np(y), ref, rtol=1e-6, atol=1e-30)
    else:  # the same rounding points: all but a few values next to a rounding tie agree exactly
        assert np.mean(to_np(y) == ref) > 0.99


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_silu_every_16bit_value(dtype):
    """The 16-bit silu (the reference's g / (1 + expf(-g)) in fp32, moe_routing.cu:129, then
    rounded) over every bf16 value with |g| <= 100 and every finite fp16 value, against the
    oracle: at most one unit in the last place apart, at least 99.9 % exact (zeros compared by
    value), and exact for g from -88.7 to -87.3, where silu's fp32 value is just above the
    denormal range and bf16 keeps it (a reciprocal-based silu flushes it to zero there)."""
    bits = np.arange(1 << 16, dtype=np.uint32)
    if dtype == "bf16":
        g = (bits << 16).view(np.float32)
        g = g[np.isfinite(g) & (np.abs(g) <= 100)]
    else:
        g = bits.astype(np.uint16).view(np.float16).astype(np.float32)
        g = g[np.isfinite(g)]
    n = g.size
    x = np.stack([g, np.ones_like(g)]).reshape(1, 2 * n)  # one row [g | u = 1]
    y = to_np(ops.silu_mul_cuda(to_dev(x, TDTYPE[dtype]))).reshape(-1)
    ref = O.silu_mul_ref(x, dtype).reshape(-1)
    assert np.mean(y == ref) >= 0.999, np.mean(y == ref)
    tdt = TDTYPE[dtype]
    as_int = lambda v: torch.from_numpy(np.ascontiguousarray(v)).to(tdt).view(torch.int16).numpy().astype(np.int32)
    # Zeros compare by value (-0 == +0; adding +0 makes every zero +0): one ulp apart at most.
    assert int(np.abs(as_int(y + np.float32(0)) - as_int(ref + np.float32(0))).max()) <= 1
    band = (g >= -88.7) & (g <= -87.3)
    if dtype == "bf16":
        assert band.any() and np.array_equal(y[band], ref[band]), (y[band], ref[band])


def test_router_feeds_the_moe_block():
    """route_top_k (int32 experts) -> routed_experts with int4 experts, on one stream,
    against the oracle's routing and routed_experts_ref."""
    e, hidden, inter, top_k, t, g = 16, 256, 128, 4, 96, 128
    rng = np.random.default_rng(11)
    gate_up = [int4_case(2 * inter, hidden, g, 1, seed=100 + i) for i in range(e)]
    down = [int4_case(hidden, inter, g, 1, seed=200 + i) for i in range(e)]
    gu_w, gu_s = ops.repack_int4_experts(torch.from_numpy(np.stack([p for p, _ in gate_up])).cuda(),
                                         torch.from_numpy(np.stack([s for _, s in gate_up])).cuda(), g)
    dn_w, dn_s = ops.repack_int4_experts(torch.from_numpy(np.stack([p for p, _ in down])).cuda(),
                                         torch.from_numpy(np.stack([s for _, s in down])).cuda(), g)
    h = O.round_to(rng.standard_normal((t, hidden)).astype(np.float32), "bf16")
    logits = rng.standard_normal((t, e)).astype(np.float32)
    out, offsets, w, experts = ops.moe_block_int4_cuda(to_dev(h, torch.bfloat16), to_dev(logits), top_k,
                                                       (gu_w, gu_s), (dn_w, dn_s), inter, g)
    w_ref, e_ref, _ = O.route_top_k_ref(logits, top_k)
    assert np.array_equal(experts.cpu().numpy(), e_ref)
    assert np.allclose(w.cpu().numpy(), w_ref, rtol=1e-6, atol=1e-6)
    gu_dense = np.stack([O.dequant_int4(p, s, 1, g) for p, s in gate_up])
    dn_dense = np.stack([O.dequant_int4(p, s, 1, g) for p, s in down])
    ref = O.routed_experts_ref(h, e_ref, w.cpu().numpy(), gu_dense, dn_dense)
    assert np.array_equal(offsets.cpu().numpy(), O.moe_sort(e_ref, e)[3])
    err = to_np(out) - ref
    assert np.linalg.norm(err) / np.linalg.norm(ref) <= 5e-3
    assert np.abs(err).max() / np.abs(ref).max() < 5e-2
