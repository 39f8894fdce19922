"""MoE on the GPU: the grouped int4 GEMM and the whole routed_experts block against
the oracle's restatement of paged_forward.cpp:108-130 over the dequantized experts.
The reference pins _grouped_mm only at model level (its arithmetic lives in PyTorch),
so at kernel level parity is against the oracle; offsets and the sort are exact."""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from pulsarlm_amd import ops
from tests._util import TDT, assert_close, to_dev, to_np


def assert_moe_close(y, ref, what):
    """The whole block chains two GEMMs through bf16 intermediates, so single elements
    can move by a bf16 ulp of the terms they sum (where those terms cancel, that is
    large next to the sum). Tolerance: the reference's own bf16 MoE check,
    max|y - ref| / max|ref| < 5e-2 (max_relative_error,
    pulsarlm-core/tests/model/test_qwen3_5_moe.cpp:322-324,420), and rel-L2 <= 5e-3."""
    _, st = O.check_close(to_np(y), ref)
    ok = st["max_abs"] / max(st["max_ref"], 1e-30) < 5e-2 and st["rel_l2"] <= 5e-3
    assert ok, f"{what}: {st}"

pytestmark = pytest.mark.gpu


def _experts(e, n, k, g, seed, scale_dtype="fp16", x_dtype="bf16"):
    rng = np.random.default_rng(seed)
    q = rng.integers(-8, 8, size=(e, n, k))
    packed = np.stack([O.pack_int4(q[i]) for i in range(e)])
    scale = np.abs(rng.standard_normal((e, n, k // g)) * 0.02) + 1e-3
    if scale_dtype == "fp16":
        scale = scale.astype(np.float16)
        s_dev = to_dev(scale)
    elif scale_dtype == "fp32":
        scale = scale.astype(np.float32)
        s_dev = to_dev(scale)
    else:  # bf16-stored scales
        scale = O.round_to(scale.astype(np.float32), "bf16")
        s_dev = to_dev(scale).to(torch.bfloat16)
    w, s = ops.repack_int4_experts(to_dev(packed), s_dev, g)
    deq = np.stack([O.dequant_int4(packed[i], scale[i], 1, g, x_dtype) for i in range(e)])
    return w, s, deq


# Below 128 rows per expert on average one shape sized to the average runs; from 128, full
# 256-row blocks (a last block of >= 192 rows counts as full) run on the 256 x 256 shape and
# the rest on 64-row tiles. [129] * 8 gives every expert the most 64-row tiles its remainder
# allows (3 each), more than the remaining rows alone would need.
@pytest.mark.parametrize("counts", [[5, 0, 17, 1, 0, 40, 3, 34], [0, 0, 0, 100, 0, 0, 0, 0], [1] * 8,
                                    [300, 20, 0, 2, 9, 0, 120, 61], [700, 130, 0, 200, 0, 0, 0, 0],
                                    [256, 512, 191, 192, 64, 63, 1, 0], [33] * 8, [129] * 8,
                                    [17, 33, 49, 1, 63, 65, 0, 47]])
def test_grouped_gemm_matches_per_expert_reference(counts):
    e, n, k, g = 8, 520, 1024, 128
    w, s, deq = _experts(e, n, k, g, seed=sum(counts))
    rows = sum(counts)
    x = O.bf16_round(np.random.default_rng(rows).standard_normal((rows, k)).astype(np.float32))
    offsets = np.cumsum(counts).astype(np.int32)
    y = ops.grouped_gemm_int4_cuda(to_dev(x, torch.bfloat16), w, s, to_dev(offsets), n, g)
    ref = np.zeros((rows, n), np.float32)
    start = 0
    for i, end in enumerate(offsets):
        if end > start:
            ref[start:end] = O.gemm_ref(x[start:end], deq[i], None)
        start = end
    assert_close(y, ref, f"grouped {counts}")


@pytest.mark.parametrize("counts", [[5, 0, 17, 1, 0, 40, 3, 34], [700, 130, 0, 200, 0, 0, 300, 0]])
@pytest.mark.parametrize("n", [520, 516])
def test_grouped_gemm_unaligned_output(counts, n):
    """The grouped kernels store 16 bytes at a time when N % 8 == 0 and y is 16-byte aligned,
    element by element otherwise: a y one element past an aligned address (and N = 516) must
    give the aligned result bit for bit and leave the rest of its buffer untouched. The
    second count list takes the two-list plan (256-row blocks, then 64-row tiles)."""
    e, k, g = 8, 1024, 128
    w, s, _ = _experts(e, n, k, g, seed=n + sum(counts))
    rows = sum(counts)
    x = to_dev(O.bf16_round(np.random.default_rng(rows).standard_normal((rows, k)).astype(np.float32)),
               torch.bfloat16)
    offsets = to_dev(np.cumsum(counts).astype(np.int32))
    ref = ops.grouped_gemm_int4_cuda(x, w, s, offsets, n, g)
    buf = torch.full((rows * n + 16,), float("nan"), dtype=torch.bfloat16, device=x.device)
    y = buf[1:1 + rows * n].view(rows, n)
    ops.grouped_gemm_int4_cuda(x, w, s, offsets, n, g, out=y)
    torch.cuda.synchronize()
    assert torch.equal(y, ref)
    assert bool(buf[:1].isnan().all()) and bool(buf[1 + rows * n:].isnan().all()), "wrote outside y"


# The 16-row grouped tiles (at most 8 rows per expert on average) and the 32-row ones (9-24)
# across scale storage, activation dtype and 256-wide groups, with an expert spanning several
# tiles and a ragged N.
SMALL_COUNTS = {16: [30, 0, 3, 1, 0, 0, 20, 2, 17, 0, 0, 19], 32: [70, 0, 3, 1, 0, 0, 20, 2, 33, 0, 0, 64]}


@pytest.mark.parametrize("tile_rows", [16, 32])
@pytest.mark.parametrize("sdt,xdt,g", [("fp32", "bf16", 128), ("bf16", "fp16", 128), ("fp16", "fp16", 256)])
def test_grouped_small_tiles(sdt, xdt, g, tile_rows):
    counts = SMALL_COUNTS[tile_rows]
    e, n, k = len(counts), 200, 1536
    w, s, deq = _experts(e, n, k, g, seed=11, scale_dtype=sdt, x_dtype=xdt)
    rows = sum(counts)
    x = O.round_to(np.random.default_rng(3).standard_normal((rows, k)).astype(np.float32), xdt)
    offsets = np.cumsum(counts).astype(np.int32)
    y = ops.grouped_gemm_int4_cuda(to_dev(x, TDT[xdt]), w, s, to_dev(offsets), n, g)
    ref = np.zeros((rows, n), np.float32)
    start = 0
    for i, end in enumerate(offsets):
        if end > start:
            ref[start:end] = O.gemm_ref(x[start:end], deq[i], None)
        start = end
    assert_close(y, ref, f"grouped {tile_rows}-row tiles {sdt} {xdt} g={g}")


def _moe_case(t, e, hidden, inter, top_k, g, seed):
    gu_w, gu_s, gu_deq = _experts(e, 2 * inter, hidden, g, seed)
    dn_w, dn_s, dn_deq = _experts(e, hidden, inter, g, seed + 1)
    h = O.bf16_round(np.random.default_rng(seed).standard_normal((t, hidden)).astype(np.float32))
    experts, weights = O.zipf_routing(t, e, top_k, seed=seed)
    return h, experts, weights, (gu_w, gu_s, gu_deq), (dn_w, dn_s, dn_deq)


@pytest.mark.parametrize("t,e,hidden,inter,top_k", [(40, 8, 256, 128, 2), (1, 8, 256, 128, 2), (256, 128, 2048, 768, 8),
                                                   (16, 1024, 128, 128, 8), (1024, 128, 256, 128, 8),
                                                   (70, 3, 128, 128, 3), (33, 1, 128, 128, 1), (300, 1, 128, 128, 1)])
def test_routed_experts_matches_oracle(t, e, hidden, inter, top_k):
    """Up to 8192 rows with one tile shape, the sort runs as one workgroup (a ballot-plane rank per
    64-row chunk and a scan of the experts x chunks table); 1024 x 128 fills that table,
    and 16 x 1024 spreads few rows over many experts. One expert: every row in one run (300
    rows take the two-list plan: a full 256-row block, then 64-row tiles)."""
    g = 128
    h, experts, weights, gu, dn = _moe_case(t, e, hidden, inter, top_k, g, seed=t + e)
    out, offsets = ops.routed_experts_int4_cuda(to_dev(h, torch.bfloat16), to_dev(experts.astype(np.int32)),
                                                to_dev(weights), gu[:2], dn[:2], inter, g)
    _, _, counts, ref_offsets = O.moe_sort(experts, e)
    assert np.array_equal(offsets.cpu().numpy(), ref_offsets)
    ref = O.routed_experts_ref(h, experts, weights, gu[2], dn[2])
    assert_moe_close(out, ref, f"moe t={t}")
    again, _ = ops.routed_experts_int4_cuda(to_dev(h, torch.bfloat16), to_dev(experts.astype(np.int32)),
                                            to_dev(weights), gu[:2], dn[:2], inter, g)
    assert torch.equal(out, again), "routed_experts must be deterministic"


def test_config5_t4096_sample():
    """benchmark config 5 at T=4096 (E=128, top-8, H=2048, I=768); the CPU oracle
    checks a sample of 64 tokens (full-size parity via the same kernels at T=256)."""
    t, e, hidden, inter, top_k, g = 4096, 128, 2048, 768, 8, 128
    h, experts, weights, gu, dn = _moe_case(t, e, hidden, inter, top_k, g, seed=5)
    out, offsets = ops.routed_experts_int4_cuda(to_dev(h, torch.bfloat16), to_dev(experts.astype(np.int32)),
                                                to_dev(weights), gu[:2], dn[:2], inter, g)
    _, _, _, ref_offsets = O.moe_sort(experts, e)
    assert np.array_equal(offsets.cpu().numpy(), ref_offsets)
    sample = np.random.default_rng(0).choice(t, 64, replace=False)
    ref = O.routed_experts_ref(h[sample], experts[sample], weights[sample], gu[2], dn[2])
    assert_moe_close(out[torch.from_numpy(sample).cuda()], ref, "moe t=4096 sample")


def test_routed_experts_graph_replays_match_eager():
    """The whole block (sort, tile lists, a two-level plan since rows >= 128 per expert,
    activation, combine) captured into a graph: every replay must equal the eager result,
    with eager work between replays (no node may depend on state left by the capture)."""
    t, e, hidden, inter, top_k, g = 1024, 8, 256, 128, 2, 128
    h, experts, weights, gu, dn = _moe_case(t, e, hidden, inter, top_k, g, seed=77)
    hd, ed, wd = to_dev(h, torch.bfloat16), to_dev(experts.astype(np.int32)), to_dev(weights)
    eager, _ = ops.routed_experts_int4_cuda(hd, ed, wd, gu[:2], dn[:2], inter, g)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        ops.routed_experts_int4_cuda(hd, ed, wd, gu[:2], dn[:2], inter, g)  # first-call set-up outside capture
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            out, _ = ops.routed_experts_int4_cuda(hd, ed, wd, gu[:2], dn[:2], inter, g)
    for i in range(4):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i} differs from the eager result"
        again, _ = ops.routed_experts_int4_cuda(hd, ed, wd, gu[:2], dn[:2], inter, g)
        torch.cuda.synchronize()
        assert torch.equal(again, eager)
    ref = O.routed_experts_ref(h, experts, weights, gu[2], dn[2])
    assert_moe_close(out, ref, "moe graph t=1024")


@pytest.mark.parametrize("t,e,hidden,inter,top_k", [(40, 8, 256, 128, 2), (1100, 16, 128, 128, 8)])
def test_routed_experts_drops_out_of_range_experts(t, e, hidden, inter, top_k):
    """Expert ids outside [0, n_experts) (-1 padding, ids >= n_experts) contribute nothing
    and are not counted in the offsets; the block stays in bounds. The first case sorts in
    one workgroup, the second (8800 rows) on the multi-kernel sort with a two-level plan.
    The reference's index_add_ would raise on such ids; dropping them is this build's rule."""
    g = 128
    h, experts, weights, gu, dn = _moe_case(t, e, hidden, inter, top_k, g, seed=t + 3)
    rng = np.random.default_rng(t)
    bad = rng.random(experts.shape) < 0.15
    bad[0, :] = True  # one token with no valid assignment: its output row is zero
    junk = rng.choice(np.array([-1, -7, e, e + 5, 1 << 20], dtype=np.int64), size=experts.shape)
    routed = np.where(bad, junk, experts)
    print(f"dropped {int(bad.sum())} of {bad.size} assignments", flush=True)
    out, offsets = ops.routed_experts_int4_cuda(to_dev(h, torch.bfloat16), to_dev(routed.astype(np.int32)),
                                                to_dev(weights), gu[:2], dn[:2], inter, g)
    counts = np.bincount(experts[~bad], minlength=e)
    assert np.array_equal(offsets.cpu().numpy(), np.cumsum(counts).astype(np.int32))
    # Oracle: the dropped assignments go to expert 0 with weight 0, so they add exact zeros.
    ref = O.routed_experts_ref(h, np.where(bad, 0, experts), np.where(bad, 0.0, weights).astype(np.float32),
                               gu[2], dn[2])
    got = to_np(out)
    assert np.all(got[0] == 0)
    assert_moe_close(out, ref, f"moe with dropped experts t={t}")


def test_grouped_gemm_clamps_offsets_to_rows():
    """Offsets past `rows` are clamped (the last expert ends at row `rows`), and a
    decreasing offset gives that expert no rows, so tiles never leave [0, rows)."""
    e, n, k, g = 3, 64, 256, 128
    w, s, deq = _experts(e, n, k, g, seed=21)
    rows = 22
    x = O.bf16_round(np.random.default_rng(5).standard_normal((rows, k)).astype(np.float32))
    y = ops.grouped_gemm_int4_cuda(to_dev(x, torch.bfloat16), w, s, to_dev(np.array([5, 15, 40], np.int32)), n, g)
    ref = np.concatenate([O.gemm_ref(x[:5], deq[0], None), O.gemm_ref(x[5:15], deq[1], None),
                          O.gemm_ref(x[15:], deq[2], None)])
    assert_close(y, ref, "offsets past rows")
    y2 = ops.grouped_gemm_int4_cuda(to_dev(x, torch.bfloat16), w, s, to_dev(np.array([5, 3, 3], np.int32)), n, g)
    assert_close(y2[:5], O.gemm_ref(x[:5], deq[0], None), "decreasing offsets")


@pytest.mark.parametrize("t,e,hidden,inter,top_k", [(256, 128, 2048, 768, 8), (1024, 8, 256, 128, 2),
                                                   (40, 8, 256, 128, 2)])
def test_fused_activation_matches_unfused_pipeline(t, e, hidden, inter, top_k):
    """routed_experts runs the activation inside the gate_up GEMM's epilogue. Composed
    from the unfused ops on the same sort -- grouped gate_up GEMM [rows, 2I], silu_mul,
    grouped down GEMM, then the weighted sum in k order in fp32 -- it must give the same
    bits (config 5 at T = 256 on one tile shape; 1024 x 2 over 8 experts on the two-level
    plan of 256-row blocks and 64-row tiles)."""
    g = 128
    h, experts, weights, gu, dn = _moe_case(t, e, hidden, inter, top_k, g, seed=t + 11)
    hd = to_dev(h, torch.bfloat16)
    out, offsets = ops.routed_experts_int4_cuda(hd, to_dev(experts.astype(np.int32)), to_dev(weights),
                                                gu[:2], dn[:2], inter, g)
    order, tokens, _, ref_offsets = O.moe_sort(experts, e)
    assert np.array_equal(offsets.cpu().numpy(), ref_offsets)
    rows = hd[torch.from_numpy(tokens).cuda()].contiguous()
    off = to_dev(ref_offsets)
    gate_up = ops.grouped_gemm_int4_cuda(rows, gu[0], gu[1], off, 2 * inter, g)
    act = ops.silu_mul_cuda(gate_up)
    d = ops.grouped_gemm_int4_cuda(act, dn[0], dn[1], off, hidden, g)
    position = np.empty(t * top_k, np.int64)
    position[order] = np.arange(t * top_k)
    w_bf = torch.from_numpy(weights.reshape(-1)).cuda().to(torch.bfloat16).float()
    acc = torch.zeros((t, hidden), dtype=torch.float32, device="cuda")
    pos = torch.from_numpy(position.reshape(t, top_k)).cuda()
    for j in range(top_k):
        term = (d[pos[:, j]].float() * w_bf.view(t, top_k)[:, j:j + 1]).to(torch.bfloat16).float()
        acc = acc + term
    assert torch.equal(out, acc.to(torch.bfloat16))


def test_empty_inputs_every_entry_point():
    """Zero rows through every entry point besides the int4 GEMM (covered with the GEMM
    tests): each returns an empty result of the right shape without launching anything
    that could read past its inputs."""
    from tests.test_fp8_gpu import _fp8_weights
    k, n, e, g, inter = 256, 128, 4, 128, 128
    _, _, wt, st = _fp8_weights(n, k, seed=3)
    x0 = torch.empty((0, k), dtype=torch.bfloat16, device="cuda")
    assert ops.gemm_fp8_marlin_cuda(x0, wt, st, n, 128, 128).shape == (0, n)
    assert ops.gemm_fp8_w8a8_cuda(x0, wt, st, n, 128, 128).shape == (0, n)
    codes, scale = ops.quantize_rows_e4m3_cuda(x0)
    assert codes.shape == (0, k) and scale.shape == (0,)
    w, s, _ = _experts(e, n, k, g, seed=4)
    offsets = torch.zeros(e, dtype=torch.int32, device="cuda")
    assert ops.grouped_gemm_int4_cuda(x0, w, s, offsets, n, g).shape == (0, n)
    gu_w, gu_s, _ = _experts(e, 2 * inter, k, g, seed=5)
    dn_w, dn_s, _ = _experts(e, k, inter, g, seed=6)
    out, _ = ops.routed_experts_int4_cuda(x0, torch.empty((0, 2), dtype=torch.int32, device="cuda"),
                                          torch.empty((0, 2), dtype=torch.float32, device="cuda"),
                                          (gu_w, gu_s), (dn_w, dn_s), inter, g)
    assert out.shape == (0, k)
    weights, chosen = ops.route_top_k_cuda(torch.empty((0, e), device="cuda"), 2)
    assert weights.shape == (0, 2) and chosen.shape == (0, 2)
    assert ops.silu_mul_cuda(torch.empty((0, 2 * inter), dtype=torch.bfloat16, device="cuda")).shape == (0, inter)


@pytest.mark.parametrize("t,e,hidden,inter,top_k", [(256, 128, 2048, 768, 8), (4096, 128, 2048, 768, 8),
                                                   (1024, 8, 256, 128, 2), (40, 8, 256, 128, 2)])
def test_persistent_grouped_launches_match(tuning_env, t, e, hidden, inter, top_k):
    """PLM_MOE_PERSIST=1 (a measurement option) runs the grouped GEMMs as persistent launches:
    each workgroup walks several items and loads the next one's first K step during the
    current one's epilogue. The arithmetic per item is unchanged, so the block (fused SwiGLU
    gate_up, down with the 16-byte epilogue) and a plain grouped GEMM on every small tile
    shape must give the same bits as the default launches."""
    g = 128
    h, experts, weights, gu, dn = _moe_case(t, e, hidden, inter, top_k, g, seed=t + 3)
    args = (to_dev(h, torch.bfloat16), to_dev(experts.astype(np.int32)), to_dev(weights), gu[:2], dn[:2], inter, g)
    counts = SMALL_COUNTS[32] + [130, 300]
    w, s, _ = _experts(len(counts), 200, 1536, g, seed=12)
    x = to_dev(O.bf16_round(np.random.default_rng(4).standard_normal((sum(counts), 1536)).astype(np.float32)),
               torch.bfloat16)
    off = to_dev(np.cumsum(counts).astype(np.int32))
    results = []
    for knob in (None, "1"):
        tuning_env("PLM_MOE_PERSIST", knob)
        out, _ = ops.routed_experts_int4_cuda(*args)
        results.append((out, ops.grouped_gemm_int4_cuda(x, w, s, off, 200, g)))
    assert torch.equal(results[0][0], results[1][0]), "persistent MoE block"
    assert torch.equal(results[0][1], results[1][1]), "persistent grouped GEMM"


@pytest.mark.parametrize("tile_rows", ["16", "32", "64"])
@pytest.mark.parametrize("sdt,xdt,g", [("fp32", "bf16", 128), ("bf16", "fp16", 128), ("fp16", "fp16", 256),
                                       ("fp16", "bf16", 64)])
def test_persistent_grouped_small_tiles_match(tuning_env, sdt, xdt, g, tile_rows):
    """The persistent grouped launches on each single-level tile shape (PLM_MOE_ROWS), with
    every scale dtype, fp16 and bf16 x and groups of 64 / 128 / 256 rows of K, against the
    default launches bit for bit."""
    counts = [70, 0, 3, 1, 0, 0, 20, 2, 33, 0, 0, 64, 5, 9]
    e, n, k = len(counts), 200, 1536
    w, s, _ = _experts(e, n, k, g, seed=31, scale_dtype=sdt, x_dtype=xdt)
    x = to_dev(O.round_to(np.random.default_rng(8).standard_normal((sum(counts), k)).astype(np.float32), xdt),
               TDT[xdt])
    off = to_dev(np.cumsum(counts).astype(np.int32))
    tuning_env("PLM_MOE_ROWS", tile_rows)
    out = []
    for knob in (None, "1"):
        tuning_env("PLM_MOE_PERSIST", knob)
        out.append(ops.grouped_gemm_int4_cuda(x, w, s, off, n, g))
    assert torch.equal(out[0], out[1]), f"persistent {tile_rows}-row tiles {sdt} {xdt} g={g}"
