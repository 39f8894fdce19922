"""Pins for the CPU oracle (oracle/oracle.py): each restated function is checked
against an independent library routine, a closed form, hand-derived known
answers, or an invariant, so a dropped term / wrong index / wrong rounding
fails here. CPU only."""

import numpy as np
import pytest
import torch

from oracle import oracle as O


# ---------------------------------------------------------------- scalar formats


def _sweep_f32(rng, n=200_000):
    v = rng.standard_normal(n).astype(np.float32) * np.exp2(rng.integers(-30, 30, n)).astype(np.float32)
    # Exact ties for bf16: low 16 bits = 0x8000, both parities of bit 16.
    ties = (rng.integers(0, 2**31, 4000, dtype=np.uint32) & ~np.uint32(0xFFFF)) | np.uint32(0x8000)
    special = np.array([0.0, -0.0, np.inf, -np.inf, 1e-40, -1e-40, 3.4e38, 65504.0, 65520.0, 6e-8, 1.0, -1.0],
                       dtype=np.float32)
    return np.concatenate([v, ties.view(np.float32), special])


def test_bf16_round_matches_torch():
    v = _sweep_f32(np.random.default_rng(0))
    got = O.bf16_round(v)
    ref = torch.from_numpy(v).to(torch.bfloat16).float().numpy()
    nan = np.isnan(ref)  # NaN payloads may differ; NaN-ness may not
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_fp16_round_matches_torch():
    v = _sweep_f32(np.random.default_rng(1))
    got = O.fp16_round(v)
    ref = torch.from_numpy(v).to(torch.float16).float().numpy()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_e4m3_decode_all_codes_match_torch():
    codes = np.arange(256, dtype=np.uint8)
    got = O.e4m3_decode(codes)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert nan.sum() == 2 and nan[0x7F] and nan[0xFF]
    assert np.array_equal(got[~nan], ref[~nan])
    # Closed-form spot checks: max normal, min subnormal, one.
    assert got[0x7E] == 448.0 and got[0x01] == 2.0**-9 and got[0x38] == 1.0 and got[0xB8] == -1.0


def test_e4m3_encode_matches_torch():
    rng = np.random.default_rng(2)
    v = np.concatenate([
        rng.standard_normal(100_000).astype(np.float32) * 100,
        rng.standard_normal(20_000).astype(np.float32) * 1e-2,
        O.e4m3_decode(np.arange(0x7F, dtype=np.uint8)),  # exact grid points
        (O.e4m3_decode(np.arange(0x7E, dtype=np.uint8)) + O.e4m3_decode(np.arange(1, 0x7F, dtype=np.uint8))) / 2,
        np.array([448, 460, 464, 465, 479, 480, 500, -470, 2**-10, 3 * 2**-10], dtype=np.float32),
    ]).astype(np.float32)
    got = O.e4m3_encode(v)
    ref = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    # torch maps NaN codes with either sign bit; compare values where not NaN, NaN-ness where NaN.
    gn = (got & 0x7F) == 0x7F
    rn = (ref & 0x7F) == 0x7F
    assert np.array_equal(gn, rn)
    assert np.array_equal(got[~gn], ref[~rn])


# ---------------------------------------------------------------- int4 packing


def test_pack_int4_known_answer():
    q = np.array([[1, 2, 3, 4, 5, 6, 7, -8], [-1, 0, 0, 0, 0, 0, 0, 0]])
    words = O.pack_int4(q).view(np.uint32)
    assert words[0, 0] == 0x87654321
    assert words[1, 0] == 0x0000000F
    assert np.array_equal(O.unpack_int4(O.pack_int4(q)), q)


def test_unpack_every_nibble():
    for v in range(16):
        word = np.array([[v << 28]], dtype=np.uint32).view(np.int32)
        q = O.unpack_int4(word)
        assert q[0, 7] == (v if v < 8 else v - 16)
        assert np.all(q[0, :7] == 0)


# ---------------------------------------------------------------- dequant


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_dequant_int4_matches_reference_expression(dtype):
    """Every nibble x a scale sweep against test_marlin.cpp:48-50 evaluated by ATen:
    weight.to(dtype) * expanded_scale.to(dtype)."""
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
    rng = np.random.default_rng(3)
    n, k, g = 64, 16 * 16, 16
    q = np.tile(np.arange(-8, 8), (n, k // 16))
    scale = (rng.random((n, k // g)).astype(np.float32) * 0.1 + 0.01).astype(np.float32)
    scale[0, :] = np.float32(1.0 / 3.0)
    scale[1, :] = np.float32(2.0 ** -20)
    got = O.dequant_int4(O.pack_int4(q), scale, 1, g, dtype)
    expanded = torch.from_numpy(scale).repeat_interleave(g, 1)
    ref = (torch.from_numpy(q).to(tdt) * expanded.to(tdt)).float().numpy()
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
@pytest.mark.parametrize("block_n", [1, 128])
def test_dequant_fp8_matches_reference_expression(dtype, block_n):
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
    rng = np.random.default_rng(4)
    n, k, g = 200, 144, 16
    codes = rng.integers(0, 256, (n, k), dtype=np.uint8)
    codes[(codes == 0x7F) | (codes == 0xFF)] = 0
    scale = (rng.random((-(-n // block_n), k // g)).astype(np.float32) * 0.1 + 0.01)
    got = O.dequant_fp8(codes, scale, block_n, g, dtype)
    w = torch.from_numpy(codes).view(torch.float8_e4m3fn)
    exp = torch.from_numpy(scale).repeat_interleave(block_n, 0)[:n].repeat_interleave(g, 1)
    ref = (w.to(tdt) * exp.to(tdt)).float().numpy()
    assert np.array_equal(got, ref)


def test_dequant_plain_int4_rounds_once():
    """int4_gemm.cu:136-138 rounds q * fp32 scale once; differs from the Marlin rounding."""
    q = np.full((1, 8), 7)
    scale = np.array([[np.float32(0.1)]], dtype=np.float32)
    plain = O.dequant_int4_plain(O.pack_int4(q), np.repeat(scale, 1, axis=1), 8, "bf16")
    ref = torch.tensor(7.0 * np.float32(0.1), dtype=torch.float32).to(torch.bfloat16).float().item()
    assert plain[0, 0] == ref


# ---------------------------------------------------------------- Marlin layout


def test_marlin_int4_known_word():
    """marlin.cu:21-30,86-88: lane L holds column L/4 of its 8-column subtile; its
    nibbles are K offsets 2p+{0,8,16,24} then 2p+1+{0,8,16,24}, p = L%4, stored as q^8."""
    n, k = 64, 32
    q = np.zeros((n, k), dtype=np.int64)
    # Column-block 0, subtile 1 (rows 8..15), lane 6 -> row 8 + 1 = 9, pair 2.
    offs = [4, 12, 20, 28, 5, 13, 21, 29]
    vals = [1, 2, 3, -1, -2, -3, 7, -8]
    for o, v in zip(offs, vals):
        q[9, o] = v
    words = O.marlin_encode_int4(O.pack_int4(q)).view(np.uint32)
    w = int(words[(0 * 8 + 1) * 32 + 6])
    expect = 0
    for p, v in enumerate(vals):
        expect |= ((v & 0xF) ^ 8) << (4 * p)
    assert w == expect
    # A lane with all-zero weights reads 0x88888888.
    assert int(words[0]) == 0x88888888


def test_marlin_fp8_known_word():
    """marlin.cu:154-155: word w of lane L holds K offsets 16w + 2p + {0, 1, 8, 9}."""
    n, k = 64, 32
    c = np.zeros((n, k), dtype=np.uint8)
    # subtile 0, lane 13 -> row 3, pair 1; word 1 -> K 16 + 2 + {0,1,8,9} = 18, 19, 26, 27.
    for o, v in zip([18, 19, 26, 27], [0x11, 0x22, 0x33, 0x44]):
        c[3, o] = v
    words = O.marlin_encode_fp8(c).view(np.uint32)
    assert int(words[(0 * 2 + 1) * 32 + 13]) == 0x44332211


@pytest.mark.parametrize("n,k", [(200, 144), (64, 32), (7, 96), (130, 1024)])
def test_marlin_round_trip(n, k):
    rng = np.random.default_rng(n * k)
    q = rng.integers(-8, 8, (n, k))
    words = O.marlin_encode_int4(O.pack_int4(q))
    assert words.size == O.marlin_words(n, k, 1)
    assert np.array_equal(O.marlin_decode_int4(words, n, k), q)
    c = rng.integers(0, 256, (n, k), dtype=np.uint8)
    wf = O.marlin_encode_fp8(c)
    assert wf.size == O.marlin_words(n, k, 2)
    assert np.array_equal(O.marlin_decode_fp8(wf, n, k), c)


# ---------------------------------------------------------------- plm layout


def test_plm_layout_int4_known_word():
    """include/pulsarlm_amd.h: word ((strip*KT + kt)*64 + lane)*4 + t, lane = 16 g + 4 c + i,
    nibble 4 (r % 2) + 2 h + r // 2 holds q + 8 of column strip*16 + 4c + r at
    K = kt*128 + 32t + 8g + 4h + i. Derived by hand for one word."""
    n, k = 32, 256
    q = np.zeros((n, k), dtype=np.int64)
    # strip 1, columns 24..27 (c = 2, r = 0..3); kt 1, t 2, g 1 (K 128 + 64 + 8 ..), i = 3.
    vals = {(24, 0): 1, (25, 0): -1, (26, 0): 2, (27, 0): -2, (24, 1): 3, (25, 1): -3, (26, 1): 7, (27, 1): -8}
    for (col, h), v in vals.items():
        q[col, 128 + 64 + 8 + 4 * h + 3] = v
    words = O.plm_layout_int4(O.pack_int4(q))
    lane = 16 * 1 + 4 * 2 + 3
    w = int(words[((1 * 2 + 1) * 64 + lane) * 4 + 2])
    # nibble p: (r, h) = (0,0) (2,0) (0,1) (2,1) (1,0) (3,0) (1,1) (3,1)
    order = [(24, 0), (26, 0), (24, 1), (26, 1), (25, 0), (27, 0), (25, 1), (27, 1)]
    expect = sum((vals[c] + 8) << (4 * p) for p, c in enumerate(order))
    assert w == expect == 0x0567FBA9  # nibbles p0..p7 = 9, A, B, F, 7, 6, 5, 0
    assert int(words[0]) == 0x88888888
    assert np.count_nonzero(words != 0x88888888) == 1


def _mfma4x4x4(a, b, c):
    """v_mfma_f32_4x4x4_16b as measured on gfx950: 16 blocks b = lane // 4; A[i][k] of a
    block in lane 4b + i, register k; B[k][j] in lane 4b + j, register k; D[i][j] (+ C)
    in lane 4b + j, register i. a, b: [64, 4] values; c: [64, 4]."""
    a = a.reshape(16, 4, 4)          # block, i, k
    bt = b.reshape(16, 4, 4)         # block, j, k
    d = np.einsum("bik,bjk->bji", a.astype(np.float64), bt.astype(np.float64))  # block, j, i
    return d.reshape(64, 4) + c


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_plm_int4_matrix_core_dequant(dtype):
    """The kernels' dequant, emulated bit for bit on the CPU: nibbles -> 16-bit floats by
    and/or masks, two 4x4x4 products with the scale diagonal, converts. Each lane must end
    up with the exact reference weights round(q * round(s)) of column lane % 16 at
    K 8 (lane // 16) + 0..7 of the slice: the B operand of v_mfma_f32_16x16x32."""
    rng = np.random.default_rng(4)
    n, k = 16, 128
    q = rng.integers(-8, 8, size=(n, k))
    s = O.round_to((rng.random(n) * 0.1 + 1e-3).astype(np.float32), dtype)
    words = O.plm_layout_int4(O.pack_int4(q)).reshape(64, 4)  # [lane, t]
    ref = O.round_to(q * s[:, None], dtype)
    lane = np.arange(64)
    j = lane % 4
    sl = s[lane % 16]
    diag = np.zeros((64, 4))
    diag[lane, j] = sl

    def f16(bits):  # 16-bit pattern -> value
        return np.array(bits, np.uint16).view(np.float16).astype(np.float64)

    for t in range(4):
        w = words[:, t].astype(np.uint64)
        if dtype == "bf16":
            half = lambda v, sh: O.bf16_from_bits(((v >> sh) & 0xF) | 0x4300).astype(np.float64)  # noqa: E731
            a0 = np.stack([half(w, 0), half(w, 16), half(w, 4), half(w, 20)], 1)
            a1 = np.stack([half(w, 8), half(w, 24), half(w, 12), half(w, 28)], 1)
            c = np.repeat((-136.0 * sl)[:, None], 4, 1)
        else:
            lo = lambda v, sh: f16(((v >> sh) & 0xF) | 0x6400)  # noqa: E731  1024 + u
            hi = lambda v, sh: f16((((v >> sh) & 0xF) << 4) | 0x5400)  # noqa: E731  64 + u
            a0 = np.stack([lo(w, 0), lo(w, 16), hi(w, 4), hi(w, 20)], 1)
            a1 = np.stack([lo(w, 8), lo(w, 24), hi(w, 12), hi(w, 28)], 1)
            c = np.repeat((np.where(j < 2, -1032.0, -72.0) * sl)[:, None], 4, 1)
        d = np.concatenate([_mfma4x4x4(a0, diag, c), _mfma4x4x4(a1, diag, c)], 1)  # [lane, 8]
        got = O.round_to(d.astype(np.float32), dtype)
        for l in range(64):
            kk = 32 * t + 8 * (l // 16) + np.arange(8)
            assert np.array_equal(got[l], ref[l % 16, kk]), (t, l)


def test_plm_layout_fp8_known_byte():
    n, k = 16, 128
    c = np.zeros((n, k), dtype=np.uint8)
    c[5, 32 * 3 + 8 * 1 + 6] = 0xAB  # t = 3, kq = 1, i = 6 -> half 1, lane 5 + 16
    out = O.plm_layout_fp8(c)
    assert out[1 * 1024 + (5 + 16) * 16 + 8 + 6] == 0xAB
    assert out.sum() == 0xAB


def test_plm_scale_layout():
    s = np.arange(1, 1 + 4 * 3, dtype=np.float16).reshape(4, 3)  # block_n = 10 -> rows 0..3, K/g = 3
    out = O.plm_layout_scale(s, 35, 96, 10, 32)
    assert out.shape == (3, 4, 16)  # strips 3, groups ceil(128/32)=4, per-column
    assert out[2, 1, 2] == s[34 // 10, 1]
    assert out[2, 1, 3] == 0  # column 35 is padding
    assert np.all(out[:, 3, :] == 0)  # padded group
    out2 = O.plm_layout_scale(np.ones((2, 1), np.float32), 200, 128, 128, 128)
    assert out2.shape == (13, 1, 1)


# ---------------------------------------------------------------- GEMM


def test_gemm_ref_matches_torch_fp32():
    rng = np.random.default_rng(5)
    x, packed, scale = O.make_w4a16(16, 256, 512, 128, seed=5)
    w = O.dequant_int4(packed, scale, 1, 128)
    got = O.gemm_ref(x, w, None)
    ref = (torch.from_numpy(x) @ torch.from_numpy(w).T).numpy()
    assert np.allclose(got, ref, rtol=1e-5, atol=1e-4)
    del rng


def test_identity_gemm_is_the_dequantized_weight():
    _, packed, scale = O.make_w4a16(1, 48, 256, 64, seed=6)
    w = O.dequant_int4(packed, scale, 1, 64)
    y = O.gemm_ref(np.eye(256, dtype=np.float32), w, "bf16")
    assert np.array_equal(y, w.T)


def test_check_close_flags_a_wrong_sign():
    x, packed, scale = O.make_w4a16(4, 64, 256, 128, seed=7)
    w = O.dequant_int4(packed, scale, 1, 128)
    y = O.gemm_ref(x, w)
    ok, _ = O.check_close(y, O.gemm_ref(x, w, None))
    assert ok
    bad = y.copy()
    bad[0, 0] = -bad[0, 0] + (1.0 if bad[0, 0] == 0 else 0.0)
    assert not O.check_close(bad, O.gemm_ref(x, w, None))[0]


# ---------------------------------------------------------------- fp8 quantizer


def test_fp8_block_quantizer_invariants():
    rng = np.random.default_rng(8)
    w = O.bf16_round(rng.standard_normal((300, 256)).astype(np.float32) * 0.02)
    codes, scale = O.fp8_block_quantize(w, 128, 128)
    assert scale.shape == (3, 2)
    deq = O.e4m3_decode(codes) * O.expand_scale(scale, 300, 256, 128, 128)
    # Each block's largest magnitude maps to 448 exactly.
    blocks = np.abs(O.e4m3_decode(codes))
    for r in range(3):
        for c in range(2):
            assert blocks[r * 128:(r + 1) * 128, c * 128:(c + 1) * 128].max() == 448.0
    rel = np.abs(deq - w) / np.maximum(np.abs(w), 1e-30)
    assert np.all((rel <= 2.0**-4 + 1e-7) | (np.abs(w) < scale.max() * 2**-6))
    ref = torch.from_numpy(w / O.expand_scale(scale, 300, 256, 128, 128)).to(torch.float8_e4m3fn)
    assert np.array_equal(codes, ref.view(torch.uint8).numpy())


# ---------------------------------------------------------------- MoE


def test_routed_experts_matches_per_expert_dense():
    rng = np.random.default_rng(9)
    e, h_dim, inter, t, top_k = 8, 64, 32, 40, 2
    h = O.bf16_round(rng.standard_normal((t, h_dim)).astype(np.float32))
    gate_up = O.bf16_round(rng.standard_normal((e, 2 * inter, h_dim)).astype(np.float32) * 0.1)
    down = O.bf16_round(rng.standard_normal((e, h_dim, inter)).astype(np.float32) * 0.1)
    experts, weights = O.zipf_routing(t, e, top_k, seed=9)
    a = O.routed_experts_ref(h, experts, weights, gate_up, down)
    b = O.sparse_moe_ref(h, experts, weights, gate_up, down)
    assert np.allclose(a, b, rtol=1e-2, atol=1e-2)
    # The offsets are inclusive cumulative counts and the sort is stable.
    order, tokens, counts, offsets = O.moe_sort(experts, e)
    assert offsets[-1] == t * top_k and np.array_equal(np.diff(np.concatenate([[0], offsets])), counts)
    flat = experts.reshape(-1)[order]
    assert np.all(np.diff(flat) >= 0)
    for ex in range(e):
        idx = order[flat == ex]
        assert np.all(np.diff(idx) > 0)


def test_zipf_routing_is_skewed_and_distinct():
    experts, w = O.zipf_routing(256, 128, 8, seed=1)
    assert all(len(set(r)) == 8 for r in experts)
    counts = np.bincount(experts.reshape(-1), minlength=128)
    assert counts[0] > 5 * counts[64:].mean()
    assert np.allclose(w.sum(-1), 1.0, atol=1e-6)


# ---------------------------------------------------------------- router and activation


@pytest.mark.parametrize("experts,k", [(16, 10), (512, 10), (128, 8)])
def test_route_top_k_ref_matches_torch(experts, k):
    """The reference test's own checks (test_fused_ops.cpp:93-99) with torch on the CPU."""
    logits = torch.randn(37, experts, generator=torch.Generator().manual_seed(experts))
    w, e, _ = O.route_top_k_ref(logits.numpy(), k)
    probabilities = torch.softmax(logits, -1, dtype=torch.float32)
    top = torch.topk(probabilities, k, -1).values
    got = probabilities.gather(1, torch.from_numpy(e))
    assert torch.allclose(got, top, rtol=1e-6, atol=0.0)
    assert torch.allclose(torch.from_numpy(w), top / top.sum(-1, keepdim=True), rtol=1e-6, atol=1e-6)
    assert np.all(np.diff(np.take_along_axis(probabilities.numpy(), e, 1), axis=1) <= 0)  # descending


def test_route_top_k_ref_breaks_ties_by_lower_expert():
    logits = np.array([[1.0, 3.0, 3.0, 2.0, 3.0], [0.0, 0.0, 0.0, 0.0, 0.0]], dtype=np.float32)
    w, e, _ = O.route_top_k_ref(logits, 5)
    assert e.tolist() == [[1, 2, 4, 3, 0], [0, 1, 2, 3, 4]]
    assert np.allclose(w[1], 0.2) and abs(w[0].sum() - 1) < 1e-6
    _, e3, _ = O.route_top_k_ref(logits, 3)
    assert e3.tolist() == [[1, 2, 4], [0, 1, 2]]
    assert np.allclose(O.route_top_k_ref(logits, 3)[0][0], 1 / 3, atol=1e-7)  # three equal winners


@pytest.mark.parametrize("dtype", ["fp32", "bf16", "fp16"])
def test_silu_mul_ref_matches_torch(dtype):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((64, 2 * 96)) * 4).astype(np.float32)
    x = x if dtype == "fp32" else O.round_to(x, dtype)
    got = O.silu_mul_ref(x, dtype)
    t = torch.from_numpy(x).double()
    expected = (torch.nn.functional.silu(t[:, :96]) * t[:, 96:]).numpy()
    tol = 1e-5 if dtype == "fp32" else 1e-2  # test_fused_ops.cpp:20-22
    assert np.allclose(got, expected, rtol=tol, atol=tol)
    # Closed forms: silu(0) = 0; silu(g) = g for large g, 0 for very negative g.
    z = O.silu_mul_ref(np.array([[0.0, 60.0, -60.0, 1.0, 2.0, 3.0]], dtype=np.float32), dtype)
    assert z[0, 0] == 0
    assert z[0, 1] == 120.0  # silu(60) = 60 in fp32, times 2 (exact in every dtype)
    assert abs(z[0, 2]) < 1e-20


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_dequant_plain_int4_every_nibble(dtype):
    """Every nibble x a sweep of fp32 scales against torch: the product rounded to fp32,
    then to the dtype (int4_gemm.cu:136-138: pack2(q * scale))."""
    rng = np.random.default_rng(9)
    q = np.tile(np.arange(-8, 8), 64)[None, :].repeat(40, 0)  # [40, 1024]
    scale = (rng.random((40, 1024 // 16)) * 0.2 + 1e-4).astype(np.float32)
    got = O.dequant_int4_plain(O.pack_int4(q), scale, 16, dtype)
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
    exp = torch.from_numpy(scale).repeat_interleave(16, 1)
    ref = (torch.from_numpy(q).float() * exp).to(tdt).float().numpy()
    assert np.array_equal(got, ref)


# ---------------------------------------------------------------- W8A8 pins


def _torch_quantize_rows(x, recip=False, clamp=1e-12, div=448.0, rounding="rne"):
    """The block quantizer of test_qwen3_5.cpp:301-311 (fp32 amax, clamp_min(1e-12),
    / 448, fp32 divide, float8_e4m3fn cast) applied per row by torch on the CPU.
    The keyword arguments build plausible mistakes, which the pins must reject."""
    xt = torch.from_numpy(np.ascontiguousarray(x)).float()
    scale = xt.abs().amax(1, keepdim=True).clamp_min(clamp) / div
    q = xt * (1.0 / scale) if recip else xt / scale
    if rounding == "trunc":  # round toward zero onto the e4m3 grid
        c = q.to(torch.float8_e4m3fn)
        over = c.float().abs() > q.abs()
        c = torch.where(over, (c.view(torch.uint8) - 1).view(torch.float8_e4m3fn), c)
        return c.view(torch.uint8).numpy(), scale[:, 0].numpy()
    return q.to(torch.float8_e4m3fn).view(torch.uint8).numpy(), scale[:, 0].numpy()


def _quantizer_rows():
    rng = np.random.default_rng(11)
    k = 512
    rows = [O.bf16_round(rng.standard_normal((6, k)).astype(np.float32) * 3)]
    rows.append(np.zeros((1, k), np.float32))                                   # zero row: scale = 1e-12/448
    tiny = O.bf16_round(rng.standard_normal((1, k)).astype(np.float32) * 1e-13)  # amax below the clamp
    rows.append(tiny)
    huge = O.bf16_round(rng.standard_normal((1, k)).astype(np.float32) * 1e37)
    rows.append(huge)
    # amax = 448 * 2^-3 makes the scale exactly 2^-3, so x / scale is exact and the
    # e4m3 midpoints below are exact ties (RNE must pick the even code).
    mids = (O.e4m3_decode(np.arange(1, 0x7E, dtype=np.uint8)) + O.e4m3_decode(np.arange(2, 0x7F, dtype=np.uint8))) / 2
    ties = np.zeros((1, k), np.float32)
    ties[0, 0] = 56.0
    t = O.bf16_round((mids * 0.125).astype(np.float32))
    t = t[O.bf16_round(t) == mids * 0.125][: k - 1]
    ties[0, 1:1 + t.size] = t * np.where(np.arange(t.size) % 2, -1, 1)
    rows.append(ties)
    # Every non-negative bf16 value up to amax = 3.1875: some quotients x / scale
    # round differently from x * (1 / scale) (found by the same search on the CPU).
    bits = (np.arange(0, 0x4060, dtype=np.uint32) << 16).view(np.float32)
    allv = np.concatenate([[np.float32(3.1875)], bits[bits <= 3.1875]]).astype(np.float32)
    rows.append(allv[None, :])
    width = max(r.shape[1] for r in rows)
    return [np.pad(r, ((0, 0), (0, width - r.shape[1]))) for r in rows]


def test_quantize_per_token_matches_reference_quantizer():
    for x in _quantizer_rows():
        codes, scale = O.quantize_per_token_e4m3(x)
        ref_c, ref_s = _torch_quantize_rows(x)
        assert np.array_equal(scale.view(np.uint32), ref_s.view(np.uint32))
        assert np.array_equal(codes, ref_c)


@pytest.mark.parametrize("mutant", [dict(recip=True), dict(clamp=1e-6), dict(div=447.0), dict(rounding="trunc")])
def test_quantizer_pin_rejects_mutants(mutant):
    """Each plausible mistake (x * (1/scale), another clamp, another divisor, truncation)
    disagrees with the reference quantizer on these rows, so the pin above resolves it."""
    differs = False
    for x in _quantizer_rows():
        c, s = _torch_quantize_rows(x, **mutant)
        ref_c, ref_s = _torch_quantize_rows(x)
        differs |= not (np.array_equal(c, ref_c) and np.array_equal(s, ref_s))
    assert differs


@pytest.mark.parametrize("block_n,group", [(128, 128), (1, 128), (16, 256)])
def test_gemm_w8a8_ref_matches_torch_float64(block_n, group):
    rng = np.random.default_rng(12)
    m, n, k = 9, 200, 512
    x = O.bf16_round(rng.standard_normal((m, k)).astype(np.float32))
    cx, sx = O.quantize_per_token_e4m3(x)
    w = O.bf16_round(rng.standard_normal((n, k)).astype(np.float32) * 0.02)
    cw, sw = O.fp8_block_quantize(w, block_n, group) if block_n == group else (
        O.e4m3_encode(w * 64), (rng.random((-(-n // block_n), k // group)) * 0.02 + 1e-3).astype(np.float32))
    got = O.gemm_w8a8_ref(cx, sx, cw, sw, block_n, group, dtype=None)
    xt = torch.from_numpy(cx).view(torch.float8_e4m3fn).double() * torch.from_numpy(sx).double()[:, None]
    st = torch.from_numpy(np.asarray(sw, np.float32)).double().repeat_interleave(block_n, 0)[:n].repeat_interleave(group, 1)
    wt = torch.from_numpy(cw).view(torch.float8_e4m3fn).double() * st
    ref = (xt @ wt.T).float().numpy()
    assert np.allclose(got, ref, rtol=1e-6, atol=1e-6)
    # A transposed scale expansion or a dropped row scale would not match.
    assert not np.allclose(got, (xt @ wt.T / torch.from_numpy(sx).double()[:, None]).float().numpy(), rtol=1e-3)
    bf = O.gemm_w8a8_ref(cx, sx, cw, sw, block_n, group)
    assert np.array_equal(bf, O.bf16_round(got))


# ---------------------------------------------------------------- MoE pins


def _routed_experts_torch(h, top_experts, top_weights, gate_up, down, round_silu=True, round_weight=True):
    """routed_experts (paged_forward.cpp:116-129) step by step with torch on the CPU,
    at::_grouped_mm included, in the activation dtype. round_silu / round_weight = False
    drop one rounding point each (plausible mistakes the pins must reject)."""
    n_experts = gate_up.shape[0]
    top_k = top_experts.shape[-1]
    assigned = top_experts.flatten()
    order = torch.argsort(assigned, stable=True)
    tokens = torch.floor_divide(order, top_k)
    counts = torch.zeros(n_experts, dtype=torch.int32).index_add_(
        0, assigned.index_select(0, order), torch.ones_like(order, dtype=torch.int32))
    offsets = torch.cumsum(counts, 0, dtype=torch.int32)
    rows = h.index_select(0, tokens)
    gu = torch._grouped_mm(rows, gate_up.transpose(1, 2), offsets)
    g, u = gu.chunk(2, -1)
    if round_silu:
        act = torch.nn.functional.silu(g) * u
    else:
        act = (torch.nn.functional.silu(g.float()) * u.float()).to(h.dtype)
    d = torch._grouped_mm(act, down.transpose(1, 2), offsets)
    w = top_weights.flatten().index_select(0, order).unsqueeze(1)
    weighted = d * w.to(d.dtype) if round_weight else (d.float() * w).to(d.dtype)
    out = torch.zeros_like(h).index_add_(0, tokens, weighted)
    return out, dict(order=order, offsets=offsets, gate_up=gu, act=act, down=d, weighted=weighted)


def _moe_case(seed=13, e=16, h_dim=128, inter=64, t=96, top_k=4):
    rng = np.random.default_rng(seed)
    h = O.bf16_round(rng.standard_normal((t, h_dim)).astype(np.float32))
    gate_up = O.bf16_round(rng.standard_normal((e, 2 * inter, h_dim)).astype(np.float32) * 0.1)
    down = O.bf16_round(rng.standard_normal((e, h_dim, inter)).astype(np.float32) * 0.1)
    experts, weights = O.zipf_routing(t, e, top_k, seed=seed)
    experts[0, 0], experts[1, 0] = experts[1, 0], experts[0, 0]  # keep an unsorted start
    bf = torch.bfloat16
    tin = (torch.from_numpy(h).to(bf), torch.from_numpy(experts), torch.from_numpy(weights),
           torch.from_numpy(gate_up).to(bf), torch.from_numpy(down).to(bf))
    return (h, experts, weights, gate_up, down), tin


def _bits_equal_frac(a, b):
    a = O.bf16_bits(np.asarray(a, np.float32))
    b = O.bf16_bits(np.asarray(b, np.float32))
    return float(np.mean(a == b)), int(np.max(np.abs(a.astype(np.int64) - b.astype(np.int64))))


def test_routed_experts_stages_match_reference_steps():
    """Each rounding point of the oracle against the reference's steps run by torch:
    sort and offsets exactly; the grouped GEMM outputs, silu(g)*u and the weighted
    terms bit for bit except where float64 and fp32 accumulation round apart (at most
    one bf16 ulp, in a small fraction); the index_add_ sum within the MoE tolerance."""
    args, tin = _moe_case()
    out, parts = O.routed_experts_ref(*args, parts=True)
    ref_out, ref = _routed_experts_torch(*tin)
    assert np.array_equal(parts["order"], ref["order"].numpy())
    assert np.array_equal(parts["offsets"], ref["offsets"].numpy())
    for name in ("gate_up", "act", "down", "weighted"):
        frac, ulps = _bits_equal_frac(parts[name], ref[name].float().numpy())
        assert frac >= 0.99 and ulps <= 1, (name, frac, ulps)
    r = ref_out.float().numpy()
    rel = np.linalg.norm(out - r) / np.linalg.norm(r)
    assert rel <= 5e-3 and np.abs(out - r).max() / np.abs(r).max() < 5e-2


@pytest.mark.parametrize("mutant", [dict(round_silu=False), dict(round_weight=False)])
def test_routed_experts_pin_rejects_dropped_rounding(mutant):
    """With a rounding point dropped, the reference's steps no longer match the
    oracle's stages at the bit level the pin above demands."""
    args, tin = _moe_case()
    _, parts = O.routed_experts_ref(*args, parts=True)
    _, mut = _routed_experts_torch(*tin, **mutant)
    stage = "act" if "round_silu" in mutant else "weighted"
    frac, _ = _bits_equal_frac(parts[stage], mut[stage].float().numpy())
    assert frac < 0.99, frac
