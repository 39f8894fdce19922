"""CPU oracle for the quantized-linear hot path.

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker (or, in the bench, as the timed CPU baseline). The product path
(``pulsarlm_amd``) never imports it and has no CPU fallback.

(``oracle/dequant.c``, loaded by ``oracle/oracle_c.py``, restates the int4 dequant once
more in C with OpenMP for the host baseline; tests check it against this module bit for bit.)

It restates, in numpy, the arithmetic of the reference's Marlin dequant-GEMM
path in pulsarlm-core:

* int4 packing, 8 signed nibbles per int32 along K, least significant first
  (``pulsarlm-core/tests/kernels/test_marlin.cpp:42-46``,
  ``pulsarlm-core/inc/pulsarlm/kernels/ops.hpp:306-311``);
* dequantization ``W = round(q * round(scale))`` in the activation dtype, i.e.
  ``weight.to(dtype) * expanded_scale.to(dtype)`` (``test_marlin.cpp:48-50``),
  which is what the kernel's ``scale_pair`` + ``__hmul2`` compute
  (``pulsarlm-core/src/kernels/marlin.cu:78-84,123-151,180-194``);
* e4m3 decode (``marlin.cu:176-194``) and the fp8 128x128 block quantizer of
  ``pulsarlm-core/tests/model/test_qwen3_5.cpp:301-311``;
* the Marlin word layout produced by ``repack_weight_kernel``
  (``marlin.cu:86-117,154-171,197-236,391-393``);
* dequantize-then-matmul with fp32 (here float64) accumulation
  (``test_marlin.cpp:90-93,108-111``), output cast once to the activation dtype;
* the non-repacked int4 GEMM's dequant ``round(q * fp32 scale)``
  (``pulsarlm-core/src/kernels/int4_gemm.cu:136-138``);
* the MoE ``routed_experts`` algorithm (``pulsarlm-core/src/engine/model/
  paged_forward.cpp:108-130``) and the per-expert dense restatement of
  ``pulsarlm-core/tests/model/test_qwen3_5_moe.cpp:229-248``;
* the router ``route_top_k`` and the activation ``silu_mul``
  (``pulsarlm-core/src/kernels/moe_routing.cu:56-131``).

How each function is pinned (checks live in ``tests/test_oracle.py``):

* ``bf16_round`` / ``fp16_round``: against torch's bf16/fp16 conversion on a
  sweep including ties, subnormals and infinities.
* ``e4m3_decode`` / ``e4m3_encode``: all 256 codes against torch's
  ``float8_e4m3fn`` conversion; encode against torch on a dense sweep.
* ``pack_int4`` / ``unpack_int4``: hand-computed known answers.
* ``dequant``: every nibble x a scale sweep against the reference test's own
  expression evaluated by ATen on the CPU (``q.to(dtype) * s.to(dtype)``).
* ``marlin_encode_*``: known answers derived by hand from the lane/offset
  description at ``marlin.cu:21-30,86-88,154-155``, and decode(encode(W)) == W.
* ``gemm_ref``: against torch fp32 matmul, and the identity-GEMM closed form.
* ``routed_experts_ref``: each rounding point (gate_up output, act(g)*u, down
  output, weighted term) against the reference's own steps
  (``paged_forward.cpp:116-129``: stable argsort, index_add_ counts, cumsum,
  ``at::_grouped_mm`` twice, silu, ``down * w.to(dtype)``, ``index_add_``) evaluated
  by torch on the CPU in bf16; order and offsets exactly; the summed output within
  the MoE tolerance; and against the per-expert dense restatement.
* ``fp8_block_quantize``: invariants (one code per block at |448|, exact
  reconstruction bound) and against torch's e4m3 cast.
* ``route_top_k_ref``: torch's softmax and topk (the reference test's own checks,
  ``pulsarlm-core/tests/kernels/test_fused_ops.cpp:83-100``) and hand-derived
  tie-breaking cases.
* ``silu_mul_ref``: torch's silu on a sweep, and the closed forms at 0 and large |g|.
* ``quantize_per_token_e4m3`` (W8A8 mode): codes and scales bit for bit against
  the reference's quantizer expression (``test_qwen3_5.cpp:301-311``: fp32
  ``amax.clamp_min(1e-12) / 448``, fp32 divide, torch ``float8_e4m3fn`` cast) applied
  per row by torch, on rows with zeros, ties, tiny and huge amax.
* ``gemm_w8a8_ref``: against a torch float64 matmul of the ``float8_e4m3fn``
  casts times their scales.
"""

from __future__ import annotations

import numpy as np

# ---------------------------------------------------------------------------
# Scalar formats
# ---------------------------------------------------------------------------


def bf16_round(x) -> np.ndarray:
    """Round float32 values to bf16 with round-to-nearest-even; float32 result."""
    f = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    bits = f.view(np.uint32).astype(np.uint64)
    nan = np.isnan(f)
    rounded = ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16) << 16
    out = (rounded & 0xFFFFFFFF).astype(np.uint32).view(np.float32).copy()
    out[nan] = np.float32(np.nan)
    return out


def bf16_bits(x) -> np.ndarray:
    return (bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)


def bf16_from_bits(bits) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint32) << 16).astype(np.uint32).view(np.float32)


def fp16_round(x) -> np.ndarray:
    """Round float32 values to fp16 (numpy's cast is round-to-nearest-even)."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def round_to(x, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return bf16_round(x)
    if dtype == "fp16":
        return fp16_round(x)
    raise ValueError(dtype)


def e4m3_decode(codes) -> np.ndarray:
    """OCP e4m3 (fn) byte -> float32. 0x7f/0xff are NaN; no infinities.

    Normal: (1 + m/8) * 2^(e-7); subnormal (e == 0): m * 2^-9.
    """
    c = np.asarray(codes, dtype=np.uint8).astype(np.int64)
    sign = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 7
    mag = np.where(e == 0, m * 2.0**-9, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    out = (sign * mag).astype(np.float32)
    out[(c & 0x7F) == 0x7F] = np.nan
    return out


_E4M3_POS = e4m3_decode(np.arange(0x7F, dtype=np.uint8)).astype(np.float64)  # codes 0..126


def e4m3_encode(x) -> np.ndarray:
    """float32 -> e4m3 byte, round-to-nearest-even, non-saturating.

    Magnitudes past the midpoint between 448 (0x7e) and the next grid value 480
    become the NaN code, as torch's ``float8_e4m3fn`` cast does.
    """
    v = np.asarray(x, dtype=np.float32).astype(np.float64)
    sign = np.signbit(v)
    a = np.abs(v)
    grid = np.concatenate([_E4M3_POS, [480.0]])  # index 127 stands for "overflow"
    hi = np.searchsorted(grid, a, side="left")
    hi = np.clip(hi, 0, 127)
    lo = np.clip(hi - 1, 0, 127)
    d_lo = np.abs(a - grid[lo])
    d_hi = np.abs(grid[hi] - a)
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & (hi % 2 == 0))
    code = np.where(pick_hi, hi, lo)
    code = np.where(a == grid[hi], hi, code)
    code = np.where(np.isnan(v), 0x7F, code).astype(np.uint8)
    code = np.where(code >= 0x7F, 0x7F, code).astype(np.uint8)
    return (code | np.where(sign, 0x80, 0).astype(np.uint8)).astype(np.uint8)


# ---------------------------------------------------------------------------
# int4 packing (test_marlin.cpp:42-46; ops.hpp:306-311)
# ---------------------------------------------------------------------------


def pack_int4(q) -> np.ndarray:
    """int values in [-8, 7], shape [N, K] (K % 8 == 0) -> int32 [N, K/8]."""
    q = np.asarray(q, dtype=np.int64)
    n, k = q.shape
    assert k % 8 == 0
    nib = (q & 0xF).reshape(n, k // 8, 8).astype(np.uint64)
    shifts = (np.arange(8, dtype=np.uint64) * 4)
    words = (nib << shifts).sum(axis=-1).astype(np.uint64)
    return (words & 0xFFFFFFFF).astype(np.uint32).view(np.int32)


def unpack_int4(packed) -> np.ndarray:
    """int32 [N, K/8] -> int8 [N, K], sign-extended nibbles, least significant first."""
    p = np.asarray(packed, dtype=np.int32).view(np.uint32).astype(np.int64)
    n, kw = p.shape
    nib = (p[:, :, None] >> (np.arange(8) * 4)) & 0xF
    q = nib - ((nib >> 3) << 4)
    return q.reshape(n, kw * 8).astype(np.int8)


def expand_scale(scale, n: int, k: int, block_n: int, group_size: int) -> np.ndarray:
    """[ceil(N/bn), K/g] -> [N, K] (test_marlin.cpp:27-29)."""
    s = np.asarray(scale, dtype=np.float32)
    return np.repeat(np.repeat(s, block_n, axis=0)[:n], group_size, axis=1)[:, :k]


def dequant_int4(packed, scale, block_n: int, group_size: int, dtype: str = "bf16") -> np.ndarray:
    """Reference Marlin dequant: round(q * round(float(scale))) in ``dtype``; float32 result."""
    q = unpack_int4(packed).astype(np.float32)
    n, k = q.shape
    s = round_to(expand_scale(scale, n, k, block_n, group_size), dtype)
    return round_to(q * s, dtype)


def dequant_fp8(codes, scale, block_n: int, group_size: int, dtype: str = "bf16") -> np.ndarray:
    """Reference fp8 Marlin dequant: round(e4m3(code) * round(scale)) in ``dtype``."""
    w = e4m3_decode(codes)
    n, k = w.shape
    s = round_to(expand_scale(scale, n, k, block_n, group_size), dtype)
    return round_to(w * s, dtype)


def dequant_int4_plain(packed, scale, group_size: int, dtype: str = "bf16") -> np.ndarray:
    """Non-repacked int4 GEMM's dequant: round(q * fp32 scale) (int4_gemm.cu:136-138)."""
    q = unpack_int4(packed).astype(np.float32)
    n, k = q.shape
    s = expand_scale(scale, n, k, 1, group_size)
    return round_to(q * s, dtype)


# ---------------------------------------------------------------------------
# GEMM
# ---------------------------------------------------------------------------


def gemm_ref(x, w_deq, dtype: str | None = "bf16") -> np.ndarray:
    """y = x @ W^T accumulated in float64 (>= the reference's fp32), cast once to ``dtype``."""
    y = np.asarray(x, dtype=np.float64) @ np.asarray(w_deq, dtype=np.float64).T
    y = y.astype(np.float32)
    return y if dtype is None else round_to(y, dtype)


def check_close(y, ref, atol=2e-2, rtol=2e-2, rel_l2=5e-3):
    """The GEMM tolerance used throughout: elementwise |y-ref| <= atol + rtol*|ref|
    (the reference test's ``allclose(2e-2, 2e-2)``, test_marlin.cpp:95,113) and
    ||y-ref||_2 / ||ref||_2 <= rel_l2. Returns (ok, stats)."""
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    err = np.abs(y - ref)
    denom = np.linalg.norm(ref)
    l2 = float(np.linalg.norm(y - ref) / denom) if denom > 0 else float(np.linalg.norm(y - ref))
    elem_ok = bool(np.all(err <= atol + rtol * np.abs(ref))) if err.size else True
    stats = {
        "max_abs": float(err.max()) if err.size else 0.0,
        "rel_l2": l2,
        "max_ref": float(np.abs(ref).max()) if ref.size else 0.0,
    }
    return elem_ok and l2 <= rel_l2 and np.all(np.isfinite(y)), stats


# ---------------------------------------------------------------------------
# The reference's Marlin word layout (marlin.cu:21-30,86-117,154-171,197-236)
# ---------------------------------------------------------------------------

MARLIN_TILE_N = 64
MARLIN_SPAN_K = 32


def marlin_words(n: int, k: int, words_per_lane: int) -> int:
    """marlin.cu:391-393."""
    return -(-n // MARLIN_TILE_N) * MARLIN_TILE_N // 8 * (-(-k // MARLIN_SPAN_K)) * words_per_lane * 32


def _marlin_index(n: int, k: int, wpl: int):
    total = marlin_words(n, k, wpl)
    idx = np.arange(total, dtype=np.int64)
    lane = idx % 32
    rest = idx // 32
    word = rest % wpl
    rest //= wpl
    subtile = rest % 8
    rest //= 8
    k_tiles = -(-k // MARLIN_SPAN_K)
    k_tile = rest % k_tiles
    block = rest // k_tiles
    row = (block * 8 + subtile) * 8 + lane // 4
    return idx, lane, word, k_tile, row


_INT4_OFFSETS = np.array([0, 8, 16, 24, 1, 9, 17, 25], dtype=np.int64)


def marlin_encode_int4(packed) -> np.ndarray:
    """[N, K/8] int32 -> the reference's Marlin int32 words (marlin.cu:96-117,197-225)."""
    q = unpack_int4(packed).astype(np.int64)
    n, k = q.shape
    idx, lane, word, k_tile, row = _marlin_index(n, k, 1)
    pair = lane % 4
    cols = k_tile[:, None] * 32 + 2 * pair[:, None] + _INT4_OFFSETS[None, :]
    valid = (row[:, None] < n) & (cols < k)
    vals = np.where(valid, q[np.minimum(row, n - 1)[:, None], np.minimum(cols, k - 1)], 0)
    nib = np.where(valid, (vals & 0xF) ^ 8, 8).astype(np.uint64)
    words = (nib << (np.arange(8, dtype=np.uint64) * 4)).sum(axis=1)
    return (words & 0xFFFFFFFF).astype(np.uint32).view(np.int32)


def marlin_decode_int4(words, n: int, k: int) -> np.ndarray:
    """Inverse of marlin_encode_int4: Marlin words -> int8 q [N, K]."""
    w = np.asarray(words, dtype=np.int32).view(np.uint32).astype(np.int64)
    idx, lane, word, k_tile, row = _marlin_index(n, k, 1)
    pair = lane % 4
    cols = k_tile[:, None] * 32 + 2 * pair[:, None] + _INT4_OFFSETS[None, :]
    nib = (w[:, None] >> (np.arange(8) * 4)) & 0xF
    vals = nib - 8  # nibbles hold (q & 0xF) ^ 8 == q + 8
    q = np.zeros((n, k), dtype=np.int8)
    valid = (row[:, None] < n) & (cols < k)
    rr = np.broadcast_to(row[:, None], cols.shape)
    q[rr[valid], cols[valid]] = vals[valid]
    return q


_FP8_OFFSETS = np.array([0, 1, 8, 9], dtype=np.int64)


def marlin_encode_fp8(codes) -> np.ndarray:
    """[N, K] e4m3 bytes -> the reference's Marlin words (marlin.cu:154-171,197-225)."""
    c = np.asarray(codes, dtype=np.uint8)
    n, k = c.shape
    idx, lane, word, k_tile, row = _marlin_index(n, k, 2)
    pair = lane % 4
    cols = k_tile[:, None] * 32 + 16 * word[:, None] + 2 * pair[:, None] + _FP8_OFFSETS[None, :]
    valid = (row[:, None] < n) & (cols < k)
    b = np.where(valid, c[np.minimum(row, n - 1)[:, None], np.minimum(cols, k - 1)], 0).astype(np.uint64)
    words = (b << (np.arange(4, dtype=np.uint64) * 8)).sum(axis=1)
    return (words & 0xFFFFFFFF).astype(np.uint32).view(np.int32)


def marlin_decode_fp8(words, n: int, k: int) -> np.ndarray:
    w = np.asarray(words, dtype=np.int32).view(np.uint32).astype(np.int64)
    idx, lane, word, k_tile, row = _marlin_index(n, k, 2)
    pair = lane % 4
    cols = k_tile[:, None] * 32 + 16 * word[:, None] + 2 * pair[:, None] + _FP8_OFFSETS[None, :]
    b = (w[:, None] >> (np.arange(4) * 8)) & 0xFF
    out = np.zeros((n, k), dtype=np.uint8)
    valid = (row[:, None] < n) & (cols < k)
    rr = np.broadcast_to(row[:, None], cols.shape)
    out[rr[valid], cols[valid]] = b[valid]
    return out


def marlin_scale(scale) -> np.ndarray:
    """transpose_scale_kernel (marlin.cu:227-236): [rows, groups] -> fp32 [groups, rows]."""
    return np.ascontiguousarray(np.asarray(scale, dtype=np.float32).T)


# ---------------------------------------------------------------------------
# fp8 quantizers
# ---------------------------------------------------------------------------


def fp8_block_quantize(w, block_n: int = 128, block_k: int = 128):
    """test_qwen3_5.cpp:301-311: scale = max(amax(block), 1e-12) / 448 per
    [block_n x block_k] block; codes = e4m3(w / expanded scale)."""
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    rows = -(-n // block_n)
    padded = np.zeros((rows * block_n, k), dtype=np.float32)
    padded[:n] = w
    amax = np.abs(padded).reshape(rows, block_n, k // block_k, block_k).max(axis=(1, 3))
    scale = (np.maximum(amax, np.float32(1e-12)) / np.float32(448.0)).astype(np.float32)
    expanded = expand_scale(scale, n, k, block_n, block_k)
    codes = e4m3_encode((w / expanded).astype(np.float32))
    return codes, scale


def quantize_per_token_e4m3(x):
    """W8A8 activation quantizer: the block quantizer of test_qwen3_5.cpp:301-311
    applied per row (one 1 x K block per token): scale = max(amax, 1e-12) / 448 in
    fp32, codes = e4m3_rne(x / scale) with an fp32 divide."""
    x = np.asarray(x, dtype=np.float32)
    amax = np.abs(x).max(axis=1) if x.size else np.zeros((x.shape[0],), np.float32)
    scale = (np.maximum(amax, np.float32(1e-12)) / np.float32(448.0)).astype(np.float32)
    codes = e4m3_encode((x / scale[:, None]).astype(np.float32))
    return codes, scale


def gemm_w8a8_ref(codes_x, scale_x, codes_w, scale_w, block_n: int, group_size: int, dtype="bf16"):
    """y = diag(sx) * e4m3(cx) @ (e4m3(cw) * s_w)^T, exact products, float64 sums,
    rounded once to ``dtype``."""
    xq = e4m3_decode(codes_x).astype(np.float64) * np.asarray(scale_x, np.float64)[:, None]
    n, k = np.asarray(codes_w).shape
    wq = e4m3_decode(codes_w).astype(np.float64) * expand_scale(scale_w, n, k, block_n, group_size)
    return gemm_ref(xq, wq, dtype)


# ---------------------------------------------------------------------------
# MoE (paged_forward.cpp:108-130; test_qwen3_5_moe.cpp:229-248)
# ---------------------------------------------------------------------------


def silu(v):
    v = np.asarray(v, dtype=np.float64)
    return v / (1.0 + np.exp(-v))


def moe_sort(top_experts, n_experts: int):
    """Stable sort of the flattened (token, k) assignments by expert, per-expert
    counts and inclusive-end int32 offsets (paged_forward.cpp:116-122)."""
    te = np.asarray(top_experts, dtype=np.int64)
    top_k = te.shape[-1]
    flat = te.reshape(-1)
    order = np.argsort(flat, kind="stable")
    tokens = order // top_k
    counts = np.bincount(flat, minlength=n_experts).astype(np.int32)
    offsets = np.cumsum(counts).astype(np.int32)
    return order, tokens, counts, offsets


def routed_experts_ref(h, top_experts, top_weights, gate_up, down, dtype="bf16", parts=False):
    """Restatement of routed_experts with dense per-expert weights (already
    dequantized): gate_up [E, 2I, H], down [E, H, I], with the reference's
    rounding points in the activation dtype: each grouped GEMM's output
    (accumulated here in float64), at::silu(g), its product with u, and each
    weighted term down * top_weight.to(dtype) (paged_forward.cpp:124-128). The
    reference's index_add_ accumulates those terms in the activation dtype in a
    scheduling-dependent order; here they are summed in float64 and rounded once.

    With ``parts=True`` it also returns the per-row stages in sorted order
    (gate_up output, act(g)*u, down output, weighted term), one per rounding point,
    so each can be compared with the reference's own steps."""
    h = np.asarray(h, dtype=np.float32)
    e_count = gate_up.shape[0]
    inter = gate_up.shape[1] // 2
    order, tokens, counts, offsets = moe_sort(top_experts, e_count)
    wflat = np.asarray(top_weights, dtype=np.float32).reshape(-1)[order]
    rows = h[tokens]
    n_rows = rows.shape[0]
    stages = {"gate_up": np.zeros((n_rows, 2 * inter), np.float32), "act": np.zeros((n_rows, inter), np.float32),
              "down": np.zeros((n_rows, h.shape[1]), np.float32), "weighted": np.zeros((n_rows, h.shape[1]), np.float32)}
    out = np.zeros(h.shape, dtype=np.float64)
    start = 0
    for e in range(e_count):
        end = int(offsets[e])
        if end > start:
            r = rows[start:end]
            gu = gemm_ref(r, gate_up[e], dtype)
            act = round_to(round_to(silu(gu[:, :inter]), dtype) * gu[:, inter:], dtype)
            d = gemm_ref(act, down[e], dtype)
            term = round_to(d * round_to(wflat[start:end], dtype)[:, None], dtype)
            np.add.at(out, tokens[start:end], term.astype(np.float64))
            for name, v in (("gate_up", gu), ("act", act), ("down", d), ("weighted", term)):
                stages[name][start:end] = v
        start = end
    result = round_to(out.astype(np.float32), dtype)
    if parts:
        return result, dict(stages, order=order, offsets=offsets)
    return result


def sparse_moe_ref(h, top_experts, top_weights, gate_up, down, dtype="bf16"):
    """Per-expert dense restatement (test_qwen3_5_moe.cpp:229-248): each expert
    over the tokens that chose it, with the same rounding points as
    routed_experts_ref. Used to pin routed_experts_ref's sort/offset logic."""
    h = np.asarray(h, dtype=np.float32)
    te = np.asarray(top_experts)
    tw = np.asarray(top_weights, dtype=np.float32)
    inter = gate_up.shape[1] // 2
    out = np.zeros(h.shape, dtype=np.float64)
    for e in range(gate_up.shape[0]):
        chosen = te == e
        toks = np.nonzero(chosen.any(-1))[0]
        if toks.size == 0:
            continue
        weight = (tw * chosen).sum(-1)[toks]
        gu = gemm_ref(h[toks], gate_up[e], dtype)
        act = round_to(round_to(silu(gu[:, :inter]), dtype) * gu[:, inter:], dtype)
        d = gemm_ref(act, down[e], dtype)
        out[toks] += round_to(d * round_to(weight, dtype)[:, None], dtype).astype(np.float64)
    return round_to(out.astype(np.float32), dtype)


# ---------------------------------------------------------------------------
# Seeded synthetic inputs (benchmark configs)
# ---------------------------------------------------------------------------


def make_w4a16(m: int, n: int, k: int, group_size: int = 128, seed: int = 0, block_n: int = 1):
    """x bf16-representable N(0,1) [M,K]; q uniform [-8,7]; fp16 scales |N(0,0.02)|+1e-3."""
    rng = np.random.default_rng(seed)
    x = bf16_round(rng.standard_normal((m, k), dtype=np.float32))
    q = rng.integers(-8, 8, size=(n, k), dtype=np.int64)
    rows = -(-n // block_n)
    scale = (np.abs(rng.standard_normal((rows, k // group_size)).astype(np.float32) * 0.02) + 1e-3)
    scale = scale.astype(np.float16)
    return x, pack_int4(q), scale


def make_fp8(m: int, n: int, k: int, seed: int = 0, block: int = 128):
    """Weights = block quantizer applied to bf16 N(0, 0.02)."""
    rng = np.random.default_rng(seed)
    x = bf16_round(rng.standard_normal((m, k), dtype=np.float32))
    w = bf16_round(rng.standard_normal((n, k), dtype=np.float32) * 0.02)
    codes, scale = fp8_block_quantize(w, block, block)
    return x, codes, scale


def zipf_routing(tokens: int, n_experts: int, top_k: int, alpha: float = 1.2, seed: int = 0):
    """top_k distinct experts per token drawn from Zipf(alpha) over expert ids
    (without replacement); weights = renormalised softmax of seeded logits."""
    rng = np.random.default_rng(seed)
    p = 1.0 / np.arange(1, n_experts + 1) ** alpha
    p /= p.sum()
    experts = np.empty((tokens, top_k), dtype=np.int64)
    for t in range(tokens):
        experts[t] = rng.choice(n_experts, size=top_k, replace=False, p=p)
    logits = rng.standard_normal((tokens, top_k)).astype(np.float32)
    w = np.exp(logits - logits.max(-1, keepdims=True))
    w = (w / w.sum(-1, keepdims=True)).astype(np.float32)
    return experts, w


# ---------------------------------------------------------------------------
# The plm tile layout (this build's format; restated from its specification in
# include/pulsarlm_amd.h so the GPU repack can be compared bit for bit)
# ---------------------------------------------------------------------------


def _plm_coords(n: int, k: int):
    """For every (row, col) of an N x K fp8 matrix: strip, k tile, step t, lane, i."""
    rows = np.arange(n)[:, None]
    cols = np.arange(k)[None, :]
    strip = rows // 16
    kt = cols // 128
    t = (cols % 128) // 32
    lane = rows % 16 + 16 * ((cols % 32) // 8)
    i = cols % 8
    return strip, kt, t, lane, i


def _plm_int4_coords(n: int, k: int):
    """For every (row, col) of an N x K int4 matrix: word index and nibble position.
    Word ((strip*KT + kt)*64 + lane)*4 + t with lane = 16 g + 4 c + i holds column
    strip*16 + 4c + r at K = kt*128 + 32t + 8g + 4h + i in nibble 4 (r % 2) + 2h + r // 2."""
    rows = np.arange(n)[:, None]
    cols = np.arange(k)[None, :]
    strip, kt, t = rows // 16, cols // 128, (cols % 128) // 32
    kk = cols % 32
    g, h, i = kk // 8, (kk % 8) // 4, kk % 4
    c, r = (rows % 16) // 4, rows % 4
    lane = 16 * g + 4 * c + i
    pos = 4 * (r % 2) + 2 * h + r // 2
    ktiles = -(-k // 128)
    widx = ((strip * ktiles + kt) * 64 + lane) * 4 + t
    return np.broadcast_to(widx, (n, k)), np.broadcast_to(pos, (n, k))


def plm_layout_int4(packed) -> np.ndarray:
    """int32 [N, K/8] -> plm int4 layout as uint32 words (padding nibbles = 8, i.e. q = 0)."""
    q = unpack_int4(packed).astype(np.int64)
    n, k = q.shape
    strips, ktiles = -(-n // 16), -(-k // 128)
    # Start from all-padding words, then set each real nibble.
    nib_all = np.full((strips * ktiles * 256, 8), 8, dtype=np.uint64)
    widx, pos = _plm_int4_coords(n, k)
    nib_all[widx.reshape(-1), pos.reshape(-1)] = ((q & 0xF) ^ 8).reshape(-1).astype(np.uint64)
    words = (nib_all << (np.arange(8, dtype=np.uint64) * 4)).sum(axis=1)
    return (words & 0xFFFFFFFF).astype(np.uint32)


def plm_layout_fp8(codes) -> np.ndarray:
    """uint8 [N, K] -> plm fp8 layout bytes (padding 0)."""
    c = np.asarray(codes, dtype=np.uint8)
    n, k = c.shape
    strips, ktiles = -(-n // 16), -(-k // 128)
    out = np.zeros(strips * ktiles * 2048, dtype=np.uint8)
    strip, kt, t, lane, i = _plm_coords(n, k)
    off = ((strip * ktiles + kt) * 2 + t // 2) * 1024 + lane * 16 + (t % 2) * 8 + i
    out[np.broadcast_to(off, c.shape).reshape(-1)] = c.reshape(-1)
    return out


def plm_layout_scale(scale, n: int, k: int, block_n: int, group_size: int) -> np.ndarray:
    """[ceil(N/bn), K/g] -> [strips, groups, cols] in the same dtype (padding 0)."""
    s = np.asarray(scale)
    strips, ktiles = -(-n // 16), -(-k // 128)
    groups = -(-(ktiles * 128) // group_size)
    cols = 1 if block_n % 16 == 0 else 16
    out = np.zeros((strips, groups, cols), dtype=s.dtype)
    for c in range(cols):
        col = np.arange(strips) * 16 + c
        ok = col < n
        out[ok, : k // group_size, c] = s[col[ok] // block_n]
    return out


# ---------------------------------------------------------------------------
# MoE router and activation (pulsarlm-core/src/kernels/moe_routing.cu)
# ---------------------------------------------------------------------------


def route_top_k_ref(logits, k: int):
    """route_top_k (moe_routing.cu:56-110): the softmax of each row in fp32, its k most
    probable experts in descending order with the lower expert first among equal
    probabilities (int64 [T, k]), and their probabilities divided by their sum, taken
    in that order (fp32 [T, k]). Returns (weights, experts, probabilities)."""
    x = np.asarray(logits, dtype=np.float32)
    shifted = np.exp(x - x.max(axis=1, keepdims=True)).astype(np.float32)
    p = (shifted / shifted.sum(axis=1, keepdims=True, dtype=np.float32)).astype(np.float32)
    idx = np.broadcast_to(np.arange(x.shape[1]), p.shape)
    order = np.lexsort((idx, -p), axis=-1)
    experts = order[:, :k].astype(np.int64)
    top = np.take_along_axis(p, experts, axis=1)
    total = np.cumsum(top, axis=1, dtype=np.float32)[:, -1:]
    return (top / total).astype(np.float32), experts, p


def silu_mul_ref(x, dtype: str = "bf16") -> np.ndarray:
    """silu_mul (moe_routing.cu:112-131): round(round(silu(g)) * u) for x = [g | u] per
    row, silu(g) = g / (1 + exp(-g)) in fp32, round = to ``dtype`` ("fp32": none)."""
    x = np.asarray(x, dtype=np.float32)
    n = x.shape[1] // 2
    g, u = x[:, :n], x[:, n:]
    rnd = (lambda v: np.asarray(v, dtype=np.float32)) if dtype == "fp32" else (lambda v: round_to(v, dtype))
    act = rnd((g / (np.float32(1) + np.exp(-g))).astype(np.float32))
    return rnd((act * u).astype(np.float32))
